"""deep_gemm for AMD MI355X (gfx950): the block-scaled FP8 / FP4 GEMM family of
DeepGEMM-Ascend behind the same Python API (the reference's deep_gemm/__init__.py:25-81).

Kernels are hand-written HIP for CDNA4 (scaled MFMA, LDS-staged operands) in
libdeep_gemm_amd.so, reached through its C ABI (include/deep_gemm_amd.h).  Importing this
package does not initialise the GPU; the library loads on the first kernel call.
"""
__version__ = '0.1.1'

import os


def get_library_root_path():
    return os.path.dirname(os.path.realpath(__file__))


from .runtime import (  # noqa: E402
    set_num_sms, get_num_sms,
    set_npu_arch, get_npu_arch,
    set_mk_alignment_for_contiguous_layout,
    get_mk_alignment_for_contiguous_layout,
    get_theoretical_mk_alignment_for_contiguous_layout,
    use_deterministic_algorithms, get_deterministic_algorithms,
    set_dry_run, get_dry_run, set_jit, get_jit, init,
)
from .layout import (transform_sf_into_required_layout, transform_k_grouped_sf_into_required_layout,  # noqa: E402
                     get_recipe)
from .gemm import (  # noqa: E402
    fp8_fp4_gemm_nt, fp8_fp4_gemm_nn, fp8_fp4_gemm_tn, fp8_fp4_gemm_tt,
    m_grouped_fp8_fp4_gemm_nt_contiguous, m_grouped_fp8_fp4_gemm_nn_contiguous,
    m_grouped_fp8_fp4_gemm_nt_masked,
    bf16_gemm_nt, bf16_gemm_nn, bf16_gemm_tn, bf16_gemm_tt,
    m_grouped_bf16_gemm_nt_contiguous, m_grouped_bf16_gemm_nn_contiguous,
    m_grouped_bf16_gemm_nt_masked,
    k_grouped_fp8_gemm_tn_contiguous, k_grouped_fp8_gemm_nt_contiguous, k_grouped_bf16_gemm_tn_contiguous,
    select_config,
    launch_plan,
)
from .einsum import fp8_bmm, bf16_bmm, einsum, fp8_einsum  # noqa: E402
from . import epilogue  # noqa: E402
from ._lib import check_errors  # noqa: E402

# FP8 aliases are the same objects as the FP8/FP4 entry points (csrc/apis/gemm.hpp:624-629)
fp8_gemm_nt = fp8_fp4_gemm_nt
fp8_gemm_nn = fp8_fp4_gemm_nn
fp8_gemm_tn = fp8_fp4_gemm_tn
fp8_gemm_tt = fp8_fp4_gemm_tt
m_grouped_fp8_gemm_nt_contiguous = m_grouped_fp8_fp4_gemm_nt_contiguous
m_grouped_fp8_gemm_nn_contiguous = m_grouped_fp8_fp4_gemm_nn_contiguous
m_grouped_fp8_gemm_nt_masked = m_grouped_fp8_fp4_gemm_nt_masked

init(__version__, get_library_root_path())
