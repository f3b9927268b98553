"""Host-side behaviour of the deep_gemm API that needs no GPU: validation order and
messages (the reference's csrc/apis/gemm.hpp and csrc/apis/layout.hpp), recipe
resolution, layout pass-through, and the lazy, fork-safe import."""
import subprocess
import sys

import pytest
import torch

import deep_gemm
from deep_gemm import layout as dl


def test_aliases_are_the_same_objects():
    assert deep_gemm.fp8_gemm_nt is deep_gemm.fp8_fp4_gemm_nt
    assert deep_gemm.fp8_gemm_tt is deep_gemm.fp8_fp4_gemm_tt
    assert deep_gemm.m_grouped_fp8_gemm_nt_contiguous is deep_gemm.m_grouped_fp8_fp4_gemm_nt_contiguous
    assert deep_gemm.m_grouped_fp8_gemm_nt_masked is deep_gemm.m_grouped_fp8_fp4_gemm_nt_masked


def test_default_arguments_match_reference():
    import inspect
    sig = inspect.signature(deep_gemm.fp8_fp4_gemm_nt)
    assert list(sig.parameters) == ['a', 'b', 'd', 'c', 'recipe', 'recipe_a', 'recipe_b', 'compiled_dims',
                                    'disable_ue8m0_cast', 'alpha', 'epilogue']
    assert sig.parameters['compiled_dims'].default == 'nk'
    assert inspect.signature(deep_gemm.fp8_fp4_gemm_tn).parameters['compiled_dims'].default == 'mn'
    sig = inspect.signature(deep_gemm.m_grouped_fp8_fp4_gemm_nt_contiguous)
    assert list(sig.parameters)[:4] == ['a', 'b', 'd', 'grouped_layout']
    assert sig.parameters['use_psum_layout'].default is True
    sig = inspect.signature(deep_gemm.transform_sf_into_required_layout)
    assert list(sig.parameters) == ['sf', 'mn', 'k', 'recipe', 'num_groups', 'is_sfa', 'disable_ue8m0_cast',
                                    'psum_layout']


def test_get_recipe_rules():
    assert dl.get_recipe() == (1, 1, 32)
    assert dl.get_recipe(recipe_a=(1, 128), recipe_b=(128, 128)) == (1, 128, 128)
    with pytest.raises(RuntimeError, match='gran_k of recipe_a and recipe_b must be the same'):
        dl.get_recipe(recipe_a=(1, 128), recipe_b=(1, 32))
    with pytest.raises(RuntimeError):
        dl.get_recipe(recipe=(1, 1, 32), recipe_a=(1, 32))
    # MX-compatible mixed granularity is accepted per operand
    assert dl.operand_recipes(recipe_a=(1, 128), recipe_b=(1, 32)) == ((1, 128), (1, 32))


def _fp8(shape):
    return torch.zeros(shape, dtype=torch.float8_e4m3fn)


def test_alpha_and_bias_rejected_before_any_device_work():
    a, b = _fp8((64, 128)), _fp8((32, 128))
    sfa, sfb = torch.ones(64, 4), torch.ones(32, 4)
    d = torch.empty(64, 32, dtype=torch.bfloat16)
    bias = torch.zeros(1, 32, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match='alpha and bias cannot be used together'):
        deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, c=bias, alpha=2.0)


def test_c_shape_validation():
    a, b = _fp8((64, 128)), _fp8((32, 128))
    d = torch.empty(64, 32, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="C must match D's pointer and shape"):
        deep_gemm.fp8_gemm_nt((a, torch.ones(64, 4)), (b, torch.ones(32, 4)), d, c=torch.zeros(2, 32, dtype=torch.bfloat16))


def test_shape_mismatch_is_reported():
    a, b = _fp8((64, 128)), _fp8((32, 256))
    d = torch.empty(64, 32, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="Conflicting shape dimension 'k'"):
        deep_gemm.fp8_gemm_nt((a, torch.ones(64, 4)), (b, torch.ones(32, 8)), d)


def test_ambiguous_major_axis():
    a = torch.zeros(4, 4, dtype=torch.float8_e4m3fn).as_strided((4, 4), (1, 1))
    b = _fp8((8, 4))
    d = torch.empty(4, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match='Ambiguous major axis'):
        deep_gemm.fp8_gemm_nt((a, torch.ones(4, 1)), (b, torch.ones(8, 1)), d)


def test_d_dtype_checked():
    a, b = _fp8((64, 128)), _fp8((32, 128))
    d = torch.empty(64, 32, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        deep_gemm.fp8_gemm_nt((a, torch.ones(64, 4)), (b, torch.ones(32, 4)), d)


def test_empty_m_returns_without_device_work():
    a, b = _fp8((0, 128)), _fp8((32, 128))
    d = torch.empty(0, 32, dtype=torch.bfloat16)
    deep_gemm.fp8_gemm_nt((a, torch.ones(0, 4)), (b, torch.ones(32, 4)), d)


def test_k_zero_zeroes_or_copies_d_on_host_tensors():
    a, b = _fp8((8, 0)), _fp8((4, 0))
    d = torch.full((8, 4), 3.0, dtype=torch.bfloat16)
    deep_gemm.fp8_gemm_nt((a, torch.ones(8, 0)), (b, torch.ones(4, 0)), d)
    assert torch.equal(d, torch.zeros(8, 4, dtype=torch.bfloat16))
    bias = torch.arange(4, dtype=torch.bfloat16).reshape(1, 4)
    deep_gemm.fp8_gemm_nt((a, torch.ones(8, 0)), (b, torch.ones(4, 0)), d, c=bias)
    assert torch.equal(d, bias.expand(8, 4))


def test_sf_layout_checks_and_passthrough():
    sf = torch.zeros(4, 1000, dtype=torch.int16).t()         # [1000, 4] MN-major packed
    assert dl.check_sf_layout(sf, 1000, 256, 1, 32, None) is True
    assert deep_gemm.transform_sf_into_required_layout(sf, 1000, 256, (1, 1, 32), is_sfa=True) is sf
    with pytest.raises(RuntimeError, match='is_sfa'):
        deep_gemm.transform_sf_into_required_layout(sf, 1000, 256, (1, 1, 32))
    with pytest.raises(RuntimeError, match='SF K extent'):
        dl.check_sf_layout(torch.zeros(1000, 3, dtype=torch.int16), 1000, 256, 1, 32, None)
    with pytest.raises(RuntimeError, match='disable_ue8m0_cast'):
        deep_gemm.transform_sf_into_required_layout(torch.ones(8, 4), 8, 128, (1, 1, 32), is_sfa=True,
                                                    disable_ue8m0_cast=True)


def test_mk_alignment_setter():
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    assert old == 256 == deep_gemm.get_theoretical_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(128)
    assert deep_gemm.get_mk_alignment_for_contiguous_layout() == 128
    with pytest.raises(RuntimeError):
        deep_gemm.set_mk_alignment_for_contiguous_layout(100)
    deep_gemm.set_mk_alignment_for_contiguous_layout(old)


def test_epilogue_checks_match_reference():
    """csrc/jit_kernels/epilogue_class.hpp:66-128: stochastic rounding needs a direct bf16 D, FP8
    quantization a direct e4m3 D with N % 128 == 0 and an M-major int16 SFD; the epilogue class,
    alpha and the FP8 pair are exclusive; the dense API only takes bf16 / fp32 D."""
    a, b = _fp8((64, 128)), _fp8((32, 128))
    sfa, sfb = torch.ones(64, 4), torch.ones(32, 4)
    d32 = torch.empty(64, 32)
    sr = deep_gemm.epilogue.BF16StochasticRounding()
    with pytest.raises(RuntimeError, match='Stochastic rounding requires a direct BF16 output'):
        deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d32, epilogue=sr)
    with pytest.raises(RuntimeError, match='exclusive'):
        deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d32, alpha=2.0, epilogue=sr)
    a3, b3 = _fp8((2, 64, 128)), _fp8((2, 256, 128))
    sfa3, sfb3 = torch.ones(2, 64, 4), torch.ones(2, 256, 4)
    # FP8 D rows hold every batch: [M, B, N] storage viewed as [B, M, N] (batch stride == N)
    d8 = torch.empty(64, 2, 256, dtype=torch.float8_e4m3fn).transpose(0, 1)
    good = torch.empty_strided((64, 2 * 256 // 64), (1, 64), dtype=torch.int16)
    bad = torch.empty(64, 2 * 256 // 64, dtype=torch.int16)
    with pytest.raises(RuntimeError):
        deep_gemm.fp8_bmm((a3, sfa3), (b3, sfb3), (d8, bad))
    with pytest.raises(RuntimeError, match='multiple of 128'):
        deep_gemm.fp8_bmm((a3, sfa3), (_fp8((2, 64, 128)), torch.ones(2, 64, 4)),
                          (torch.empty(64, 2, 64, dtype=torch.float8_e4m3fn).transpose(0, 1),
                           torch.empty_strided((64, 2), (1, 64), dtype=torch.int16)))
    with pytest.raises(RuntimeError, match='exclusive'):
        deep_gemm.fp8_bmm((a3, sfa3), (b3, sfb3), (d8, good), epilogue=deep_gemm.epilogue.FP8Quantization(good))
    # K == 0: D and SFD are zero-filled on the host without a launch
    d0 = torch.ones(64, 2, 256).to(torch.float8_e4m3fn).transpose(0, 1)
    s0 = good.fill_(7)
    deep_gemm.fp8_bmm((_fp8((2, 64, 0)), torch.ones(2, 64, 0)), (_fp8((2, 256, 0)), torch.ones(2, 256, 0)), (d0, s0))
    assert int(d0.view(torch.uint8).count_nonzero()) == 0 and int(s0.count_nonzero()) == 0


def test_import_is_lazy_and_fork_safe():
    """Importing deep_gemm loads neither the HIP library nor a GPU context (the reference
    keeps import fork-safe, tests/test_lazy_init.py)."""
    code = ('import sys, torch; sys.path.insert(0, "deepgemm-ascend_amd"); import deep_gemm; '
            'from deep_gemm import _lib; assert _lib._lib is None; '
            'assert not torch.cuda.is_initialized(); print("ok")')
    out = subprocess.run([sys.executable, '-c', code], capture_output=True, text=True, cwd=str(__import__('pathlib').Path(__file__).resolve().parents[1]))
    assert out.returncode == 0 and 'ok' in out.stdout, out.stderr


def test_batched_and_k_grouped_signatures_match_reference():
    """csrc/apis/einsum.hpp:201-220 and csrc/apis/gemm.hpp bindings."""
    import inspect
    assert list(inspect.signature(deep_gemm.fp8_bmm).parameters) == ['a', 'b', 'd', 'c', 'recipe', 'compiled_dims',
                                                                      'epilogue']
    assert inspect.signature(deep_gemm.fp8_bmm).parameters['recipe'].default == (1, 1, 32)
    assert list(inspect.signature(deep_gemm.bf16_bmm).parameters) == ['a', 'b', 'd', 'c', 'compiled_dims', 'epilogue']
    assert list(inspect.signature(deep_gemm.einsum).parameters) == ['expr', 'a', 'b', 'd', 'c', 'use_cublaslt',
                                                                    'epilogue']
    assert list(inspect.signature(deep_gemm.fp8_einsum).parameters) == ['expr', 'a', 'b', 'd', 'c', 'recipe',
                                                                        'epilogue']
    sig = inspect.signature(deep_gemm.k_grouped_fp8_gemm_tn_contiguous)
    assert list(sig.parameters) == ['a', 'b', 'd', 'ks_cpu', 'grouped_layout', 'c', 'recipe', 'compiled_dims',
                                    'use_psum_layout', 'epilogue']
    assert list(inspect.signature(deep_gemm.transform_k_grouped_sf_into_required_layout).parameters) == \
        ['sf', 'mn', 'k', 'recipe', 'is_sfa', 'psum_layout']


def test_einsum_validation_on_host():
    x = torch.empty(2, 2, 2, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match='Unsupported einsum expression'):
        deep_gemm.einsum('bhd,hrd->bhr', x, x, x)
    with pytest.raises(RuntimeError, match='use_cublaslt'):
        deep_gemm.einsum('bhr,hdr->bhd', x, x, x, use_cublaslt=True)
    with pytest.raises(RuntimeError, match='Unsupported einsum expression'):
        deep_gemm.fp8_einsum('xyz', (x, x), (x, x), x)


def test_bmm_shape_checks_and_empty_batch():
    a, b = _fp8((2, 16, 64)), _fp8((3, 8, 64))
    sf = torch.ones(2, 16, 2)
    d = torch.empty(2, 16, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        deep_gemm.fp8_bmm((a, sf), (b, torch.ones(3, 8, 2)), d)
    # batch 0 returns before any device work
    deep_gemm.bf16_bmm(torch.empty(0, 4, 8, dtype=torch.bfloat16), torch.empty(0, 4, 8, dtype=torch.bfloat16),
                       torch.empty(0, 4, 4, dtype=torch.bfloat16))
    # K == 0 zero-fills D on host tensors (csrc/utils/layout.hpp:54-86)
    d0 = torch.full((2, 4, 3), 5.0, dtype=torch.bfloat16)
    deep_gemm.bf16_bmm(torch.empty(2, 4, 0, dtype=torch.bfloat16), torch.empty(2, 3, 0, dtype=torch.bfloat16), d0)
    assert int(d0.count_nonzero()) == 0


def test_k_grouped_host_checks():
    a, b = _fp8((512, 64)), _fp8((512, 32))     # [Ktot, M], [Ktot, N] MN-major
    sfa, sfb = torch.ones(16, 64), torch.ones(16, 32)
    d = torch.empty(2, 64, 32, dtype=torch.bfloat16)
    layout = torch.tensor([256, 512], dtype=torch.int32)
    with pytest.raises(RuntimeError, match='use_psum_layout must be true'):
        deep_gemm.k_grouped_fp8_gemm_tn_contiguous((a, sfa), (b, sfb), d, None, layout, use_psum_layout=False)
    with pytest.raises(RuntimeError, match='MN-major'):
        deep_gemm.k_grouped_fp8_gemm_tn_contiguous((a.t().contiguous().t(), sfa), (b, sfb), d, None, layout)
    with pytest.raises(RuntimeError, match='D must be'):
        deep_gemm.k_grouped_fp8_gemm_tn_contiguous((a, sfa), (b, sfb), d[:1], None, layout)
    with pytest.warns(DeprecationWarning), pytest.raises(RuntimeError, match='D must be'):
        deep_gemm.k_grouped_fp8_gemm_nt_contiguous((a.t(), sfa.t()), (b.t(), sfb.t()), d[:1], None, layout)
