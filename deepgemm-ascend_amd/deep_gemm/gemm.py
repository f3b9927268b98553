"""GEMM API: validation, descriptor building and dispatch onto the HIP library.

Mirrors the reference's csrc/apis/gemm.hpp (get_gemm_desc :60-197, fp8_fp4_gemm :225-256,
m_grouped_fp8_fp4_gemm_contiguous :289-324, bf16_gemm :424-453, bindings :552-678) and
csrc/utils/layout.hpp (major detection :37-52, gemm_early_return :54-86, shape specs
:141-219): same names, argument order, defaults and error messages.  Every launch goes
through ``dg_gemm`` of libdeep_gemm_amd.so on the current HIP stream.

The kernels read K-major operands with 16-byte-aligned rows.  Operands given MN-major, or
with a K extent / stride that is not 16-byte aligned, are first copied into that layout on
the device (a layout conversion, not a change of the arithmetic).
"""
import ctypes
import os
import threading
from typing import Optional, Tuple

import torch

from . import _lib
from . import epilogue as _epi
from .layout import (transform_sf_into_required_layout, transform_k_grouped_sf_into_required_layout, get_recipe,
                     transform_sf_rows,
                     operand_recipes, _assert)
from .runtime import get_num_sms, get_mk_alignment_for_contiguous_layout, get_dry_run, get_jit

PACKED_FP4 = torch.int8   # the reference's kPackedFP4 (csrc/utils/dtype.hpp:9)
_FP4_TYPES = (torch.int8, getattr(torch, 'float4_e2m1fn_x2', torch.int8))


def _is_fp4(t: torch.Tensor) -> bool:
    return t.dtype in _FP4_TYPES


def _as_int8(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int8 else t.view(torch.int8)


def _major_is_k(t: torch.Tensor) -> bool:
    """csrc/utils/layout.hpp:37-47."""
    if t.stride(-2) == 1 and t.stride(-1) == 1 and t.size(-1) > 1 and t.size(-2) > 1:
        raise RuntimeError(f'Ambiguous major axis, the tensor has both last two dimensions contiguous, '
                           f'strides={list(t.stride())}')
    if t.stride(-1) == 1:
        return True
    _assert(t.stride(-2) == 1)
    return False


def _logical_k(t: torch.Tensor, k_is_major: bool) -> int:
    return t.size(-1) * (2 if _is_fp4(t) and k_is_major else 1)


def _logical_mn(t: torch.Tensor, k_is_major: bool) -> int:
    return t.size(-2) * (2 if _is_fp4(t) and not k_is_major else 1)


def _to_kernel_operand(t: torch.Tensor, k: int) -> torch.Tensor:
    """Return a [..., MN, K-storage] K-major tensor whose rows are 16-byte aligned."""
    fp4 = _is_fp4(t)
    k_major = _major_is_k(t)
    if fp4:
        t = _as_int8(t)
        if not k_major:
            # packed along MN -> packed along K, one pass of the HIP repack kernel
            return _fp4_to_k_major(t, k)
        kbytes, align_elems, esize = k // 2, 32, 1
    else:
        if not k_major:
            return _transpose_to_k_major(t, k)
        esize = t.element_size()
        kbytes, align_elems = k * esize, 16 // esize
    row_stride_bytes = t.stride(-2) * (1 if fp4 else esize)
    ok = (kbytes % 16 == 0 and row_stride_bytes % 16 == 0 and t.data_ptr() % 16 == 0 and t.stride(-1) == 1)
    if t.dim() == 3:
        ok = ok and (t.stride(0) * (1 if fp4 else esize)) % 16 == 0
    if ok:
        return t
    kpad = (k + align_elems - 1) // align_elems * align_elems
    store_k = kpad // 2 if fp4 else kpad
    out = torch.zeros((*t.shape[:-1], store_k), dtype=t.dtype, device=t.device)
    out[..., :t.size(-1)] = t
    return out


def _fp4_to_k_major(t: torch.Tensor, k: int) -> torch.Tensor:
    """FP4 operand packed along MN (an int8 [.., MN/2, K] view, stride(-2) == 1: bytes hold MN pairs)
    -> new [.., MN, align(K, 32) / 2] int8 tensor packed along K (zero K padding)."""
    if t.stride(-1) < t.size(-2) or (t.dim() == 3 and t.stride(0) < t.size(-2) * t.size(-1)):
        t = t.transpose(-2, -1).contiguous().transpose(-2, -1)   # explicit [.., K, MN/2] rows
    mn, kpad = t.size(-2) * 2, (k + 31) // 32 * 32
    out = torch.empty((*t.shape[:-2], mn, kpad // 2), dtype=torch.int8, device=t.device)
    if out.numel() == 0 or get_dry_run():
        return out
    batches = t.size(0) if t.dim() == 3 else 1
    lib = _lib.load()
    _lib.check(lib.dg_fp4_to_k_major(
        t.data_ptr(), batches, t.stride(0) if t.dim() == 3 else 0, t.stride(-1), k, mn,
        out.data_ptr(), mn * kpad // 2, kpad // 2, kpad, _stream(t)), lib)
    return out


def _transpose_to_k_major(t: torch.Tensor, k: int) -> torch.Tensor:
    """MN-major [.., MN, K] view (stride(-2) == 1) -> new K-major [.., MN, align(K, 16 B)] tensor
    (zero K padding), with the HIP transpose kernel."""
    esize = t.element_size()
    align_elems = 16 // esize
    kpad = (k + align_elems - 1) // align_elems * align_elems
    mn = t.size(-2)
    if t.stride(-1) < mn:   # degenerate strides of a size-1 K axis: make the MN-major rows explicit
        t = t.transpose(-2, -1).contiguous().transpose(-2, -1)
    batches = t.size(0) if t.dim() == 3 else 1
    out = torch.empty((*t.shape[:-2], mn, kpad), dtype=t.dtype, device=t.device)
    if out.numel() == 0 or get_dry_run():
        return out
    lib = _lib.load()
    _lib.check(lib.dg_transpose_to_k_major(
        t.data_ptr(), esize, batches, t.stride(0) if t.dim() == 3 else 0, t.stride(-1), k, mn,
        out.data_ptr(), mn * kpad, kpad, kpad, _stream(t)), lib)
    return out


def _mn_in_place(t: torch.Tensor, k: int) -> bool:
    """An e4m3 or bf16 MN-major operand ([.., MN, K] view with stride(-2) == 1) that the tile kernels
    can read in place: 16-byte aligned K rows and 16-byte K.  DG_MN_COPY=1 (tuning, tests) always
    copies instead."""
    if t.dtype not in (torch.float8_e4m3fn, torch.bfloat16) or _major_is_k(t) or os.environ.get('DG_MN_COPY') == '1':
        return False
    per16 = 16 // t.element_size()   # elements per 16 bytes
    if k % per16 or t.size(-1) < 2 or t.stride(-2) != 1 or t.stride(-1) % per16 or t.stride(-1) < t.size(-2):
        return False
    return t.data_ptr() % 16 == 0 and (t.dim() == 2 or t.stride(0) % per16 == 0)


def _launch_operands(args: _lib.GemmArgs, d: torch.Tensor, a: torch.Tensor, b: torch.Tensor, k: int,
                     batch_a: bool, batch_b: bool) -> None:
    """Set A and B (strides, batch strides, K) and launch.  e4m3 / bf16 MN-major operands are read in
    place by the 128-byte-stage tile kernels (the reference takes operand majors as kernel parameters,
    deep_gemm/include/deep_gemm/fp8_gemm.hpp:18-35), and MN-major B also by the skinny-M decode kernel
    (with both operands MN-major a decode call copies A only); a plan with another kernel (DG_ENOKERNEL)
    and every other operand get a K-major copy."""
    if args.kind in (_lib.DG_KIND_FP8_FP8, _lib.DG_KIND_BF16) and not get_dry_run() and not args.jit:
        a_mn, b_mn = _mn_in_place(a, k), _mn_in_place(b, k)
        if args.kind == _lib.DG_KIND_BF16 and not a_mn and args.gemm_type == _lib.DG_GEMM_NORMAL and args.m > 128:
            # dense bf16 with only B MN-major (nn) measured faster with B copied (4096x2112x7168: 176.0
            # vs 199.5 us; tn / tt gain in place: 183.9 vs 207.3, 172.1 vs 190.5).  M-grouped B is the
            # whole expert-weight tensor, read in place; decode shapes (M <= 128) read B in place with the
            # skinny-M kernel where their plan takes it.
            b_mn = False
        if a_mn or b_mn:
            a_k = a if a_mn else _to_kernel_operand(a, k)
            b_k = b if b_mn else _to_kernel_operand(b, k)
            if (a_mn or a_k.size(-1) == k) and (b_mn or b_k.size(-1) == k):
                args.k = k
                args.a, args.b = a_k.data_ptr(), b_k.data_ptr()
                args.lda = a_k.stride(-1) if a_mn else a_k.stride(-2)
                args.ldb = b_k.stride(-1) if b_mn else b_k.stride(-2)
                if batch_a:
                    args.batch_stride_a = a_k.stride(0)
                if batch_b:
                    args.batch_stride_b = b_k.stride(0)
                args.a_mn_major, args.b_mn_major = int(a_mn), int(b_mn)
                if _launch(args, d, allow_no_kernel=True):
                    return
                if a_mn and b_mn:
                    # (decode plans read MN-major B, not A, in place: copy only A, the smaller operand)
                    a_c = _to_kernel_operand(a, k)
                    if a_c.size(-1) == k:
                        args.a, args.lda, args.a_mn_major = a_c.data_ptr(), a_c.stride(-2), 0
                        if batch_a:
                            args.batch_stride_a = a_c.stride(0)
                        if _launch(args, d, allow_no_kernel=True):
                            return
                args.a_mn_major = args.b_mn_major = 0
    a_k = _to_kernel_operand(a, k)
    b_k = _to_kernel_operand(b, k)
    k_kernel = max(a_k.size(-1) * (2 if _is_fp4(a_k) else 1), b_k.size(-1) * (2 if _is_fp4(b_k) else 1))
    a_k, b_k = _pad_k(a_k, k_kernel), _pad_k(b_k, k_kernel)
    args.k = k_kernel
    args.a, args.b = a_k.data_ptr(), b_k.data_ptr()
    args.lda, args.ldb = a_k.stride(-2), b_k.stride(-2)
    if batch_a:
        args.batch_stride_a = a_k.stride(0)
    if batch_b:
        args.batch_stride_b = b_k.stride(0)
    _launch(args, d)


_raw_stream = getattr(torch._C, '_cuda_getCurrentRawStream', None)


def _stream(t: torch.Tensor) -> int:
    # (torch's raw current-stream handle skips building a Stream object on every launch)
    if _raw_stream is not None and t.device.index is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def _kind(a: torch.Tensor, b: torch.Tensor) -> int:
    """dispatch_fp8_fp4_gemm (csrc/apis/gemm.hpp:22-33)."""
    fa, fb = _is_fp4(a), _is_fp4(b)
    if a.dtype == torch.float8_e4m3fn and b.dtype == torch.float8_e4m3fn:
        return _lib.DG_KIND_FP8_FP8
    if fa and fb:
        return _lib.DG_KIND_FP4_FP4
    if a.dtype == torch.float8_e4m3fn and fb:
        return _lib.DG_KIND_FP8_FP4
    raise RuntimeError('Unsupported operand dtypes')


# The C++ host path (csrc/torch_ext.cpp) serves the common calls: K-major aligned operands, no
# bias, alpha or output epilogue, no dry run, JIT or tuning override.  It returns False for
# anything else, and the Python path below then runs (and raises the reference's errors).
_OVERRIDES = ('DG_SPLIT_K', 'DG_FORCE_BLOCK', 'DG_CHECK_SF')
_recipe_cache = {}


def _fast():
    """The extension when the fast path may serve this call, else None."""
    from . import runtime as _rt
    if _rt._dry_run or _rt._jit:
        return None
    env = os.environ
    for key in _OVERRIDES:
        if key in env:
            return None
    return _lib.ext()


def _fast_recipes(recipe, recipe_a, recipe_b):
    """operand_recipes flattened to (gran_a_mn, gran_a_k, gran_b_mn, gran_b_k), memoised."""
    key = (recipe, recipe_a, recipe_b)
    try:
        hit = _recipe_cache.get(key)
    except TypeError:   # (unhashable recipe lists)
        (ga, ka), (gb, kb) = operand_recipes(recipe, recipe_a, recipe_b)
        return ga, ka, gb, kb
    if hit is None:
        (ga, ka), (gb, kb) = operand_recipes(recipe, recipe_a, recipe_b)
        hit = _recipe_cache[key] = (ga, ka, gb, kb)
    return hit


def _fast_gemm(gemm_type, a, sfa, b, sfb, d, c, layout, recipes) -> bool:
    if not d.is_cuda:
        return False
    ext = _fast()
    if ext is None:
        return False
    from . import runtime as _rt
    ga, ka, gb, kb = recipes
    return ext.gemm(gemm_type, a, sfa, b, sfb, d, c, layout, ga, ka, gb, kb, _rt._num_sms, _rt._mk_alignment,
                    _stream(d))


def _launch(args: _lib.GemmArgs, d: torch.Tensor, allow_no_kernel: bool = False) -> bool:
    """Launch (or, in a dry run, compile); with allow_no_kernel a plan without a compiled kernel
    returns False instead of raising."""
    _lib.raise_pending()
    if get_dry_run():
        # the reference's dry run compiles the kernel without loading or launching it
        # (csrc/jit_kernels/fp8_gemm.hpp:75-78); ahead-of-time kernels need nothing
        if args.jit:
            lib = _lib.load()
            _lib.check(lib.dg_jit_compile(args), lib)
        return True
    lib = _lib.load()
    stream = _stream(d)
    forced = os.environ.get('DG_SPLIT_K')   # tuning override: 1 = never split, n > 1 = split n ways
    if forced:
        args.split_k = int(forced)
    if args.gemm_type in (_lib.DG_GEMM_NORMAL, _lib.DG_GEMM_BATCHED) and args.split_k != 1:
        # split-K partials and tile counters go to the library's workspace of this stream (grown
        # only outside graph capture, never freed)
        args.library_workspace = 1
    rc = lib.dg_gemm(args, stream)
    if allow_no_kernel and rc == _lib.DG_ENOKERNEL:
        return False
    _lib.check(rc, lib)
    return True


def _fill_common(args, d, k_kernel, alpha, kind, dims: str = 'nk'):
    args.kind = kind
    args.d = d.data_ptr()
    args.ldd = d.stride(-2)
    args.d_dtype = {torch.float32: _lib.DG_DTYPE_F32, torch.float8_e4m3fn: _lib.DG_DTYPE_FP8_E4M3}.get(
        d.dtype, _lib.DG_DTYPE_BF16)
    args.alpha = 1.0 if alpha is None else float(alpha)
    args.k = k_kernel
    args.num_cus = get_num_sms()
    args.alignment = get_mk_alignment_for_contiguous_layout()
    # run-time compiled kernels (set_jit): the GEMM type and K split, plus the `compiled_dims` sizes,
    # become compile-time constants (the reference's compiled_dims, csrc/jit_kernels/fp8_gemm.hpp:42-44)
    args.jit = 1 if get_jit() else 0
    args.compiled_dims = (_lib.DG_COMPILED_M if 'm' in dims else 0) | (_lib.DG_COMPILED_N if 'n' in dims else 0) | \
        (_lib.DG_COMPILED_K if 'k' in dims else 0)
    forced = os.environ.get('DG_FORCE_BLOCK')   # e.g. "256x224": tuning override of the heuristic
    if forced:
        args.block_m, args.block_n = (int(x) for x in forced.split('x'))


def _early_return(m, n, k, d, c, is_cd_same, with_bias, sfd=None) -> bool:
    """csrc/utils/layout.hpp:54-86."""
    if m == 0 or n == 0:
        return True
    _assert(sfd is None or c is None)
    if is_cd_same:
        _assert(c.shape == d.shape and c.stride() == d.stride())
    _assert(d.dtype in (torch.bfloat16, torch.float32, torch.float8_e4m3fn))
    _assert((d.dtype == torch.float8_e4m3fn) == (sfd is not None))
    if c is not None:
        _assert(c.stride(-1) == 1)
        _assert(d.dtype == c.dtype)
    if k == 0:
        if not is_cd_same:
            if c is not None and not with_bias:
                d.copy_(c)
            elif c is not None:
                d.copy_(c.expand_as(d))
            else:
                d.zero_()
        if sfd is not None:
            sfd.zero_()
        return True
    return False


def _apply_epilogue(args, epi) -> None:
    """Epilogue class -> dg_gemm_args fields (after _fill_common)."""
    if isinstance(epi, _epi.BF16StochasticRounding):
        args.epilogue = _lib.DG_EPI_BF16_SR
    elif isinstance(epi, _epi.FP8Quantization):
        args.d_dtype = _lib.DG_DTYPE_FP8_E4M3
        args.sfd = epi.sfd.data_ptr()
        args.sfd_ld = epi.sfd.stride(1)


def _dense_gemm(a, sfa, b, sfb, d, c, recipe, recipe_a, recipe_b, disable_ue8m0_cast, alpha, epilogue,
                bf16: bool, dims: str = 'nk'):
    """fp8_fp4_gemm / bf16_gemm after the nt/nn/tn/tt transposes (csrc/apis/gemm.hpp:225-256, 424-453)."""
    _assert(d.dtype in (torch.bfloat16, torch.float32))
    if bf16:
        _assert(a.dtype == torch.bfloat16)
        _assert(b.dtype == torch.bfloat16)
    epi = _epi.resolve(epilogue, c, d, alpha)
    ka, kb = _major_is_k(a), _major_is_k(b)
    m, k = _logical_mn(a, ka), _logical_k(a, ka)
    n, k_b = _logical_mn(b, kb), _logical_k(b, kb)
    if k != k_b:
        raise RuntimeError(f"Conflicting shape dimension 'k': A gives {k}, B gives {k_b}")
    _assert(d.dim() == 2 and d.size(0) == m and d.size(1) == n, f'D shape {tuple(d.shape)} != ({m}, {n})')
    _assert(d.stride(-1) == 1)
    is_cd_same = c is not None and c.data_ptr() == d.data_ptr() and d.numel() > 0
    with_bias = c is not None and not is_cd_same
    if c is not None:
        _assert(c.dim() == 2 and c.size(0) == (1 if with_bias else m) and c.size(1) == n,
                "C must match D's pointer and shape for accumulation, or be a separate [1, N] bias")
        _assert(c.device == d.device, 'C and D must be on the same device')
    if with_bias:
        _assert(c.is_contiguous(), 'Bias must be contiguous')
        _assert(not isinstance(epi, _epi.Alpha), 'alpha and bias cannot be used together')
    if _early_return(m, n, k, d, c, is_cd_same, with_bias):
        return
    alpha_v = epi.alpha if isinstance(epi, _epi.Alpha) else None

    args = _lib.GemmArgs()
    if bf16:
        kind = _lib.DG_KIND_BF16
    else:
        kind = _kind(a, b)
        ra, rb = operand_recipes(recipe, recipe_a, recipe_b)
        sfa_t = transform_sf_into_required_layout(sfa, m, k, ra, None, True, disable_ue8m0_cast)
        sfb_t = transform_sf_into_required_layout(sfb, n, k, rb, None, False, disable_ue8m0_cast)
        args.sfa, args.sfb = sfa_t.data_ptr(), sfb_t.data_ptr()
        args.sfa_ld, args.sfb_ld = sfa_t.stride(-1), sfb_t.stride(-1)
    _fill_common(args, d, k, alpha_v, kind, dims)
    args.gemm_type = _lib.DG_GEMM_NORMAL
    args.m, args.n, args.num_groups = m, n, 1
    args.accumulate = 1 if is_cd_same else 0
    args.bias = c.data_ptr() if with_bias else None
    _apply_epilogue(args, epi)
    _launch_operands(args, d, a, b, k, batch_a=False, batch_b=False)


def _pad_k(t: torch.Tensor, k: int) -> torch.Tensor:
    store = k // 2 if _is_fp4(t) else k
    if t.size(-1) == store:
        return t
    out = torch.zeros((*t.shape[:-1], store), dtype=t.dtype, device=t.device)
    out[..., :t.size(-1)] = t
    return out


def _make_fp8_fp4_gemm(trans_a: bool, trans_b: bool, default_dims: str):
    def fn(a: Tuple[torch.Tensor, torch.Tensor], b: Tuple[torch.Tensor, torch.Tensor], d: torch.Tensor,
           c: Optional[torch.Tensor] = None, recipe=None, recipe_a=None, recipe_b=None,
           compiled_dims: str = default_dims, disable_ue8m0_cast: bool = False,
           alpha: Optional[float] = None, epilogue=None) -> None:
        (a_, sfa), (b_, sfb) = a, b
        if not (trans_a or trans_b) and alpha is None and epilogue is None and not disable_ue8m0_cast and \
                _fast_gemm(0, a_, sfa, b_, sfb, d, c, None, _fast_recipes(recipe, recipe_a, recipe_b)):
            return
        if trans_a:
            a_, sfa = a_.transpose(0, 1), sfa.transpose(0, 1)
        if trans_b:
            b_, sfb = b_.transpose(0, 1), sfb.transpose(0, 1)
        _dense_gemm(a_, sfa, b_, sfb, d, c, recipe, recipe_a, recipe_b, disable_ue8m0_cast, alpha, epilogue,
                    bf16=False, dims=compiled_dims)
    return fn


fp8_fp4_gemm_nt = _make_fp8_fp4_gemm(False, False, 'nk')
fp8_fp4_gemm_nn = _make_fp8_fp4_gemm(False, True, 'nk')
fp8_fp4_gemm_tn = _make_fp8_fp4_gemm(True, True, 'mn')
fp8_fp4_gemm_tt = _make_fp8_fp4_gemm(True, False, 'mn')
for _f, _name in ((fp8_fp4_gemm_nt, 'nt'), (fp8_fp4_gemm_nn, 'nn'), (fp8_fp4_gemm_tn, 'tn'), (fp8_fp4_gemm_tt, 'tt')):
    _f.__name__ = f'fp8_fp4_gemm_{_name}'
    _f.__doc__ = (f'D = A @ B^T (+ C) with the `{_name}` logical operand shapes; block-scaled e4m3/e2m1 '
                  f'operands (csrc/apis/gemm.hpp:199-256).')


def _make_bf16_gemm(trans_a: bool, trans_b: bool, default_dims: str):
    def fn(a: torch.Tensor, b: torch.Tensor, d: torch.Tensor, c: Optional[torch.Tensor] = None,
           compiled_dims: str = default_dims, alpha: Optional[float] = None, epilogue=None) -> None:
        if not (trans_a or trans_b) and alpha is None and epilogue is None and \
                _fast_gemm(0, a, None, b, None, d, c, None, (0, 0, 0, 0)):
            return
        a_ = a.transpose(0, 1) if trans_a else a
        b_ = b.transpose(0, 1) if trans_b else b
        _dense_gemm(a_, None, b_, None, d, c, None, None, None, False, alpha, epilogue, bf16=True, dims=compiled_dims)
    return fn


bf16_gemm_nt = _make_bf16_gemm(False, False, 'nk')
bf16_gemm_nn = _make_bf16_gemm(False, True, 'nk')
bf16_gemm_tn = _make_bf16_gemm(True, True, 'mn')
bf16_gemm_tt = _make_bf16_gemm(True, False, 'mn')
for _f, _name in ((bf16_gemm_nt, 'nt'), (bf16_gemm_nn, 'nn'), (bf16_gemm_tn, 'tn'), (bf16_gemm_tt, 'tt')):
    _f.__name__ = f'bf16_gemm_{_name}'


def _grouped_contiguous(a, sfa, b, sfb, d, grouped_layout, recipe, recipe_a, recipe_b, disable_ue8m0_cast,
                        use_psum_layout, epilogue, bf16: bool, dims: str = 'nk'):
    """m_grouped_fp8_fp4_gemm_contiguous / m_grouped_bf16_gemm_contiguous (csrc/apis/gemm.hpp:289-324, 470-499)."""
    if bf16:
        _assert(a.dtype == torch.bfloat16)
        _assert(b.dtype == torch.bfloat16)
    else:
        _assert(a.dtype == torch.float8_e4m3fn or _is_fp4(a))
        _assert(b.dtype == torch.float8_e4m3fn or _is_fp4(b))
    _assert(d.dtype in (torch.bfloat16, torch.float32))
    epi = _epi.resolve(epilogue, None, d)
    _assert(_major_is_k(a))
    kb = _major_is_k(b)
    m, k = _logical_mn(a, True), _logical_k(a, True)
    _assert(b.dim() == 3, 'B must be [G, N, K]')
    g = b.size(0)
    n, k_b = _logical_mn(b, kb), _logical_k(b, kb)
    _assert(k == k_b, f"Conflicting shape dimension 'k': A gives {k}, B gives {k_b}")
    _assert(d.dim() == 2 and d.size(0) == m and d.size(1) == n and d.stride(-1) == 1)
    _assert(grouped_layout.is_contiguous())
    _assert(grouped_layout.dtype == torch.int32)
    if use_psum_layout:
        _assert(grouped_layout.numel() == g, f"Conflicting shape dimension 'g': {grouped_layout.numel()} vs {g}")
    else:
        _assert(grouped_layout.numel() == m, 'm_indices must have one entry per row of A')
    if m == 0 or n == 0:
        return
    if k == 0:
        d.zero_()
        return
    alignment = get_mk_alignment_for_contiguous_layout()
    args = _lib.GemmArgs()
    if bf16:
        kind = _lib.DG_KIND_BF16
    else:
        kind = _kind(a, b)
        ra, rb = operand_recipes(recipe, recipe_a, recipe_b)
        sfa_t = transform_sf_rows(sfa, m, k, ra, None, True, disable_ue8m0_cast,
                                  grouped_layout if use_psum_layout else None,
                                  None if use_psum_layout else grouped_layout)
        sfb_t = transform_sf_into_required_layout(sfb, n, k, rb, g, False, disable_ue8m0_cast)
        args.sfa, args.sfb = sfa_t.data_ptr(), sfb_t.data_ptr()
        args.sfa_ld, args.sfb_ld = sfa_t.stride(-1), sfb_t.stride(-1)
        args.sfb_batch_stride = sfb_t.stride(0)
    _fill_common(args, d, k, None, kind, dims)
    args.alignment = alignment
    args.gemm_type = _lib.DG_GEMM_MGROUPED_PSUM if use_psum_layout else _lib.DG_GEMM_MGROUPED_IDX
    args.grouped_layout = grouped_layout.data_ptr()
    args.m, args.n, args.num_groups = m, n, g
    _apply_epilogue(args, epi)
    _launch_operands(args, d, a, b, k, batch_a=False, batch_b=True)


def _make_m_grouped_fp8_fp4(trans_b: bool):
    def fn(a, b, d, grouped_layout, recipe=None, recipe_a=None, recipe_b=None, compiled_dims: str = 'nk',
           disable_ue8m0_cast: bool = False, use_psum_layout: bool = True, ensure_zero_padding: bool = True,
           expected_m_for_psum_layout: Optional[int] = None, epilogue=None) -> None:
        (a_, sfa), (b_, sfb) = a, b
        if not trans_b and epilogue is None and not disable_ue8m0_cast and \
                _fast_gemm(2 if use_psum_layout else 3, a_, sfa, b_, sfb, d, None, grouped_layout,
                           _fast_recipes(recipe, recipe_a, recipe_b)):
            return
        if trans_b:
            b_, sfb = b_.transpose(1, 2), sfb.transpose(1, 2)
        _grouped_contiguous(a_, sfa, b_, sfb, d, grouped_layout, recipe, recipe_a, recipe_b, disable_ue8m0_cast,
                            use_psum_layout, epilogue, bf16=False, dims=compiled_dims)
    return fn


m_grouped_fp8_fp4_gemm_nt_contiguous = _make_m_grouped_fp8_fp4(False)
m_grouped_fp8_fp4_gemm_nn_contiguous = _make_m_grouped_fp8_fp4(True)
m_grouped_fp8_fp4_gemm_nt_contiguous.__name__ = 'm_grouped_fp8_fp4_gemm_nt_contiguous'
m_grouped_fp8_fp4_gemm_nn_contiguous.__name__ = 'm_grouped_fp8_fp4_gemm_nn_contiguous'


def _make_m_grouped_bf16(trans_b: bool):
    def fn(a, b, d, grouped_layout, compiled_dims: str = 'nk', use_psum_layout: bool = True,
           ensure_zero_padding: bool = True, expected_m_for_psum_layout: Optional[int] = None,
           epilogue=None) -> None:
        if not trans_b and epilogue is None and \
                _fast_gemm(2 if use_psum_layout else 3, a, None, b, None, d, None, grouped_layout, (0, 0, 0, 0)):
            return
        b_ = b.transpose(1, 2) if trans_b else b
        _grouped_contiguous(a, None, b_, None, d, grouped_layout, None, None, None, False, use_psum_layout,
                            epilogue, bf16=True, dims=compiled_dims)
    return fn


m_grouped_bf16_gemm_nt_contiguous = _make_m_grouped_bf16(False)
m_grouped_bf16_gemm_nn_contiguous = _make_m_grouped_bf16(True)


def _masked(a, sfa, b, sfb, d, masked_m, recipe, recipe_a, recipe_b, disable_ue8m0_cast, bf16: bool, dims: str = 'nk'):
    """Masked grouped GEMM, upstream DeepGEMM semantics: D[g, :masked_m[g]] = A[g, :masked_m[g]] @ B[g]^T.
    The reference has no masked kernel (csrc/apis/gemm.hpp:606,630)."""
    _assert(a.dim() == 3 and b.dim() == 3 and d.dim() == 3, 'masked GEMM takes A [G,M,K], B [G,N,K], D [G,M,N]')
    _assert(d.dtype in (torch.bfloat16, torch.float32))
    _assert(_major_is_k(a))
    kb = _major_is_k(b)
    g, m, k = a.size(0), _logical_mn(a, True), _logical_k(a, True)
    n, k_b = _logical_mn(b, kb), _logical_k(b, kb)
    _assert(k == k_b and b.size(0) == g and d.size(0) == g and d.size(1) == m and d.size(2) == n)
    _assert(d.stride(-1) == 1)
    _assert(masked_m.dtype == torch.int32 and masked_m.is_contiguous() and masked_m.numel() == g)
    if m == 0 or n == 0 or k == 0:
        if k == 0:
            d.zero_()
        return
    args = _lib.GemmArgs()
    if bf16:
        kind = _lib.DG_KIND_BF16
    else:
        kind = _kind(a, b)
        ra, rb = operand_recipes(recipe, recipe_a, recipe_b)
        sfa_t = transform_sf_into_required_layout(sfa, m, k, ra, g, True, disable_ue8m0_cast)
        sfb_t = transform_sf_into_required_layout(sfb, n, k, rb, g, False, disable_ue8m0_cast)
        args.sfa, args.sfb = sfa_t.data_ptr(), sfb_t.data_ptr()
        args.sfa_ld, args.sfb_ld = sfa_t.stride(-1), sfb_t.stride(-1)
        args.sfa_batch_stride, args.sfb_batch_stride = sfa_t.stride(0), sfb_t.stride(0)
    a_k = _to_kernel_operand(a, k)
    b_k = _to_kernel_operand(b, k)
    k_kernel = max(a_k.size(-1) * (2 if _is_fp4(a_k) else 1), b_k.size(-1) * (2 if _is_fp4(b_k) else 1))
    a_k, b_k = _pad_k(a_k, k_kernel), _pad_k(b_k, k_kernel)
    _fill_common(args, d, k_kernel, None, kind, dims)
    args.gemm_type = _lib.DG_GEMM_MASKED
    args.a, args.b = a_k.data_ptr(), b_k.data_ptr()
    args.lda, args.ldb = a_k.stride(-2), b_k.stride(-2)
    args.batch_stride_a, args.batch_stride_b, args.batch_stride_d = a_k.stride(0), b_k.stride(0), d.stride(0)
    args.grouped_layout = masked_m.data_ptr()
    args.m, args.n, args.num_groups = m, n, g
    _launch(args, d)


def m_grouped_fp8_fp4_gemm_nt_masked(a, b, d, masked_m: torch.Tensor, expected_m: int, recipe=None,
                                     recipe_a=None, recipe_b=None, compiled_dims: str = 'nk',
                                     disable_ue8m0_cast: bool = False) -> None:
    (a_, sfa), (b_, sfb) = a, b
    if not disable_ue8m0_cast and _fast_gemm(4, a_, sfa, b_, sfb, d, None, masked_m,
                                             _fast_recipes(recipe, recipe_a, recipe_b)):
        return
    _masked(a_, sfa, b_, sfb, d, masked_m, recipe, recipe_a, recipe_b, disable_ue8m0_cast, bf16=False, dims=compiled_dims)


def m_grouped_bf16_gemm_nt_masked(a, b, d, masked_m: torch.Tensor, expected_m: int,
                                  compiled_dims: str = 'nk') -> None:
    if _fast_gemm(4, a, None, b, None, d, None, masked_m, (0, 0, 0, 0)):
        return
    _masked(a, None, b, None, d, masked_m, None, None, None, False, bf16=True, dims=compiled_dims)


def _batched(a, sfa, b, sfb, d, c, recipe, bf16: bool, epilogue=None, dims: str = 'nk'):
    """Batched GEMM D[i] = A[i] @ B[i]^T (+ C[i]): fp8_bmm / bf16_bmm (csrc/apis/einsum.hpp:37-97),
    get_gemm_desc with GemmType::Batched (csrc/apis/gemm.hpp:60-197).  ``d`` may be an
    (e4m3 D, SFD) pair (fp8_bmm only)."""
    sfd = None
    if isinstance(d, tuple):
        _assert(not bf16, 'bf16_bmm has no FP8 output')
        d, sfd = d
    if bf16:
        _assert(a.dtype == torch.bfloat16)
        _assert(b.dtype == torch.bfloat16)
        _assert(d.dtype in (torch.float32, torch.bfloat16))
    else:
        _assert(a.dtype == torch.float8_e4m3fn)
        _assert(b.dtype == torch.float8_e4m3fn)
    _assert(a.dim() == 3 and b.dim() == 3 and d.dim() == 3, 'batched GEMM takes A [B,M,K], B [B,N,K], D [B,M,N]')
    ka, kb = _major_is_k(a), _major_is_k(b)
    bs, m, k = a.size(0), _logical_mn(a, ka), _logical_k(a, ka)
    n, k_b = _logical_mn(b, kb), _logical_k(b, kb)
    if k != k_b:
        raise RuntimeError(f"Conflicting shape dimension 'k': A gives {k}, B gives {k_b}")
    _assert(b.size(0) == bs and d.size(0) == bs and d.size(1) == m and d.size(2) == n,
            f'D shape {tuple(d.shape)} != ({bs}, {m}, {n})')
    _assert(d.stride(-1) == 1)
    if bs == 0:
        return
    epi = _epi.resolve(epilogue, c, d, None, sfd)
    if isinstance(epi, _epi.FP8Quantization):
        sfd = epi.sfd
    is_cd_same = c is not None and c.data_ptr() == d.data_ptr() and d.numel() > 0
    if c is not None:
        _assert(c.shape == d.shape and c.dtype == d.dtype and c.stride(-1) == 1)
    if _early_return(m, n, k, d, c, is_cd_same, False, sfd):
        return
    args = _lib.GemmArgs()
    if bf16:
        kind = _lib.DG_KIND_BF16
    else:
        kind = _lib.DG_KIND_FP8_FP8
        ra, rb = operand_recipes(recipe, None, None)
        sfa_t = transform_sf_into_required_layout(sfa, m, k, ra, bs, True)
        sfb_t = transform_sf_into_required_layout(sfb, n, k, rb, bs, False)
        if sfa_t.dim() == 2:
            sfa_t = sfa_t.unsqueeze(0)
        if sfb_t.dim() == 2:
            sfb_t = sfb_t.unsqueeze(0)
        args.sfa, args.sfb = sfa_t.data_ptr(), sfb_t.data_ptr()
        args.sfa_ld, args.sfb_ld = sfa_t.stride(-1), sfb_t.stride(-1)
        args.sfa_batch_stride, args.sfb_batch_stride = sfa_t.stride(0), sfb_t.stride(0)
    if c is not None and not is_cd_same:
        d.copy_(c)   # the reference's legacy accumulation path (csrc/utils/layout.hpp:82-84)
    _fill_common(args, d, k, None, kind, dims)
    args.gemm_type = _lib.DG_GEMM_BATCHED
    args.batch_stride_d = d.stride(0)
    args.m, args.n, args.num_groups = m, n, bs
    args.accumulate = 1 if c is not None else 0
    _apply_epilogue(args, epi)
    _launch_operands(args, d, a, b, k, batch_a=True, batch_b=True)


def _k_grouped(a, sfa, b, sfb, d, grouped_layout, c, recipe, use_psum_layout, epilogue, bf16: bool, dims: str = 'mn'):
    """K-grouped contiguous GEMM, D[g] = A[Kg]^T @ B[Kg] (+ C[g]) with A [Ktot, M], B [Ktot, N]
    (the `tn` layout) and K split by a psum layout: k_grouped_fp8_gemm_tn_contiguous
    (csrc/apis/gemm.hpp:351-387) and k_grouped_bf16_gemm_tn_contiguous (:515-...)."""
    _assert(use_psum_layout, 'use_psum_layout must be true')
    # [K, M] -> logical [M, K] (a view; the data stays MN-major)
    a_t, b_t = a.transpose(0, 1), b.transpose(0, 1)
    if bf16:
        _assert(a.dtype == torch.bfloat16)
        _assert(b.dtype == torch.bfloat16)
    else:
        _assert(a.dtype == torch.float8_e4m3fn or _is_fp4(a))
        _assert(b.dtype == torch.float8_e4m3fn or _is_fp4(b))
    _assert(d.dtype in (torch.bfloat16, torch.float32))
    epi = _epi.resolve(epilogue, c, d)
    _assert(grouped_layout.is_contiguous() and grouped_layout.dtype == torch.int32 and grouped_layout.dim() == 1)
    g = grouped_layout.numel()
    ka, kb = _major_is_k(a_t), _major_is_k(b_t)
    _assert(not ka and not kb, 'K-grouped operands must be MN-major ([K, M] / [K, N] contiguous along MN)')
    m, k = _logical_mn(a_t, ka), _logical_k(a_t, ka)
    n, k_b = _logical_mn(b_t, kb), _logical_k(b_t, kb)
    if k != k_b:
        raise RuntimeError(f"Conflicting shape dimension 'k': A gives {k}, B gives {k_b}")
    _assert(d.dim() == 3 and d.size(0) == g and d.size(1) == m and d.size(2) == n and d.stride(-1) == 1,
            f'D must be [{g}, {m}, {n}]')
    is_cd_same = c is not None and c.data_ptr() == d.data_ptr() and d.numel() > 0
    if c is not None:
        _assert(c.shape == d.shape and c.dtype == d.dtype and c.stride(-1) == 1)
    if _early_return(m, n, k, d, c, is_cd_same, False):
        return
    alignment = get_mk_alignment_for_contiguous_layout()
    _assert(alignment % 64 == 0, 'K-grouped GEMMs need an mk alignment that is a multiple of 64')
    args = _lib.GemmArgs()
    if bf16:
        kind = _lib.DG_KIND_BF16
    else:
        kind = _kind(a, b)
        rcp = get_recipe(recipe, None, None)
        sfa_t = transform_k_grouped_sf_into_required_layout(sfa.transpose(0, 1), m, k, rcp, True, grouped_layout)
        sfb_t = transform_k_grouped_sf_into_required_layout(sfb.transpose(0, 1), n, k, rcp, False, grouped_layout)
        args.sfa, args.sfb = sfa_t.data_ptr(), sfb_t.data_ptr()
        args.sfa_ld, args.sfb_ld = sfa_t.stride(-1), sfb_t.stride(-1)
    if c is not None and not is_cd_same:
        d.copy_(c)
    _fill_common(args, d, k, None, kind, dims)
    args.alignment = alignment
    args.gemm_type = _lib.DG_GEMM_KGROUPED
    args.batch_stride_d = d.stride(0)
    args.grouped_layout = grouped_layout.data_ptr()
    args.m, args.n, args.num_groups = m, n, g
    args.accumulate = 1 if c is not None else 0
    _apply_epilogue(args, epi)
    _launch_operands(args, d, a_t, b_t, k, batch_a=False, batch_b=False)


def k_grouped_fp8_gemm_tn_contiguous(a, b, d, ks_cpu, grouped_layout, c=None, recipe=(1, 1, 32),
                                     compiled_dims: str = 'mn', use_psum_layout: bool = True, epilogue=None) -> None:
    """K-grouped contiguous low-precision GEMM (csrc/apis/gemm.hpp:326-387): A [Ktot, M], B [Ktot, N], D [G, M, N].
    ``ks_cpu`` is a hint only (the reference uses it for its cost model)."""
    (a_, sfa), (b_, sfb) = a, b
    _k_grouped(a_, sfa, b_, sfb, d, grouped_layout, c, recipe, use_psum_layout, epilogue, bf16=False, dims=compiled_dims)


def k_grouped_fp8_gemm_nt_contiguous(a, b, d, ks_cpu, grouped_layout, c=None, recipe=(1, 1, 32),
                                     compiled_dims: str = 'mn', use_psum_layout: bool = True, epilogue=None) -> None:
    """Deprecated `nt` form (csrc/apis/gemm.hpp:389-411): A [M, Ktot], B [N, Ktot]."""
    import warnings
    warnings.warn('Calling k_grouped_fp8_gemm_nt_contiguous is deprecated, please transpose a, b into [k, m] and '
                  '[k, n] shape and call `k_grouped_fp8_gemm_tn_contiguous` instead', DeprecationWarning, stacklevel=2)
    (a_, sfa), (b_, sfb) = a, b
    k_grouped_fp8_gemm_tn_contiguous((a_.transpose(0, 1), sfa.transpose(0, 1)), (b_.transpose(0, 1), sfb.transpose(0, 1)),
                                     d, ks_cpu, grouped_layout, c, recipe, compiled_dims, use_psum_layout, epilogue)


def k_grouped_bf16_gemm_tn_contiguous(a, b, d, ks_cpu, grouped_layout, c=None, compiled_dims: str = 'mn',
                                      use_psum_layout: bool = True, epilogue=None) -> None:
    """K-grouped contiguous bf16 GEMM (csrc/apis/gemm.hpp:515-...)."""
    _k_grouped(a, None, b, None, d, grouped_layout, c, None, use_psum_layout, epilogue, bf16=True, dims=compiled_dims)


def select_config(m: int, n: int, k: int, kind: int = _lib.DG_KIND_FP8_FP8, gemm_type: int = _lib.DG_GEMM_NORMAL,
                  num_groups: int = 1) -> Tuple[int, int]:
    """Tile shape (block_m, block_n) the library heuristic picks (for DG_PRINT_CONFIGS-style inspection)."""
    args = _lib.GemmArgs()
    args.kind, args.gemm_type, args.m, args.n, args.k, args.num_groups = kind, gemm_type, m, n, k, num_groups
    args.alignment = get_mk_alignment_for_contiguous_layout()
    args.num_cus = get_num_sms()
    import ctypes
    bm, bn = ctypes.c_int32(), ctypes.c_int32()
    lib = _lib.load()
    _lib.check(lib.dg_select_config(args, ctypes.byref(bm), ctypes.byref(bn)), lib)
    return bm.value, bn.value


def launch_plan(m: int, n: int, k: int, kind: int = _lib.DG_KIND_FP8_FP8, gemm_type: int = _lib.DG_GEMM_NORMAL,
                num_groups: int = 1, split_k: int = 0) -> dict:
    """The launch the library would make for a K-major GEMM of this shape under the current
    runtime settings (set_num_sms, mk alignment): tile, workgroups, threads, tiles, K split and
    whether the workgroups walk tiles persistently (split_k > 1 forces a K split, as DG_SPLIT_K
    does for the calls).  Nothing is launched."""
    import ctypes
    args = _lib.GemmArgs()
    # K as the calls pass it to the kernels: padded so rows stay whole 16-byte pieces
    k = -(-k // {_lib.DG_KIND_BF16: 8, _lib.DG_KIND_FP4_FP4: 32, _lib.DG_KIND_FP8_FP4: 32}.get(kind, 16)) * \
        {_lib.DG_KIND_BF16: 8, _lib.DG_KIND_FP4_FP4: 32, _lib.DG_KIND_FP8_FP4: 32}.get(kind, 16)
    args.kind, args.gemm_type, args.m, args.n, args.k, args.num_groups = kind, gemm_type, m, n, k, num_groups
    # leading dimensions in storage elements (packed FP4: two per byte)
    args.lda = k // 2 if kind == _lib.DG_KIND_FP4_FP4 else k
    args.ldb = k // 2 if kind in (_lib.DG_KIND_FP4_FP4, _lib.DG_KIND_FP8_FP4) else k
    args.ldd = n
    args.batch_stride_a, args.batch_stride_b = m * args.lda, n * args.ldb
    args.batch_stride_d = m * n
    nk64 = (k + 63) // 64
    args.sfa_ld, args.sfb_ld = (m + 1) // 2 * 2, (n + 1) // 2 * 2
    args.sfa_batch_stride, args.sfb_batch_stride = args.sfa_ld * nk64, args.sfb_ld * nk64
    args.alignment = get_mk_alignment_for_contiguous_layout()
    args.num_cus = get_num_sms()
    # (dense and batched calls may split K into the library's per-stream workspace)
    args.library_workspace = 1 if gemm_type in (_lib.DG_GEMM_NORMAL, _lib.DG_GEMM_BATCHED) else 0
    args.split_k = split_k
    forced = os.environ.get('DG_FORCE_BLOCK')   # the tuning override the calls honour
    if forced:
        args.block_m, args.block_n = (int(x) for x in forced.split('x'))
    info = _lib.LaunchInfo()
    lib = _lib.load()
    _lib.check(lib.dg_launch_plan(args, ctypes.byref(info)), lib)
    return {f: getattr(info, f) for f, _ in _lib.LaunchInfo._fields_}
