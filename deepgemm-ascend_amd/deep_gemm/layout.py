"""Scale-factor layout contract (the reference's csrc/apis/layout.hpp:37-140).

``transform_sf_into_required_layout`` returns the packed UE8M0x2 int16, MN-major SF the
GEMM kernels consume, launching the HIP ``transform_sf`` kernel when the input is not
already in that layout.  Extension over the reference: fp32 SF with ``gran_k == 128``
(the DeepSeek-V3 1x128 / 128x128 recipe) is accepted and expanded to per-32 exponents.
"""
import os
from typing import Optional, Tuple

import torch

from . import _lib
from .runtime import get_mk_alignment_for_contiguous_layout


def _ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


def _assert(cond: bool, msg: str = 'Assertion error') -> None:
    if not cond:
        raise RuntimeError(msg)


def _split_recipe(recipe, is_sfa: Optional[bool]) -> Tuple[int, int]:
    if len(recipe) == 2:
        return int(recipe[0]), int(recipe[1])
    _assert(len(recipe) == 3, 'recipe must be (gran_m, gran_n, gran_k) or (gran_mn, gran_k)')
    _assert(is_sfa is not None, 'is_sfa must be set for a 3-element recipe')
    return (int(recipe[0]) if is_sfa else int(recipe[1])), int(recipe[2])


def _align(x: int, a: int) -> int:
    return (x + a - 1) // a * a


def check_sf_layout(sf: torch.Tensor, mn: int, k: int, gran_mn: int, gran_k: int,
                    num_groups: Optional[int]) -> bool:
    """Validate ``sf``; True when it is already in the required layout (csrc/apis/layout.hpp:37-65)."""
    dt = sf.dtype
    _assert(dt in (torch.float32, torch.int16), 'SF must be float32 or int16 (packed ue8m0x2)')
    st, sz = sf.stride(), sf.shape
    _assert(len(sz) == (1 if num_groups is not None else 0) + 2, 'SF rank mismatch')
    _assert(st[-1] == 1 or st[-2] == 1, 'SF input must be contiguous in either the last or second-to-last dimension')
    if num_groups is not None:
        _assert(sz[-3] == num_groups, 'SF group count mismatch')
    if dt == torch.float32:
        _assert(gran_k in (32, 128), 'gran_k must be 32 (or 128 for float32 SF)')
        div_k = gran_k
    else:
        _assert(gran_k == 32, 'gran_k must be 32')
        div_k = 64
    _assert(sz[-2] == _ceil_div(mn, gran_mn), f'SF MN extent {sz[-2]} != ceil({mn}/{gran_mn})')
    _assert(sz[-1] == _ceil_div(k, div_k), f'SF K extent {sz[-1]} != ceil({k}/{div_k})')
    if dt == torch.int16 and gran_mn == 1 and st[-2] == 1 and st[-1] == _align(sz[-2], 2):
        if num_groups is not None:
            return st[-3] == st[-1] * sz[-1]
        return True
    return False


def _launch_transform_sf(sf: torch.Tensor, mn: int, k: int, gran_mn: int, gran_k: int,
                         psum: Optional[torch.Tensor], m_indices: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The reference's launch_transform_sf (csrc/jit_kernels/transform_sf.hpp:15-105)."""
    squeeze = sf.dim() == 2
    if squeeze:
        sf = sf.unsqueeze(0)
    _assert(1 <= gran_mn <= 128 and (gran_mn & (gran_mn - 1)) == 0,
            'gran_mn only support a power of two in [1, 128]')
    _assert(sf.is_cuda, 'SF must be a device tensor')
    num_batches, sf_mn, sf_k = sf.shape
    num_groups, alignment = 0, get_mk_alignment_for_contiguous_layout()
    if psum is not None:
        _assert(num_batches == 1, 'Grouped transform SF requires one logical batch and grouped_layout')
        _assert(psum.device == sf.device, 'grouped_layout must be on the same device as the SF input')
        _assert(psum.dtype == torch.int32 and psum.dim() == 1 and psum.is_contiguous(),
                'grouped_layout must be a contiguous 1D int32 tensor')
        num_groups = psum.numel()
        _assert(num_groups > 0, 'grouped_layout must contain at least one group')
    rows_layout = psum
    if m_indices is not None and psum is None and num_batches == 1 and gran_mn == 1:
        # padding rows (negative m_indices) are neither read nor validated
        rows_layout, num_groups = m_indices, -1
    k64 = _ceil_div(k, 64)
    # MN axis padded to an even leading dimension (the GEMM kernels fetch SF rows in pairs)
    ld = _align(mn, 2)
    out = torch.empty((num_batches, k64, ld), dtype=torch.int16, device=sf.device)[:, :, :mn].transpose(-2, -1)
    if out.numel() == 0 or get_dry_run_safe():
        return out.squeeze(0) if squeeze else out
    check_err = os.environ.get('DG_CHECK_SF', '0') == '1' and sf.dtype == torch.float32
    err = torch.zeros(1, dtype=torch.int32, device=sf.device) if check_err else None
    lib = _lib.load()
    rc = lib.dg_transform_sf(
        sf.data_ptr(), _lib.DG_SF_F32 if sf.dtype == torch.float32 else _lib.DG_SF_I16,
        sf.stride(0), sf.stride(1), sf.stride(2), num_batches, sf_mn, sf_k, mn, k, gran_mn, gran_k,
        rows_layout.data_ptr() if rows_layout is not None else None, num_groups, alignment,
        out.data_ptr(), k64 * ld, err.data_ptr() if err is not None else None,
        torch.cuda.current_stream(sf.device).cuda_stream)
    _lib.check(rc, lib)
    if err is not None and int(err.item()) != 0:
        raise RuntimeError('Invalid float32 SF: only the 8-bit exponent may be set (sign and mantissa must be 0)')
    return out.squeeze(0) if squeeze else out


def get_dry_run_safe() -> bool:
    from .runtime import get_dry_run
    return get_dry_run()


def transform_sf_into_required_layout(sf: torch.Tensor, mn: int, k: int, recipe,
                                      num_groups: Optional[int] = None,
                                      is_sfa: Optional[bool] = None,
                                      disable_ue8m0_cast: bool = False,
                                      psum_layout: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Same contract as the reference (csrc/apis/layout.hpp:68-92, bound at :131-137)."""
    return transform_sf_rows(sf, mn, k, recipe, num_groups, is_sfa, disable_ue8m0_cast, psum_layout)


def transform_sf_rows(sf, mn, k, recipe, num_groups, is_sfa, disable_ue8m0_cast, psum_layout=None, m_indices=None):
    """transform_sf_into_required_layout, plus an m_indices layout of an M-grouped A (its padding
    rows, negative indices, are neither read nor validated)."""
    _assert(is_sfa is not None, 'is_sfa must be set')
    gran_mn, gran_k = _split_recipe(recipe, is_sfa)
    if check_sf_layout(sf, mn, k, gran_mn, gran_k, num_groups):
        return sf
    if sf.dtype == torch.float32:
        _assert(not disable_ue8m0_cast,
                'Float32 SF must be converted into ue8m0, but disable_ue8m0_cast is set true')
    return _launch_transform_sf(sf, mn, k, gran_mn, gran_k, psum_layout, m_indices)


def transform_k_grouped_sf_into_required_layout(sf: torch.Tensor, mn: int, k: int, recipe, is_sfa: Optional[bool],
                                                psum_layout: torch.Tensor) -> torch.Tensor:
    """Same contract as the reference (csrc/apis/layout.hpp:94-111): ``sf`` is [ceil(MN/gran_mn),
    ceil(Ktot/gran_k)] (fp32) or [.., ceil(Ktot/64)] (packed int16) over the K axis that ``psum_layout``
    splits into groups; the SF of the K padding between groups becomes 0 in the output."""
    _assert(is_sfa is not None, 'is_sfa must be set')
    gran_mn, gran_k = _split_recipe(recipe, is_sfa)
    if check_sf_layout(sf, mn, k, gran_mn, gran_k, None):
        return sf
    _assert(1 <= gran_mn <= 128 and (gran_mn & (gran_mn - 1)) == 0,
            'gran_mn only support a power of two in [1, 128]')
    _assert(sf.is_cuda, 'SF must be a device tensor')
    _assert(psum_layout.device == sf.device, 'grouped_layout must be on the same device as the SF input')
    _assert(psum_layout.dtype == torch.int32 and psum_layout.dim() == 1 and psum_layout.is_contiguous(),
            'grouped_layout must be a contiguous 1D int32 tensor')
    num_groups = psum_layout.numel()
    _assert(num_groups > 0, 'grouped_layout must contain at least one group')
    alignment = get_mk_alignment_for_contiguous_layout()
    sf_mn, sf_k = sf.shape
    k64, ld = _ceil_div(k, 64), _align(mn, 2)
    out = torch.empty((k64, ld), dtype=torch.int16, device=sf.device)[:, :mn].transpose(0, 1)
    if out.numel() == 0 or get_dry_run_safe():
        return out
    check_err = os.environ.get('DG_CHECK_SF', '0') == '1' and sf.dtype == torch.float32
    err = torch.zeros(1, dtype=torch.int32, device=sf.device) if check_err else None
    lib = _lib.load()
    rc = lib.dg_transform_k_grouped_sf(
        sf.data_ptr(), _lib.DG_SF_F32 if sf.dtype == torch.float32 else _lib.DG_SF_I16,
        sf.stride(0), sf.stride(1), sf_mn, sf_k, mn, k, gran_mn, gran_k,
        psum_layout.data_ptr(), num_groups, alignment, out.data_ptr(),
        err.data_ptr() if err is not None else None, torch.cuda.current_stream(sf.device).cuda_stream)
    _lib.check(rc, lib)
    if err is not None and int(err.item()) != 0:
        raise RuntimeError('Invalid float32 SF: only the 8-bit exponent may be set (sign and mantissa must be 0)')
    return out


def operand_recipes(recipe=None, recipe_a=None, recipe_b=None):
    """((gran_m, gran_k_a), (gran_n, gran_k_b)) for the two operands.

    Same rules as ``get_recipe``, except that A and B may use different K granularities when
    both are MX-compatible (32 or 128): each is expanded to per-32 exponents, so a 1x128
    activation recipe pairs with a 1x32 FP4 weight recipe."""
    if recipe is None and recipe_a is not None and recipe_b is not None and recipe_a[1] != recipe_b[1]:
        _assert(recipe_a[1] in (32, 128) and recipe_b[1] in (32, 128),
                'gran_k of recipe_a and recipe_b must be the same')
        return (int(recipe_a[0]), int(recipe_a[1])), (int(recipe_b[0]), int(recipe_b[1]))
    gm, gn, gk = get_recipe(recipe, recipe_a, recipe_b)
    return (gm, gk), (gn, gk)


def get_recipe(recipe=None, recipe_a=None, recipe_b=None) -> Tuple[int, int, int]:
    """csrc/apis/layout.hpp:113-128."""
    _assert(not (recipe is not None and (recipe_a is not None or recipe_b is not None)))
    if recipe is not None:
        return tuple(int(x) for x in recipe)
    gran_m, gran_k_a = recipe_a if recipe_a is not None else (1, 32)
    gran_n, gran_k_b = recipe_b if recipe_b is not None else (1, 32)
    _assert(gran_k_a == gran_k_b, 'gran_k of recipe_a and recipe_b must be the same')
    return int(gran_m), int(gran_n), int(gran_k_a)
