"""GEMM oracle (test infrastructure only; see ``oracle/__init__.py``).

The reference's own reference path: dequantise each operand per block to fp32 (codes x
2^(e-127)), multiply in fp32, apply alpha / bias / accumulate, cast to the output dtype
(``tests/generators.py:320-322``; grouped ``:351-353``).  ``calc_diff`` is
``tests/utils.py:36-43``.

* ``dequant_operand`` works from the kernel-side inputs (codes plus the packed MN-major
  int16 SF that ``transform_sf_into_required_layout`` returns), so it checks exactly what
  the GPU path consumes.
* ``gemm_nt``                 -- D = alpha * A @ B^T (+ bias | + C), fp32 math.
* ``m_grouped_contiguous``   -- psum layout (group g rows [align(psum[g-1]), psum[g]) use
  B[g], padding rows are 0) or m_indices layout (row r uses B[idx[r]], -1 rows are 0).
* ``batched_nt``              -- D[i] = A[i] @ B[i]^T (+ C[i]) per batch (tests/generators.py:392-419).
* ``k_grouped_tn``            -- D[g] = A[Kg]^T @ B[Kg] (+ C[g]) over the K ranges
  Kg = [align(psum[g-1]), psum[g]) of A [Ktot, M] / B [Ktot, N]; an empty group gives 0 (+ C)
  (tests/generators.py:361-390).
* ``einsum_ref``              -- the three fixed expressions of csrc/apis/einsum.hpp:99-199 as
  torch.einsum in fp32 (a library routine, independent of the permutations the API uses).
* ``m_grouped_masked``        -- D[g, :masked_m[g]] = A[g, :masked_m[g]] @ B[g]^T; the rest
  is not compared (upstream DeepGEMM semantics; the reference has no masked kernel, so
  this function is "parity unpinned" with respect to the reference and pinned only by the
  closed form checks in tests/test_oracle.py).

Pinned by tests/test_oracle.py: fp64 brute-force triple loops on tiny shapes, identity /
permutation / linearity properties, and calc_diff closed forms.
"""
import torch

from . import quant
from .layout import psum_slices, unpack_sf_bytes, sf_bytes_to_fp32


def calc_diff(x: torch.Tensor, y: torch.Tensor) -> float:
    """1 - 2<x,y> / (|x|^2 + |y|^2), in float64 (tests/utils.py:36-43)."""
    x, y = x.double(), y.double()
    den = (x * x + y * y).sum()
    if den == 0:
        return 0.0
    return float(1 - 2 * (x * y).sum() / den)


def dequant_operand(data: torch.Tensor, packed_sf: torch.Tensor, k: int) -> torch.Tensor:
    """fp32 [..., MN, K] from K-major codes and packed int16 SF [..., MN, ceil(K/64)].

    ``data`` is logically [..., MN, K] (e4m3) or [..., MN, K/2] (packed fp4 int8, K the
    contiguous axis)."""
    vals = quant.decode(data, -1)
    assert vals.size(-1) == k
    ex = unpack_sf_bytes(packed_sf, k)                    # [..., MN, ceil(K/32)]
    scale = sf_bytes_to_fp32(ex).repeat_interleave(32, dim=-1)[..., :k]
    return vals * scale


def gemm_nt(a: torch.Tensor, b: torch.Tensor, out_dtype=torch.bfloat16, alpha=None,
            bias=None, c=None) -> torch.Tensor:
    """a [M,K] fp32, b [N,K] fp32 -> (alpha * a @ b.T + bias/c).to(out_dtype)."""
    d = a.float() @ b.float().T
    if alpha is not None:
        d = alpha * d
    if bias is not None:
        d = d + bias.float()
    if c is not None:
        d = d + c.float()
    return d.to(out_dtype)


def m_grouped_contiguous(a: torch.Tensor, b: torch.Tensor, layout: torch.Tensor,
                         use_psum_layout: bool = True, alignment: int = 256,
                         out_dtype=torch.bfloat16) -> torch.Tensor:
    """a [M,K] fp32, b [G,N,K] fp32."""
    m = a.size(0)
    d = torch.zeros(m, b.size(1), dtype=torch.float32)
    if use_psum_layout:
        for g, sl in enumerate(psum_slices(layout.tolist(), alignment)):
            if sl.stop > sl.start:
                d[sl] = a[sl] @ b[g].T
    else:
        idx = layout.long()
        for g in range(b.size(0)):
            rows = (idx == g).nonzero().flatten()
            if rows.numel():
                d[rows] = a[rows] @ b[g].T
    return d.to(out_dtype)


def m_grouped_masked(a: torch.Tensor, b: torch.Tensor, masked_m: torch.Tensor,
                     out_dtype=torch.bfloat16) -> torch.Tensor:
    """a [G,Mmax,K] fp32, b [G,N,K] fp32; rows >= masked_m[g] are returned as 0."""
    g_, mmax, _ = a.shape
    d = torch.zeros(g_, mmax, b.size(1), dtype=torch.float32)
    for g in range(g_):
        mg = int(masked_m[g])
        if mg:
            d[g, :mg] = a[g, :mg] @ b[g].T
    return d.to(out_dtype)


def brute_force_nt(a, b):
    """fp64 triple loop, tiny shapes only."""
    m, k = a.shape
    n = b.shape[0]
    out = torch.zeros(m, n, dtype=torch.float64)
    for i in range(m):
        for j in range(n):
            s = 0.0
            for t in range(k):
                s += float(a[i, t]) * float(b[j, t])
            out[i, j] = s
    return out


def batched_nt(a: torch.Tensor, b: torch.Tensor, c=None, out_dtype=torch.bfloat16) -> torch.Tensor:
    """a [B,M,K] fp32, b [B,N,K] fp32 -> [B,M,N] (tests/generators.py:392-419)."""
    d = torch.stack([a[i].float() @ b[i].float().T for i in range(a.size(0))]) if a.size(0) else \
        torch.zeros(0, a.size(1), b.size(1))
    if c is not None:
        d = d + c.float()
    return d.to(out_dtype)


def k_grouped_tn(a: torch.Tensor, b: torch.Tensor, psum, alignment: int = 256, c=None,
                 out_dtype=torch.bfloat16) -> torch.Tensor:
    """a [Ktot,M] fp32, b [Ktot,N] fp32, psum list of G K-ends -> [G,M,N] (tests/generators.py:361-390)."""
    g_ = len(psum)
    d = torch.zeros(g_, a.size(1), b.size(1), dtype=torch.float32)
    for g, sl in enumerate(psum_slices(list(psum), alignment)):
        if sl.stop > sl.start:
            d[g] = a[sl].float().T @ b[sl].float()
    if c is not None:
        d = d + c.float()
    return d.to(out_dtype)


EINSUM_EXPRS = ('bhr,hdr->bhd', 'bhd,hdr->bhr', 'bhd,bhr->hdr')


def einsum_ref(expr: str, a: torch.Tensor, b: torch.Tensor, c=None, out_dtype=torch.bfloat16) -> torch.Tensor:
    assert expr in EINSUM_EXPRS
    d = torch.einsum(expr, a.double(), b.double())
    if c is not None:
        d = d + c.double()
    return d.to(out_dtype)
