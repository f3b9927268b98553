"""Batched GEMMs and the fixed einsum contractions (the reference's csrc/apis/einsum.hpp).

``fp8_bmm`` / ``bf16_bmm`` run the batched mode of the same HIP GEMM kernel (one B[i] per batch,
per-batch operand / SF / D offsets); ``einsum`` / ``fp8_einsum`` permute their operands (views
only) and dispatch to them, exactly as the reference does (einsum.hpp:99-222).
"""
from typing import Optional, Tuple

import torch

from .gemm import _batched
from .layout import _assert


def fp8_bmm(a: Tuple[torch.Tensor, torch.Tensor], b: Tuple[torch.Tensor, torch.Tensor], d, c: Optional[torch.Tensor] = None,
            recipe=(1, 1, 32), compiled_dims: str = 'nk', epilogue=None) -> None:
    """Batched FP8 GEMM D[i] = A[i] @ B[i]^T (+ C[i]) (csrc/apis/einsum.hpp:22-71).
    A [B, M, K] e4m3, B [B, N, K] e4m3, SFs fp32 or packed int16 in any major; D [B, M, N] bf16 /
    fp32, or an (e4m3 D, SFD) pair / FP8Quantization(sfd) with SFD int16 [M, B * N / 64], M-major."""
    (a_, sfa), (b_, sfb) = a, b
    _batched(a_, sfa, b_, sfb, d, c, recipe, False, epilogue, dims=compiled_dims)


def bf16_bmm(a: torch.Tensor, b: torch.Tensor, d: torch.Tensor, c: Optional[torch.Tensor] = None,
             compiled_dims: str = 'nk', epilogue=None) -> None:
    """Batched bf16 GEMM D[i] = A[i] @ B[i]^T (+ C[i]) (csrc/apis/einsum.hpp:73-97)."""
    _assert(d.dtype in (torch.float32, torch.bfloat16))
    _batched(a, None, b, None, d, c, None, True, epilogue, dims=compiled_dims)


def _perm(t: Optional[torch.Tensor], p):
    return t.permute(*p) if t is not None else None


def einsum(expr: str, a: torch.Tensor, b: torch.Tensor, d: torch.Tensor, c: Optional[torch.Tensor] = None,
           use_cublaslt: bool = False, epilogue=None) -> None:
    """bf16 einsum over the reference's fixed expressions (csrc/apis/einsum.hpp:99-136)."""
    if use_cublaslt:
        raise RuntimeError('einsum: use_cublaslt will call ascend einsum kernel, but is not implemented in current version')
    if expr == 'bhr,hdr->bhd':
        bf16_bmm(a.permute(1, 0, 2), b, d.permute(1, 0, 2), _perm(c, (1, 0, 2)), 'nk', epilogue)
    elif expr == 'bhd,hdr->bhr':
        bf16_bmm(a.permute(1, 0, 2), b.permute(0, 2, 1), d.permute(1, 0, 2), _perm(c, (1, 0, 2)), 'nk', epilogue)
    elif expr == 'bhd,bhr->hdr':
        bf16_bmm(a.permute(1, 2, 0), b.permute(1, 2, 0), d, c, 'mn', epilogue)
    else:
        raise RuntimeError('Unsupported einsum expression')


def fp8_einsum(expr: str, a: Tuple[torch.Tensor, torch.Tensor], b: Tuple[torch.Tensor, torch.Tensor], d,
               c: Optional[torch.Tensor] = None, recipe=(1, 1, 32), epilogue=None) -> None:
    """FP8 einsum over the reference's fixed expressions (csrc/apis/einsum.hpp:138-199); the SFs are
    permuted with their operands."""
    (a_, sfa), (b_, sfb) = a, b
    if expr == 'bhr,hdr->bhd':
        # A=[b,h,r] B=[h,d,r] D=[b,h,d] -> (B,M,N,K) = (h,b,d,r); the output SF of an FP8 D stays as given
        perm_d = (d[0].permute(1, 0, 2), d[1]) if isinstance(d, tuple) else d.permute(1, 0, 2)
        fp8_bmm((a_.permute(1, 0, 2), sfa.permute(1, 0, 2)), (b_, sfb), perm_d, _perm(c, (1, 0, 2)),
                recipe, 'nk', epilogue)
    elif expr == 'bhd,hdr->bhr':
        # A=[b,h,d] B=[h,d,r] D=[b,h,r] -> (h,b,r,d)
        _assert(not isinstance(d, tuple))
        fp8_bmm((a_.permute(1, 0, 2), sfa.permute(1, 0, 2)), (b_.permute(0, 2, 1), sfb.permute(0, 2, 1)),
                d.permute(1, 0, 2), _perm(c, (1, 0, 2)), recipe, 'nk', epilogue)
    elif expr == 'bhd,bhr->hdr':
        # A=[b,h,d] B=[b,h,r] D=[h,d,r] -> (h,d,r,b): batch h, contraction over b
        _assert(not isinstance(d, tuple))
        fp8_bmm((a_.permute(1, 2, 0), sfa.permute(1, 2, 0)), (b_.permute(1, 2, 0), sfb.permute(1, 2, 0)),
                d, c, recipe, 'mn', epilogue)
    else:
        raise RuntimeError('Unsupported einsum expression')
