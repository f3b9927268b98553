"""Output-epilogue oracle (test infrastructure only; see ``oracle/__init__.py``).

* ``stochastic_round_bf16`` -- the reference's stochastic bf16 rounding check
  (``tests/utils.py:70-92``): per row, quartets of four consecutive fp32 outputs (zeros past
  the row's end) hash with their quartet index into 4 x 16 random bits; a value rounds up
  (truncated bf16 + 1) when its discarded low 16 bits exceed 0xffff minus its random bits;
  NaN becomes 0x7fc0.
* ``quantize_fp8_output``   -- the FP8 output check of ``tests/test_einsum.py:70-86``: the bf16
  D of a batched GEMM, stored as [M, B*N], quantised per (row, 32 columns) by
  ``quant.quantize_blockwise`` (``tests/generators.py:61-95``), the UE8M0 bytes packed in
  pairs into int16 (lower byte = even 32-column block), M-major [M, B*N/64].

Pinned by tests/test_oracle.py: a scalar Python-int evaluation of the hash on hand-picked
quartets, the up/down property (every output is the truncation or one ulp above it), exact
bf16 inputs passing through unchanged, NaN canonicalisation, the mean of many roundings
against the fp32 mean (unbiasedness), and the FP8 packing against a per-block loop.
"""
import numpy as np
import torch

from . import quant


def _u32(x):
    return np.uint32(x)


def stochastic_round_bf16(x: torch.Tensor) -> torch.Tensor:
    """fp32 [..., N] -> bf16 [..., N] (tests/utils.py:70-92)."""
    values = x.detach().cpu().float().contiguous().numpy().view(np.uint32)
    n = values.shape[-1]
    values = np.pad(values, [(0, 0)] * (values.ndim - 1) + [(0, -n % 4)])
    values = values.reshape(*values.shape[:-1], -1, 4)
    with np.errstate(over='ignore'):
        h = (values[..., 0] * _u32(0x5671d42b) + values[..., 1] * _u32(0x9995e499) +
             values[..., 2] * _u32(0xace1b8a5) + values[..., 3] * _u32(0xe153538d) +
             np.arange(values.shape[-2], dtype=np.uint32))
        h = (h ^ (h >> _u32(23))) * _u32(0x7feb352d)
        h ^= h >> _u32(16)
        h1, h2 = h * _u32(0x846ca68b), h * _u32(0xd35a2d97)
    h1 ^= h1 >> _u32(11)
    h2 ^= h2 >> _u32(11)
    rnd = np.stack((h1 & _u32(0xffff), h1 >> _u32(16), h2 & _u32(0xffff), h2 >> _u32(16)), axis=-1)
    rounded = (values >> _u32(16)) + ((values & _u32(0xffff)) > (_u32(0xffff) - rnd)).astype(np.uint32)
    rounded = np.where((values & _u32(0x7fffffff)) > _u32(0x7f800000), _u32(0x7fc0), rounded).astype(np.uint16)
    out = rounded.reshape(*rounded.shape[:-2], -1)[..., :n].copy()
    return torch.from_numpy(out.view(np.int16)).view(torch.bfloat16)


def quantize_fp8_output(d_rows: torch.Tensor):
    """bf16/fp32 [M, C] (C = B*N, a multiple of 64) -> (e4m3 [M, C], int16 SFD [M, C/64] M-major)."""
    data, sf, _ = quant.quantize_blockwise(d_rows.float(), (1, 32), 'e4m3')
    ex = ((sf.view(torch.int32) >> 23) & 0xff).to(torch.int32).reshape(d_rows.size(0), -1, 2)
    sfd = (ex[..., 0] + ex[..., 1] * 256).to(torch.int32)
    sfd = torch.where(sfd >= 32768, sfd - 65536, sfd).to(torch.int16)
    return data, sfd.t().contiguous().t()
