"""Seeded operand generators for the tests (CPU-side; data is copied to the GPU).

Follows the reference's tests/generators.py: random e4m3 / e2m1 codes with power-of-two
scales (``generate_random_quantized_with_major``, :124-166) or N(0,1) data quantised with
UE8M0 block scales from blockwise absmax (``quantize_with_major``, :61-95).
"""
import torch

from oracle import quant, layout, gemm as ogemm


def gen(seed: int = 0) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def operand(rows: int, k: int, quant_kind: str, gran, g: torch.Generator, mode: str = 'codes',
            batch: int = 0):
    """(data [.., rows, K(-storage)] K-major, sf fp32 [.., ceil(rows/gm), ceil(K/gk)], dequant fp32)."""
    shape = (batch, rows, k) if batch else (rows, k)
    gran_full = ((1,) if batch else ()) + tuple(gran)
    if mode == 'codes':
        return quant.random_codes(shape, quant_kind, -1, g, gran_full)
    x = torch.randn(shape, generator=g)
    return quant.quantize_blockwise(x, gran_full, quant_kind, -1)


def to_dev(*ts):
    return tuple(t.cuda() if isinstance(t, torch.Tensor) else t for t in ts)


def packed_sf(sf: torch.Tensor, mn: int, k: int, gran_mn: int, gran_k: int, psum=None, alignment=256):
    return layout.transform_sf(sf, mn, k, gran_mn, gran_k, psum=psum, alignment=alignment)


calc_diff = ogemm.calc_diff
