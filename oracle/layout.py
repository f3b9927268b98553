"""Scale-factor layout oracle (test infrastructure only; see ``oracle/__init__.py``).

* ``transform_sf``      -- the closed form ``reference()`` of ``tests/test_layout.py:39-50``:
  fp32 SF -> exponent byte (bits 23..30), two K-adjacent bytes packed per int16 (even index
  in the low byte), MN-major ``[..., MN, ceil(K/64)]`` with stride(-2) == 1, each SF row
  repeated ``gran_mn`` times and cropped to MN.  M-grouped psum padding rows are zeroed
  (``tests/test_layout.py:93-95``, ``deep_gemm/include/deep_gemm/transform_sf.hpp:586-593``).
  Extension: ``gran_k == 128`` fp32 input is first expanded to four identical per-32 scales.
* ``transform_k_grouped_sf`` -- the same layout over a K axis split by a psum layout; the SF of
  the K padding between groups (columns ``psum_pad_slices(psum, alignment, w)`` with w = gran_k
  for fp32 and 64 for packed int16) becomes 0 (``tests/test_layout.py:96-98``).
* ``psum_*`` / ``m_indices_*`` -- ``tests/generators.py:212-235`` (psum layout walk) and the
  m_indices convention (one int32 per row, -1 on padding rows).

Pinned by tests/test_oracle.py: hand-computed known answers, the int16 byte order against
numpy's little-endian view, brute-force per-element definitions and psum<->m_indices
round trips.
"""
import torch

from .quant import align, ceil_div


def sf_exponent_bytes(sf: torch.Tensor) -> torch.Tensor:
    """UE8M0 byte of each fp32 power-of-two scale."""
    return ((sf.contiguous().view(torch.int32) >> 23) & 0xff).to(torch.uint8)


def sf_is_valid(sf: torch.Tensor) -> bool:
    bits = sf.contiguous().view(torch.int32)
    return bool(((bits & 0x807fffff) == 0).all())


def psum_slices(psum, alignment: int):
    """Valid row span of each group: [align(psum[g-1]), psum[g]) (tests/generators.py:224-228)."""
    last = 0
    for p in psum:
        yield slice(last, p)
        last = align(p, alignment)


def psum_pad_slices(psum, alignment: int, gran: int = 1):
    """Padding span of each group in units of ``gran`` rows (tests/generators.py:231-235)."""
    for p in psum:
        s0 = ceil_div(p, gran)
        s1 = align(p, alignment) // gran
        if s0 < s1:
            yield slice(s0, s1)


def psum_from_sizes(sizes, alignment: int):
    """(total_rows, psum list) for per-group row counts (tests/generators.py:212-221)."""
    psum, acc = [], 0
    for s in sizes:
        psum.append(acc + s)
        acc = align(acc + s, alignment)
    return acc, psum


def m_indices_from_psum(psum, alignment: int, total_rows: int):
    """Per-row group index (-1 on padding rows) equivalent to a psum layout."""
    idx = torch.full((total_rows,), -1, dtype=torch.int32)
    for g, sl in enumerate(psum_slices(psum, alignment)):
        idx[sl] = g
    return idx


def transform_sf(sf: torch.Tensor, mn: int, k: int, gran_mn: int, gran_k: int = 32,
                 psum=None, alignment: int = 256) -> torch.Tensor:
    """Packed-int16 MN-major SF exactly as ``transform_sf_into_required_layout`` returns it."""
    assert sf.dtype in (torch.float32, torch.int16)
    sf = sf.clone()
    if psum is not None:
        # padding rows of an M-grouped SFA become zero (in source-row units)
        for span in psum_pad_slices(psum, alignment, gran_mn):
            sf[..., span, :] = 0
    if sf.dtype == torch.float32:
        assert gran_k in (32, 128)
        if gran_k == 128:
            sf = sf.repeat_interleave(4, dim=-1)[..., :ceil_div(k, 32)]
        assert sf.size(-1) == ceil_div(k, 32)
        ex = sf_exponent_bytes(sf)
        if ex.size(-1) % 2:
            ex = torch.nn.functional.pad(ex, (0, 1))
        packed = ex.contiguous().view(torch.int16)
    else:
        assert gran_k == 32 and sf.size(-1) == ceil_div(k, 64)
        packed = sf
    out = packed.transpose(-2, -1).repeat_interleave(gran_mn, -1)[..., :mn]
    return out.contiguous().transpose(-2, -1)


def transform_k_grouped_sf(sf: torch.Tensor, mn: int, k: int, gran_mn: int, psum, gran_k: int = 32,
                           alignment: int = 256) -> torch.Tensor:
    """``transform_k_grouped_sf_into_required_layout`` of an [ceil(MN/gran_mn), ceil(K/w)] SF."""
    sf = sf.clone()
    w = gran_k if sf.dtype == torch.float32 else 64
    for span in psum_pad_slices(psum, alignment, w):
        sf[..., span] = 0
    return transform_sf(sf, mn, k, gran_mn, gran_k)


def unpack_sf_bytes(packed: torch.Tensor, k: int) -> torch.Tensor:
    """[..., MN, ceil(K/64)] packed int16 -> [..., MN, ceil(K/32)] uint8 exponents."""
    b = packed.contiguous().view(torch.uint8)
    return b[..., :ceil_div(k, 32)]


def sf_bytes_to_fp32(ex: torch.Tensor) -> torch.Tensor:
    """UE8M0 byte -> fp32 2^(e-127) (byte 0 -> 2^-127, a denormal, exactly as the MFMA scale)."""
    e = ex.to(torch.float64) - 127.0
    return torch.pow(torch.tensor(2.0, dtype=torch.float64), e).to(torch.float32)
