"""Quantisation oracle (test infrastructure only; see ``oracle/__init__.py``).

Restates the reference's data generators:

* ``ceil_to_ue8m0``           -- ``tests/generators.py:27-31``
* ``quantize_fp4_codes``      -- ``tests/generators.py:34-50`` (boundaries 0.25 ... 5.0)
* ``quantize_blockwise``      -- ``tests/generators.py:61-95`` (absmax / 448 or / 6, UE8M0 ceil)
* ``FP4_VALUES`` / decode     -- ``tests/generators.py:98-102``
* e4m3 decode                 -- OCP E4M3FN (``torch.float8_e4m3fn``), ``tests/generators.py:53-58``

Pinned by tests/test_oracle.py: every e4m3 code against torch's own float8 decode and an
independent bit-field formula; every fp4 code against the e2m1 bit-field formula and the
rounding boundaries; ``ceil_to_ue8m0`` against ``math.frexp`` on random and edge values.
"""
import math
import numpy as np
import torch

FP4_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


def align(a: int, b: int) -> int:
    return ceil_div(a, b) * b


def ceil_to_ue8m0(x: torch.Tensor) -> torch.Tensor:
    """Smallest power of two >= |x|, exponent clamped to [1, 254] (tests/generators.py:27-31)."""
    bits = x.abs().float().contiguous().view(torch.int32)
    exp = ((bits >> 23) & 0xff) + ((bits & 0x7fffff) != 0).to(torch.int32)
    return (exp.clamp(1, 254) << 23).view(torch.float32)


def e4m3_decode_table() -> np.ndarray:
    """fp32 value of each of the 256 OCP e4m3 codes (NaN for 0x7f / 0xff)."""
    out = np.empty(256, dtype=np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xf
        m = c & 7
        if e == 0xf and m == 7:
            out[c] = np.nan
        elif e == 0:
            out[c] = s * (m / 8.0) * 2.0 ** -6
        else:
            out[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


def fp4_decode_table() -> np.ndarray:
    return np.array(FP4_VALUES, dtype=np.float32)


def quantize_fp4_codes(x: torch.Tensor) -> torch.Tensor:
    """Round-to-nearest e2m1 code (uint8 nibble, sign in bit 3) (tests/generators.py:34-50)."""
    ax = x.abs()
    code = torch.zeros_like(x, dtype=torch.uint8)
    for boundary in (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0):
        code += (ax > boundary).to(torch.uint8)
    sign = (x < 0) & (code != 0)
    return code | (sign.to(torch.uint8) << 3)


def pack_fp4(codes: torch.Tensor, major_dim: int) -> torch.Tensor:
    """Pack nibbles two per byte along ``major_dim``; the even element is the low nibble
    (tests/generators.py:46-49).  Returns an int8 tensor whose ``major_dim`` has half the extent
    and is the contiguous axis."""
    c = codes.transpose(major_dim, -1).contiguous()
    packed = (c[..., ::2] & 0x0f) | ((c[..., 1::2] & 0x0f) << 4)
    return packed.view(torch.int8).transpose(major_dim, -1)


def unpack_fp4(packed: torch.Tensor, major_dim: int) -> torch.Tensor:
    """Inverse of ``pack_fp4``: float32 values, ``major_dim`` doubled."""
    p = packed.transpose(major_dim, -1).contiguous().view(torch.uint8)
    lut = torch.tensor(FP4_VALUES, dtype=torch.float32)
    lo = lut[(p & 0x0f).long()]
    hi = lut[(p >> 4).long()]
    out = torch.stack((lo, hi), dim=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)
    return out.transpose(major_dim, -1)


def decode(data: torch.Tensor, major_dim: int = -1) -> torch.Tensor:
    """fp32 value of quantised codes (e4m3 tensors or packed-fp4 int8 tensors)."""
    if data.dtype == torch.float8_e4m3fn:
        lut = torch.from_numpy(e4m3_decode_table())
        return lut[data.contiguous().view(torch.uint8).long()].reshape(data.shape)
    if data.dtype == torch.int8:
        return unpack_fp4(data, major_dim % data.dim())
    if data.dtype == torch.bfloat16:
        return data.float()
    raise ValueError(f'unsupported dtype {data.dtype}')


def expand_sf(sf: torch.Tensor, shape, gran) -> torch.Tensor:
    """Broadcast a per-block fp32 SF tensor onto ``shape`` (repeat_interleave then crop)."""
    full = sf
    for dim, g in enumerate(gran):
        full = full.repeat_interleave(g, dim=dim)
    return full[tuple(slice(0, s) for s in shape)]


def quantize_blockwise(x: torch.Tensor, gran, quant: str = 'e4m3', major_dim: int = -1):
    """Block quantisation (tests/generators.py:61-95).

    Returns ``(data, sf, dequant)``: ``data`` e4m3 (or packed-fp4 int8) stored with
    ``major_dim`` contiguous, ``sf`` fp32 powers of two of shape ceil(shape/gran), and the
    exact fp32 value of ``data * sf``."""
    x = x.float()
    shape = list(x.shape)
    major_dim %= len(shape)
    padded = [align(s, g) for s, g in zip(shape, gran)]
    t = torch.zeros(padded, dtype=torch.float32)
    t[tuple(slice(0, s) for s in shape)] = x
    view = sum([[s // g, g] for s, g in zip(padded, gran)], [])
    perm = list(range(0, 2 * len(shape), 2)) + list(range(1, 2 * len(shape), 2))
    sf_shape = [s // g for s, g in zip(padded, gran)]
    blocks = t.reshape(*view).permute(perm).reshape(*sf_shape, -1)
    div = 448.0 if quant == 'e4m3' else 6.0
    sf = ceil_to_ue8m0(blocks.abs().amax(dim=-1).clamp(1e-4) / div).contiguous()
    full = expand_sf(sf, shape, gran)
    scaled = x / full
    if quant == 'e4m3':
        data = scaled.to(torch.float8_e4m3fn)
        data = data.transpose(major_dim, -1).contiguous().transpose(major_dim, -1)
        deq = decode(data) * full
    else:
        codes = quantize_fp4_codes(scaled)
        data = pack_fp4(codes, major_dim)
        deq = unpack_fp4(data, major_dim) * full
    return data, sf, deq.contiguous()


def random_codes(shape, quant: str, major_dim: int, gen: torch.Generator, gran):
    """Random-code operand generator (tests/generators.py:124-166): every non-NaN e4m3 code
    (or every fp4 nibble) uniformly, with UE8M0 block scales drawn from a small table."""
    shape = tuple(shape)
    major_dim %= len(shape)
    sf_shape = tuple(ceil_div(s, g) for s, g in zip(shape, gran))
    table = torch.tensor((2.0 ** -9, 2.0 ** -8, 2.0 ** -7) if quant == 'e4m3' else (0.25, 0.5, 1.0))
    sf = table[torch.randint(0, 3, sf_shape, generator=gen)].contiguous()
    storage = list(shape)
    storage[major_dim], storage[-1] = storage[-1], storage[major_dim]
    if quant == 'e4m3':
        raw = torch.randint(0, 254, storage, dtype=torch.uint8, generator=gen)
        raw += (raw >= 0x7f).to(torch.uint8)
        data = raw.view(torch.float8_e4m3fn).transpose(major_dim, -1)
        vals = decode(data)
    else:
        storage[-1] //= 2
        packed = torch.randint(-128, 128, storage, dtype=torch.int8, generator=gen)
        data = packed.transpose(major_dim, -1)
        vals = unpack_fp4(data, major_dim)
    deq = vals * expand_sf(sf, shape, gran)
    return data, sf, deq.contiguous()


def check_pow2(x: float) -> bool:
    m, _ = math.frexp(x)
    return m == 0.5
