"""GPU transform_sf_into_required_layout against the oracle, bit-exact (the reference's
tests/test_layout.py:53-58 bar), over dtype x major x MN x K x batches x gran_mn, plus the
psum M-grouped padding rows (tests/test_layout.py:75-109)."""
import itertools

import pytest
import torch

import deep_gemm
from oracle import layout as ol
from helpers import gen

pytestmark = pytest.mark.gpu


def _make_sf(shape, dtype, g):
    if dtype == torch.float32:
        e = torch.randint(1, 255, shape, dtype=torch.int32, generator=g)
        return (e << 23).view(torch.float32)
    return torch.randint(-32768, 32768, shape, dtype=torch.int32, generator=g).to(torch.int16)


def _with_major(sf, mn_major):
    if mn_major and sf.size(-2) > 1 and sf.size(-1) > 1:
        return sf.transpose(-2, -1).contiguous().transpose(-2, -1)
    return sf


def _check(out, exp):
    assert out.dtype == torch.int16
    assert tuple(out.shape) == tuple(exp.shape)
    mn = out.size(-2)
    ld = mn + (mn & 1)   # even leading dimension; the padding element of each column is 0
    assert out.stride(-2) == 1 and out.stride(-1) == ld
    assert torch.equal(out.cpu(), exp)
    if mn & 1:
        full = torch.as_strided(out, out.shape[:-2] + (ld, out.size(-1)), out.stride())
        assert torch.all(full[..., mn, :].cpu() == 0)


CASES = list(itertools.product((torch.float32, torch.int16), (False, True), (4096, 4097, 8192), (128, 7168, 7296),
                               (1, 2), (1, 32, 128)))


@pytest.mark.parametrize('dtype,mn_major,mn,k,batches,gran_mn', CASES)
def test_transform_sf(dtype, mn_major, mn, k, batches, gran_mn):
    g = gen(mn + k + batches + gran_mn)
    div = 32 if dtype == torch.float32 else 64
    shape = ((batches,) if batches > 1 else ()) + ((mn + gran_mn - 1) // gran_mn, (k + div - 1) // div)
    sf = _with_major(_make_sf(shape, dtype, g), mn_major)
    exp = ol.transform_sf(sf, mn, k, gran_mn)
    out = deep_gemm.transform_sf_into_required_layout(sf.cuda(), mn, k, (gran_mn, gran_mn, 32),
                                                      num_groups=batches if batches > 1 else None, is_sfa=True)
    torch.cuda.synchronize()
    _check(out, exp)


@pytest.mark.parametrize('gran_k', [32, 128])
def test_transform_sf_gran_k(gran_k):
    g = gen(3)
    mn, k = 300, 1000
    sf = _make_sf((mn, (k + gran_k - 1) // gran_k), torch.float32, g)
    exp = ol.transform_sf(sf, mn, k, 1, gran_k)
    out = deep_gemm.transform_sf_into_required_layout(sf.cuda(), mn, k, (1, gran_k), is_sfa=True)
    torch.cuda.synchronize()
    _check(out, exp)


@pytest.mark.parametrize('dtype', [torch.float32, torch.int16])
@pytest.mark.parametrize('gran_mn', [1, 32, 128])
@pytest.mark.parametrize('mn_major', [False, True])
def test_transform_sf_psum(dtype, gran_mn, mn_major):
    g = gen(gran_mn)
    alignment, k = 256, 7168
    sizes = [700, 0, 256, 1, 513, 1000]
    total, ps = ol.psum_from_sizes(sizes, alignment)
    div = 32 if dtype == torch.float32 else 64
    sf = _make_sf(((total + gran_mn - 1) // gran_mn, (k + div - 1) // div), dtype, g)
    exp_src = sf.clone()
    for span in ol.psum_pad_slices(ps, alignment, gran_mn):
        exp_src[span] = 0
        sf[span] = -1 if dtype == torch.float32 else 0     # invalid SF in padding must be ignored
    sf = _with_major(sf, mn_major)
    exp = ol.transform_sf(exp_src, total, k, gran_mn)
    out = deep_gemm.transform_sf_into_required_layout(sf.cuda(), total, k, (gran_mn, gran_mn, 32), is_sfa=True,
                                                      psum_layout=torch.tensor(ps, dtype=torch.int32).cuda())
    torch.cuda.synchronize()
    _check(out, exp)


def test_transform_sf_passthrough():
    """Already-required-layout int16 SF is returned as is (csrc/apis/layout.hpp:57-62)."""
    sf = torch.zeros(4, 1000, dtype=torch.int16, device='cuda').t()
    out = deep_gemm.transform_sf_into_required_layout(sf, 1000, 256, (1, 1, 32), is_sfa=False)
    assert out.data_ptr() == sf.data_ptr()


def test_transform_sf_invalid_flag(monkeypatch):
    monkeypatch.setenv('DG_CHECK_SF', '1')
    sf = torch.full((8, 4), 1.5, device='cuda')
    with pytest.raises(RuntimeError, match='Invalid float32 SF'):
        deep_gemm.transform_sf_into_required_layout(sf, 8, 128, (1, 1, 32), is_sfa=True)


def test_transform_sf_invalid_flag_mn_major(monkeypatch):
    """The same check on the vectorised path (MN-major fp32 SF, 4 MN per thread): one bad value."""
    monkeypatch.setenv('DG_CHECK_SF', '1')
    sf = torch.ones(4, 64, device='cuda').t()            # [MN=64, K/32=4] view, MN contiguous
    sf_bad = sf.clone().t().contiguous().t()
    sf_bad[37, 2] = -2.0
    out = deep_gemm.transform_sf_into_required_layout(sf, 64, 128, (1, 1, 32), is_sfa=True)
    torch.cuda.synchronize()
    assert out.shape[0] == 64
    with pytest.raises(RuntimeError, match='Invalid float32 SF'):
        deep_gemm.transform_sf_into_required_layout(sf_bad, 64, 128, (1, 1, 32), is_sfa=True)


@pytest.mark.parametrize('dtype', [torch.float8_e4m3fn, torch.bfloat16])
@pytest.mark.parametrize('batch,k,mn', [(0, 64, 64), (0, 2048, 7168), (0, 100, 37), (3, 130, 257), (2, 1, 5), (0, 7, 300)])
def test_transpose_to_k_major(dtype, batch, k, mn):
    """MN-major -> K-major operand copy: bit-exact against torch's transpose, zero K padding."""
    from deep_gemm.gemm import _transpose_to_k_major
    g = torch.Generator().manual_seed(k + mn)
    shape = (batch, k, mn) if batch else (k, mn)
    raw = torch.randint(0, 255, shape, generator=g, dtype=torch.uint8)
    src = raw.view(torch.float8_e4m3fn) if dtype != torch.bfloat16 else torch.randn(shape, generator=g).bfloat16()
    # the caller's MN-major [.., MN, K] view of a [.., K, MN] tensor, with a padded K-row stride
    big = torch.zeros((*shape[:-1], mn + 24), dtype=src.dtype) if dtype == torch.bfloat16 else \
        torch.zeros((*shape[:-1], mn + 24), dtype=torch.uint8).view(src.dtype)
    big[..., :mn] = src
    view = big.cuda()[..., :mn].transpose(-2, -1)
    out = _transpose_to_k_major(view, k)
    torch.cuda.synchronize()
    esize = src.element_size()
    kpad = -(-k // (16 // esize)) * (16 // esize)
    assert out.shape == (*shape[:-2], mn, kpad) and out.is_contiguous()
    bits = torch.int16 if esize == 2 else torch.uint8
    expect = src.transpose(-2, -1).contiguous().view(bits)
    got = out.cpu().view(bits)
    assert torch.equal(got[..., :k], expect)
    assert int(got[..., k:].count_nonzero()) == 0
