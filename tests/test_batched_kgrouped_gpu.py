"""GPU parity of the batched GEMMs (fp8_bmm / bf16_bmm), the fixed einsum contractions
(einsum / fp8_einsum) and the K-grouped contiguous GEMMs against the CPU oracle, through
libdeep_gemm_amd.so.  Threshold: calc_diff < 1e-5 (the reference's bar,
tests/test_fp8_gemm.py:21); empty K groups and untouched outputs are checked bit-exactly.

Operand construction follows the reference's generators: batched operands per batch
(tests/generators.py:392-419); K-grouped operands MN-major [Ktot, M] / [Ktot, N] with the K
padding between groups zeroed and garbage written into the SF of that padding
(tests/generators.py:361-390)."""
import pytest
import torch

import deep_gemm
from oracle import gemm as og, layout as ol
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


# ----------------------------------------------------------------------------- batched
def _bmm_case(bs, m, n, k, seed):
    g = gen(seed)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g, 'codes', batch=bs)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, 'codes', batch=bs)
    return a, sfa, a_deq, b, sfb, b_deq


@pytest.mark.parametrize('bs,m,n,k', [(4, 128, 256, 512), (3, 130, 257, 640), (2, 1, 2112, 7168),
                                      (8, 64, 128, 4096), (1, 256, 512, 1024), (5, 33, 48, 96)])
@pytest.mark.parametrize('out_dtype', [torch.bfloat16, torch.float32])
def test_fp8_bmm(bs, m, n, k, out_dtype):
    print(f'fp8_bmm bs={bs} m={m} n={n} k={k} {out_dtype}', flush=True)
    a, sfa, a_deq, b, sfb, b_deq = _bmm_case(bs, m, n, k, seed=m + n)
    d = torch.empty(bs, m, n, dtype=out_dtype, device='cuda')
    deep_gemm.fp8_bmm((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    ref = og.batched_nt(a_deq, b_deq, None, out_dtype)
    for i in range(bs):   # per batch: a wrong batch offset cannot hide behind the others
        assert calc_diff(d[i].cpu(), ref[i]) < THRESH, i


@pytest.mark.parametrize('aliased', [True, False])
def test_fp8_bmm_accumulate(aliased):
    bs, m, n, k = 3, 128, 384, 768
    a, sfa, a_deq, b, sfb, b_deq = _bmm_case(bs, m, n, k, seed=5)
    c = torch.randn(bs, m, n, generator=gen(6))
    d = c.clone().cuda() if aliased else torch.empty(bs, m, n, device='cuda')
    c_dev = d if aliased else c.cuda()
    deep_gemm.fp8_bmm((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, c=c_dev)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.batched_nt(a_deq, b_deq, c, torch.float32)) < THRESH


def test_fp8_bmm_mn_major_and_strided_batch():
    """MN-major A (wgrad-style) and a D whose batch stride is not M*N."""
    bs, m, n, k = 3, 192, 256, 512
    a, sfa, a_deq, b, sfb, b_deq = _bmm_case(bs, m, n, k, seed=7)
    a_mn = a.cuda().transpose(1, 2).contiguous().transpose(1, 2)
    big = torch.zeros(bs, m + 8, n, dtype=torch.bfloat16, device='cuda')
    d = big[:, 4:4 + m]
    deep_gemm.fp8_bmm((a_mn, sfa.cuda().transpose(1, 2).contiguous().transpose(1, 2)), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.batched_nt(a_deq, b_deq)) < THRESH
    assert int(big[:, :4].count_nonzero()) == 0 and int(big[:, 4 + m:].count_nonzero()) == 0


@pytest.mark.parametrize('bs,m,n,k', [(4, 128, 256, 512), (3, 130, 257, 200)])
def test_bf16_bmm(bs, m, n, k):
    print(f'bf16_bmm bs={bs} m={m} n={n} k={k}', flush=True)
    g = gen(8)
    a = torch.randn(bs, m, k, generator=g).bfloat16()
    b = torch.randn(bs, n, k, generator=g).bfloat16()
    c = torch.randn(bs, m, n, generator=g)
    d = c.cuda()
    deep_gemm.bf16_bmm(a.cuda(), b.cuda(), d, c=d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.batched_nt(a.float(), b.float(), c, torch.float32)) < THRESH


def test_bmm_empty_batch_and_k0():
    a = torch.empty(0, 4, 64, dtype=torch.bfloat16, device='cuda')
    d = torch.empty(0, 4, 8, dtype=torch.bfloat16, device='cuda')
    deep_gemm.bf16_bmm(a, torch.empty(0, 8, 64, dtype=torch.bfloat16, device='cuda'), d)
    a0 = torch.empty(2, 4, 0, dtype=torch.bfloat16, device='cuda')
    d0 = torch.full((2, 4, 8), 3.0, dtype=torch.bfloat16, device='cuda')
    deep_gemm.bf16_bmm(a0, torch.empty(2, 8, 0, dtype=torch.bfloat16, device='cuda'), d0)
    torch.cuda.synchronize()
    assert int(d0.count_nonzero()) == 0


# ----------------------------------------------------------------------------- einsum
# (API permutation of A, of B) per expression (csrc/apis/einsum.hpp:99-199): view = orig.permute(p)
_PERMS = {
    'bhr,hdr->bhd': ((1, 0, 2), (0, 1, 2)),
    'bhd,hdr->bhr': ((1, 0, 2), (0, 2, 1)),
    'bhd,bhr->hdr': ((1, 2, 0), (1, 2, 0)),
}


def _inv(p):
    return tuple(p.index(i) for i in range(len(p)))


def _einsum_views(expr, B, H, D, R):
    """(batch, M, N, K) of the batched GEMM the expression becomes."""
    return {'bhr,hdr->bhd': (H, B, D, R), 'bhd,hdr->bhr': (H, B, R, D), 'bhd,bhr->hdr': (H, D, R, B)}[expr]


@pytest.mark.parametrize('expr', list(_PERMS))
@pytest.mark.parametrize('acc', [False, True])
def test_fp8_einsum(expr, acc):
    print(f'fp8_einsum {expr} acc={acc}', flush=True)
    B, H, D, R = 96, 4, 128, 192
    bs, m, n, k = _einsum_views(expr, B, H, D, R)
    g = gen(9)
    a_v, sfa_v, a_deq_v = operand(m, k, 'e4m3', (1, 32), g, 'codes', batch=bs)
    b_v, sfb_v, b_deq_v = operand(n, k, 'e4m3', (1, 32), g, 'codes', batch=bs)
    pa, pb = _PERMS[expr]
    # the caller's tensors: contiguous in the expression's own index order
    a = a_v.permute(*_inv(pa)).contiguous()
    sfa = sfa_v.permute(*_inv(pa)).contiguous()
    b = b_v.permute(*_inv(pb)).contiguous()
    sfb = sfb_v.permute(*_inv(pb)).contiguous()
    a_deq, b_deq = a_deq_v.permute(*_inv(pa)), b_deq_v.permute(*_inv(pb))
    out_shape = og.einsum_ref(expr, a_deq, b_deq, None, torch.float32).shape
    c = torch.randn(out_shape, generator=gen(10)) if acc else None
    d = c.clone().cuda() if acc else torch.empty(out_shape, device='cuda')
    deep_gemm.fp8_einsum(expr, (a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, c=d if acc else None)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.einsum_ref(expr, a_deq, b_deq, c, torch.float32)) < THRESH


@pytest.mark.parametrize('expr', list(_PERMS))
def test_bf16_einsum(expr):
    print(f'einsum {expr}', flush=True)
    B, H, D, R = 80, 3, 96, 128
    sizes = {'b': B, 'h': H, 'd': D, 'r': R}
    ins, out = expr.split('->')
    ta, tb = ins.split(',')
    g = gen(11)
    a = torch.randn([sizes[x] for x in ta], generator=g).bfloat16()
    b = torch.randn([sizes[x] for x in tb], generator=g).bfloat16()
    d = torch.empty([sizes[x] for x in out], dtype=torch.bfloat16, device='cuda')
    deep_gemm.einsum(expr, a.cuda(), b.cuda(), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.einsum_ref(expr, a.float(), b.float())) < THRESH


def test_einsum_rejects_unknown_and_cublaslt():
    x = torch.empty(2, 2, 2, dtype=torch.bfloat16, device='cuda')
    with pytest.raises(RuntimeError, match='Unsupported einsum expression'):
        deep_gemm.einsum('bhd,hrd->bhr', x, x, x)
    with pytest.raises(RuntimeError, match='use_cublaslt'):
        deep_gemm.einsum('bhr,hdr->bhd', x, x, x, use_cublaslt=True)


# ----------------------------------------------------------------------------- K-grouped
def _k_grouped_case(m, n, ks, seed, alignment=256):
    """A [Ktot, M], B [Ktot, N] e4m3 MN-major with zero K padding between groups; fp32 SF
    [Ktot/32, M] / [Ktot/32, N] with garbage (negative, non-power-of-two) in the padding."""
    total, psum = ol.psum_from_sizes(ks, alignment)
    g = gen(seed)
    keep = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(psum, alignment):
        keep[sl] = True
    out = [psum]
    for rows in (m, n):
        x, sf, deq = operand(rows, total, 'e4m3', (1, 32), g, 'codes')     # [rows, Ktot] K-major
        raw = x.view(torch.uint8).clone()
        raw[:, ~keep] = 0
        for span in ol.psum_pad_slices(psum, alignment, 32):
            sf[:, span] = -torch.rand(sf[:, span].shape, generator=g) - 0.3
        x_tn = raw.t().contiguous().view(torch.float8_e4m3fn)                # [Ktot, rows]
        out += [x_tn, sf.t(), (deq * keep).t()]
    return out


@pytest.mark.parametrize('g_,m,n,ks', [
    (4, 256, 384, [512, 300, 0, 1000]),
    (1, 128, 128, [1]),
    (3, 130, 257, [0, 64, 0]),
    (8, 512, 256, [256, 256, 200, 512, 0, 17, 700, 256]),
    (4, 4096, 2048, [1500, 2000, 0, 2560]),
])
@pytest.mark.parametrize('acc,out_dtype', [(False, torch.bfloat16), (True, torch.float32), (False, torch.float32)])
def test_k_grouped_fp8_gemm_tn(g_, m, n, ks, acc, out_dtype):
    print(f'k_grouped tn G={g_} m={m} n={n} ks={ks} acc={acc} {out_dtype}', flush=True)
    psum, a_tn, sfa, a_deq, b_tn, sfb, b_deq = _k_grouped_case(m, n, ks, seed=m + n + g_)
    c = torch.randn(g_, m, n, generator=gen(12)) if acc else None
    d = c.clone().cuda() if acc else torch.full((g_, m, n), float('nan'), dtype=out_dtype, device='cuda')
    layout = torch.tensor(psum, dtype=torch.int32, device='cuda')
    deep_gemm.k_grouped_fp8_gemm_tn_contiguous((a_tn.cuda(), sfa.cuda()), (b_tn.cuda(), sfb.cuda()), d,
                                               ks, layout, c=d if acc else None)
    torch.cuda.synchronize()
    ref = og.k_grouped_tn(a_deq, b_deq, psum, 256, c, out_dtype)
    dc = d.cpu()
    for gi in range(g_):
        if ks[gi] == 0:   # empty group: exactly 0 (+ C)
            assert torch.equal(dc[gi], ref[gi]), gi
        else:
            assert calc_diff(dc[gi], ref[gi]) < THRESH, gi


def test_k_grouped_fp8_gemm_nt_deprecated():
    m, n, ks = 128, 256, [300, 512]
    psum, a_tn, sfa, a_deq, b_tn, sfb, b_deq = _k_grouped_case(m, n, ks, seed=13)
    d = torch.empty(2, m, n, dtype=torch.bfloat16, device='cuda')
    layout = torch.tensor(psum, dtype=torch.int32, device='cuda')
    with pytest.warns(DeprecationWarning):
        deep_gemm.k_grouped_fp8_gemm_nt_contiguous((a_tn.cuda().t(), sfa.cuda().t()), (b_tn.cuda().t(), sfb.cuda().t()),
                                                   d, ks, layout)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.k_grouped_tn(a_deq, b_deq, psum, 256)) < THRESH


def test_k_grouped_bf16_gemm_tn():
    m, n, ks = 256, 384, [700, 0, 256, 90]
    total, psum = ol.psum_from_sizes(ks, 256)
    g = gen(14)
    keep = torch.zeros(total, 1)
    for sl in ol.psum_slices(psum, 256):
        keep[sl] = 1
    a = (torch.randn(total, m, generator=g) * keep).bfloat16()
    b = (torch.randn(total, n, generator=g) * keep).bfloat16()
    c = torch.randn(len(ks), m, n, generator=g)
    d = c.clone().cuda()
    deep_gemm.k_grouped_bf16_gemm_tn_contiguous(a.cuda(), b.cuda(), d, ks,
                                                torch.tensor(psum, dtype=torch.int32, device='cuda'), c=d)
    torch.cuda.synchronize()
    ref = og.k_grouped_tn(a.float(), b.float(), psum, 256, c, torch.float32)
    assert torch.equal(d[1].cpu(), c[1])
    assert calc_diff(d.cpu(), ref) < THRESH


@pytest.mark.parametrize('dtype', [torch.float32, torch.int16])
@pytest.mark.parametrize('mn,gran_mn', [(4096, 1), (4097, 32), (300, 128)])
def test_transform_k_grouped_sf(dtype, mn, gran_mn):
    """Bit-exact against the oracle; the padding SF holds values that would be rejected
    (negative fp32) and must come out as 0 (tests/test_layout.py:96-98)."""
    ks = [2000, 300, 0, 4096 - 16]
    total, psum = ol.psum_from_sizes(ks, 256)
    w = 32 if dtype == torch.float32 else 64
    g = gen(15)
    shape = (-(-mn // gran_mn), -(-total // w))
    if dtype == torch.float32:
        sf = (torch.randint(1, 255, shape, generator=g, dtype=torch.int32) << 23).view(torch.float32)
        pad_val = -1.0
    else:
        sf = torch.randint(-32768, 32768, shape, generator=g, dtype=torch.int16)
        pad_val = 0x7777
    for span in ol.psum_pad_slices(psum, 256, w):
        sf[:, span] = pad_val
    expect = ol.transform_k_grouped_sf(sf, mn, total, gran_mn, psum, 32, 256)
    out = deep_gemm.transform_k_grouped_sf_into_required_layout(
        sf.cuda(), mn, total, (gran_mn, gran_mn, 32), True, torch.tensor(psum, dtype=torch.int32, device='cuda'))
    torch.cuda.synchronize()
    assert out.stride(-2) == 1 and out.shape == expect.shape
    assert torch.equal(out.cpu(), expect)
