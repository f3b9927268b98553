"""GPU parity at every BASELINE configuration, at the sizes the configurations name.

Data follows the configurations: seeded N(0,1) operands quantised to e4m3 with 1x128 (A) /
128x128 (B) UE8M0 scales (``quantize_with_major``, tests/generators.py:61-95 of the
reference), e2m1 weights with 1x32 scales, bf16 operands N(0,1) * 0.1.  The oracle is the
reference's own reference path (dequantise -> fp32 matmul -> bf16, tests/generators.py:320-322).
Bar: calc_diff < 1e-5 (the reference's tests/test_fp8_gemm.py:21), grouped padding rows exact 0.
"""
import pytest
import torch

import deep_gemm
from oracle import gemm as og, layout as ol, quant
from helpers import gen, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5
NK = [(2112, 7168), (24576, 1536), (7168, 16384), (4096, 7168), (7168, 2048)]


def _q(rows, k, gran, kind, g, batch=0):
    if not batch:
        return quant.quantize_blockwise(torch.randn(rows, k, generator=g), gran, kind)
    # one batch at a time into preallocated outputs, so the quantiser's temporaries stay one
    # batch in size
    out = None
    for i in range(batch):
        parts = quant.quantize_blockwise(torch.randn(rows, k, generator=g), gran, kind)
        if out is None:
            out = [torch.empty((batch,) + tuple(t.shape), dtype=t.dtype) for t in parts]
        for o, t in zip(out, parts):
            o[i] = t
    return tuple(out)


@pytest.mark.parametrize('n,k', NK)
@pytest.mark.parametrize('m', [1, 64, 128, 4096])
def test_config2_fp8_gemm_nt(m, n, k):
    print(f'config2 fp8_gemm_nt m={m} n={n} k={k} tile={deep_gemm.select_config(m, n, k)}', flush=True)
    g = gen(100 + m)
    a, sfa, a_deq = _q(m, k, (1, 128), 'e4m3', g)
    b, sfb, b_deq = _q(n, k, (128, 128), 'e4m3', g)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    diff = calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq))
    assert diff < THRESH, diff


@pytest.mark.parametrize('m,n,k', [(4096, 7168, 2048), (4096, 2112, 7168), (128, 4096, 7168), (1, 24576, 1536)])
def test_config2_bias(m, n, k):
    """The optional bf16 [1, N] bias of config 2, added in the epilogue."""
    print(f'config2 bias m={m} n={n} k={k}', flush=True)
    g = gen(200 + m)
    a, sfa, a_deq = _q(m, k, (1, 128), 'e4m3', g)
    b, sfb, b_deq = _q(n, k, (128, 128), 'e4m3', g)
    bias = torch.randn(1, n, generator=g).to(torch.bfloat16)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, c=bias.cuda(),
                          recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    diff = calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq, bias=bias))
    assert diff < THRESH, diff


@pytest.mark.parametrize('layout', ['nt', 'nn'])
@pytest.mark.parametrize('n,k', NK)
@pytest.mark.parametrize('m', [1, 64, 128, 4096])
def test_config3_bf16_gemm(m, n, k, layout):
    print(f'config3 bf16_gemm_{layout} m={m} n={n} k={k}', flush=True)
    g = gen(300 + m)
    a = (torch.randn(m, k, generator=g) * 0.1).to(torch.bfloat16)
    b = (torch.randn(n, k, generator=g) * 0.1).to(torch.bfloat16)
    ref = og.gemm_nt(a.float(), b.float())
    bd = b.cuda()
    if layout == 'nn':
        bd = bd.t().contiguous()     # B physically [K, N]
        fn = deep_gemm.bf16_gemm_nn
    else:
        fn = deep_gemm.bf16_gemm_nt
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    fn(a.cuda(), bd, d)
    torch.cuda.synchronize()
    diff = calc_diff(d.cpu(), ref)
    assert diff < THRESH, diff


def routed_counts(num_tokens=8192, num_experts=256, topk=8, local=32, seed=0):
    """Tokens per local expert: top-8 of N(0,1) logits over 256 experts, first 32 experts."""
    g = torch.Generator().manual_seed(seed)
    idx = torch.randn(num_tokens, num_experts, generator=g).topk(topk, dim=-1).indices.flatten()
    return torch.bincount(idx, minlength=num_experts)[:local].tolist()


_B_CACHE = {}


def _grouped_weights(n, k):
    """[32, N, K] e4m3 weights with 128x128 scales (cached: three tests share each shape)."""
    if (n, k) not in _B_CACHE:
        _B_CACHE[(n, k)] = _q(n, k, (128, 128), 'e4m3', gen(400 + n), batch=32)
    return _B_CACHE[(n, k)]


@pytest.mark.parametrize('psum', [True, False])
@pytest.mark.parametrize('n,k', [(4096, 7168), (7168, 2048)])
def test_config4_m_grouped_contiguous(n, k, psum):
    counts = routed_counts()
    alignment = 128
    total, ps = ol.psum_from_sizes(counts, alignment)
    print(f'config4 contiguous G=32 rows={total} valid={sum(counts)} n={n} k={k} psum={psum}', flush=True)
    g = gen(401)
    a, sfa, a_deq = _q(total, k, (1, 128), 'e4m3', g)
    for sl in ol.psum_pad_slices(ps, alignment):
        a.view(torch.uint8)[sl] = 0
        a_deq[sl] = 0
    b, sfb, b_deq = _grouped_weights(n, k)
    layout_t = torch.tensor(ps, dtype=torch.int32) if psum else ol.m_indices_from_psum(ps, alignment, total)
    d = torch.full((total, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, layout_t.cuda(),
                                                   recipe_a=(1, 128), recipe_b=(128, 128), use_psum_layout=psum)
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    torch.cuda.synchronize()
    out = d.cpu()
    valid = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(ps, alignment):
        valid[sl] = True
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid])), 'padding rows must be exact zeros'
    ref = og.m_grouped_contiguous(a_deq, b_deq, layout_t, psum, alignment)
    diff = calc_diff(out[valid], ref[valid])
    assert diff < THRESH, diff


@pytest.mark.parametrize('n,k', [(7168, 2048), (4096, 7168)])
def test_config4_m_grouped_masked(n, k):
    counts = routed_counts()
    max_m = 256
    masked = torch.tensor([min(c, max_m) for c in counts], dtype=torch.int32)
    print(f'config4 masked G=32 max_m={max_m} valid={int(masked.sum())} n={n} k={k}', flush=True)
    g = gen(402)
    a, sfa, a_deq = _q(max_m, k, (1, 128), 'e4m3', g, batch=32)
    b, sfb, b_deq = _grouped_weights(n, k)
    d = torch.full((32, max_m, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    deep_gemm.m_grouped_fp8_gemm_nt_masked((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, masked.cuda(),
                                           int(masked.float().mean()), recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    out = d.cpu()
    ref = og.m_grouped_masked(a_deq, b_deq, masked)
    for i in range(32):
        mg = int(masked[i])
        if mg:
            assert calc_diff(out[i, :mg], ref[i, :mg]) < THRESH, i
        # rows past masked_m are not written
        assert torch.isnan(out[i, mg:].float()).all(), i


@pytest.mark.parametrize('n,k', [(7168, 2048), (4096, 7168)])
@pytest.mark.parametrize('m', [128, 4096])
def test_config5_fp8_fp4_gemm(m, n, k):
    print(f'config5 fp8_fp4_gemm_nt m={m} n={n} k={k}', flush=True)
    g = gen(500 + m)
    a, sfa, a_deq = _q(m, k, (1, 128), 'e4m3', g)
    b, sfb, b_deq = _q(n, k, (1, 32), 'e2m1', g)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, recipe_a=(1, 128), recipe_b=(1, 32))
    torch.cuda.synchronize()
    diff = calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq))
    assert diff < THRESH, diff


@pytest.mark.parametrize('layout', ['nt', 'nn'])
@pytest.mark.parametrize('psum', [True, False])
def test_m_grouped_bf16_contiguous(layout, psum):
    """m_grouped_bf16_gemm_{nt,nn}_contiguous: psum and m_indices layouts, an empty group."""
    alignment = 128
    sizes = [300, 0, 129, 77, 512, 1]
    total, ps = ol.psum_from_sizes(sizes, alignment)
    n, k = 768, 1024
    print(f'm_grouped_bf16_{layout} contiguous rows={total} psum={psum}', flush=True)
    g = gen(600)
    a = (torch.randn(total, k, generator=g) * 0.1).to(torch.bfloat16)
    for sl in ol.psum_pad_slices(ps, alignment):
        a[sl] = 0
    b = (torch.randn(len(sizes), n, k, generator=g) * 0.1).to(torch.bfloat16)
    layout_t = torch.tensor(ps, dtype=torch.int32) if psum else ol.m_indices_from_psum(ps, alignment, total)
    ref = og.m_grouped_contiguous(a.float(), b.float(), layout_t, psum, alignment)
    bd = b.cuda()
    if layout == 'nn':
        bd = bd.transpose(1, 2).contiguous()      # [G, K, N]
    d = torch.full((total, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        getattr(deep_gemm, f'm_grouped_bf16_gemm_{layout}_contiguous')(a.cuda(), bd, d, layout_t.cuda(),
                                                                       use_psum_layout=psum)
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    torch.cuda.synchronize()
    out = d.cpu()
    valid = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(ps, alignment):
        valid[sl] = True
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid]))
    assert calc_diff(out[valid], ref[valid]) < THRESH


def test_m_grouped_bf16_masked():
    gnum, max_m, n, k = 6, 192, 512, 768
    g = gen(601)
    a = (torch.randn(gnum, max_m, k, generator=g) * 0.1).to(torch.bfloat16)
    b = (torch.randn(gnum, n, k, generator=g) * 0.1).to(torch.bfloat16)
    masked = torch.tensor([192, 0, 1, 64, 100, 191], dtype=torch.int32)
    d = torch.full((gnum, max_m, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    deep_gemm.m_grouped_bf16_gemm_nt_masked(a.cuda(), b.cuda(), d, masked.cuda(), 96)
    torch.cuda.synchronize()
    out = d.cpu()
    ref = og.m_grouped_masked(a.float(), b.float(), masked)
    for i in range(gnum):
        mg = int(masked[i])
        if mg:
            assert calc_diff(out[i, :mg], ref[i, :mg]) < THRESH, i
        assert torch.isnan(out[i, mg:].float()).all(), i
