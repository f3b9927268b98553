"""GPU parity of the GEMM family against the CPU oracle (calc_diff threshold 1e-5, the
reference's own bar: tests/test_fp8_gemm.py:21, test_bf16_gemm.py:17).  Every call goes
through libdeep_gemm_amd.so; padding / index handling is checked bit-exactly."""
import pytest
import torch

import deep_gemm
from oracle import gemm as og, layout as ol
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


def _ref_nt(a_deq, b_deq, out_dtype=torch.bfloat16, **kw):
    return og.gemm_nt(a_deq, b_deq, out_dtype, **kw)


def _fp8_case(m, n, k, gran_a=(1, 32), gran_b=(1, 32), mode='codes', seed=0, b_kind='e4m3', a_kind='e4m3'):
    g = gen(seed)
    a, sfa, a_deq = operand(m, k, a_kind, gran_a, g, mode)
    b, sfb, b_deq = operand(n, k, b_kind, gran_b, g, mode)
    return a, sfa, a_deq, b, sfb, b_deq


@pytest.mark.parametrize('m,n,k', [(128, 256, 512), (256, 512, 1024), (4096, 7168, 2048), (1, 2112, 7168),
                                   (64, 4096, 7168), (130, 257, 2048), (17, 4096, 4096), (513, 257, 4096),
                                   (64, 64, 4), (1024, 2048, 17), (128, 128, 234), (4, 4, 64)])
def test_fp8_gemm_nt_codes(m, n, k):
    print(f'fp8_gemm_nt codes m={m} n={n} k={k}', flush=True)
    a, sfa, a_deq, b, sfb, b_deq, = _fp8_case(m, n, k)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    ref = _ref_nt(a_deq, b_deq)
    diff = calc_diff(d.cpu(), ref)
    assert diff < THRESH, diff


@pytest.mark.parametrize('m,n,k', [(128, 256, 512), (4096, 7168, 2048), (128, 7168, 2048)])
def test_fp8_gemm_nt_deepseek_recipe(m, n, k):
    """BASELINE config: N(0,1) data, 1x128 activation and 128x128 weight UE8M0 scales."""
    print(f'fp8_gemm_nt 1x128/128x128 m={m} n={n} k={k}', flush=True)
    a, sfa, a_deq, b, sfb, b_deq = _fp8_case(m, n, k, (1, 128), (128, 128), mode='randn', seed=1)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    diff = calc_diff(d.cpu(), _ref_nt(a_deq, b_deq))
    assert diff < THRESH, diff


@pytest.mark.parametrize('layout', ['nt', 'nn', 'tn', 'tt'])
@pytest.mark.parametrize('m,n,k', [(256, 512, 1024), (130, 257, 640)])
def test_fp8_gemm_layouts(layout, m, n, k):
    print(f'fp8_gemm_{layout} m={m} n={n} k={k}', flush=True)
    a, sfa, a_deq, b, sfb, b_deq = _fp8_case(m, n, k, seed=2)
    a, sfa, b, sfb = a.cuda(), sfa.cuda(), b.cuda(), sfb.cuda()
    # logical shapes: A [M,K] (n*) or [K,M] (t*); B [N,K] (*t) or [K,N] (*n)
    if layout[0] == 't':
        a, sfa = a.t().contiguous().t().t(), sfa.t()
    if layout[1] == 'n':
        b, sfb = b.t().contiguous().t().t(), sfb.t()
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    getattr(deep_gemm, f'fp8_gemm_{layout}')((a, sfa), (b, sfb), d)
    torch.cuda.synchronize()
    diff = calc_diff(d.cpu(), _ref_nt(a_deq, b_deq))
    assert diff < THRESH, diff


def test_fp8_gemm_mn_major_operands():
    """dgrad/wgrad style: physically MN-major A and B behind the nt call."""
    m, n, k = 256, 384, 512
    a, sfa, a_deq, b, sfb, b_deq = _fp8_case(m, n, k, seed=3)
    a_mn = a.cuda().t().contiguous().t()      # [M,K] with stride(0) == 1
    b_mn = b.cuda().t().contiguous().t()
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a_mn, sfa.cuda()), (b_mn, sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), _ref_nt(a_deq, b_deq)) < THRESH


def test_fp8_gemm_bias_alpha_accumulate():
    m, n, k = 300, 520, 768
    a, sfa, a_deq, b, sfb, b_deq = _fp8_case(m, n, k, seed=4)
    a, sfa, b, sfb = a.cuda(), sfa.cuda(), b.cuda(), sfb.cuda()
    g = gen(5)
    # bias
    bias = torch.randn(1, n, generator=g).to(torch.bfloat16)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, c=bias.cuda())
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), _ref_nt(a_deq, b_deq, bias=bias)) < THRESH
    # alpha
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, alpha=-0.37)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), _ref_nt(a_deq, b_deq, alpha=-0.37)) < THRESH
    # accumulate into fp32 D
    c = torch.randn(m, n, generator=g)
    d = c.cuda().clone()
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, c=d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), _ref_nt(a_deq, b_deq, torch.float32, c=c)) < THRESH
    # fp32 out, alpha + accumulate
    d = c.cuda().clone()
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, c=d, alpha=0.5)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), _ref_nt(a_deq, b_deq, torch.float32, c=c, alpha=0.5)) < THRESH
    # alpha + bias is rejected
    with pytest.raises(RuntimeError, match='alpha and bias cannot be used together'):
        deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d.to(torch.bfloat16), c=bias.cuda(), alpha=2.0)


@pytest.mark.parametrize('recipe', [(1, 32, 32), (32, 1, 32), (32, 32, 32), (1, 128, 128)])
def test_fp8_gemm_recipes(recipe):
    m, n, k = 512, 384, 1024
    a, sfa, a_deq, b, sfb, b_deq = _fp8_case(m, n, k, (recipe[0], recipe[2]), (recipe[1], recipe[2]), seed=6)
    d = torch.empty(m, n, dtype=torch.float32, device='cuda')
    deep_gemm.fp8_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, recipe=recipe)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), _ref_nt(a_deq, b_deq, torch.float32)) < THRESH


def test_fp8_gemm_k_zero_and_empty():
    a = torch.empty(64, 0, dtype=torch.float8_e4m3fn, device='cuda')
    b = torch.empty(32, 0, dtype=torch.float8_e4m3fn, device='cuda')
    sfa = torch.empty(64, 0, dtype=torch.float32, device='cuda')
    sfb = torch.empty(32, 0, dtype=torch.float32, device='cuda')
    d = torch.full((64, 32), 7.0, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d)
    torch.cuda.synchronize()
    assert torch.equal(d.cpu(), torch.zeros(64, 32, dtype=torch.bfloat16))


@pytest.mark.parametrize('layout', ['nt', 'nn', 'tn', 'tt'])
@pytest.mark.parametrize('m,n,k', [(256, 512, 1024), (4096, 7168, 2048), (77, 130, 200)])
def test_bf16_gemm(layout, m, n, k):
    print(f'bf16_gemm_{layout} m={m} n={n} k={k}', flush=True)
    if (m, n, k) == (4096, 7168, 2048) and layout != 'nt':
        pytest.skip('large shape checked for nt only')
    g = gen(7)
    a = (torch.randn(m, k, generator=g) * 0.1).to(torch.bfloat16)
    b = (torch.randn(n, k, generator=g) * 0.1).to(torch.bfloat16)
    ref = _ref_nt(a.float(), b.float())
    ad, bd = a.cuda(), b.cuda()
    if layout[0] == 't':
        ad = ad.t()
    if layout[1] == 'n':
        bd = bd.t()
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    getattr(deep_gemm, f'bf16_gemm_{layout}')(ad, bd, d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), ref) < THRESH


def _group_sizes(num_groups, expected_m, g):
    return [max(int(expected_m * (0.7 + 0.6 * float(torch.rand(1, generator=g)))), 0) for _ in range(num_groups)]


@pytest.mark.parametrize('num_groups,expected_m,n,k,alignment', [
    (4, 200, 512, 1024, 256), (8, 300, 768, 512, 128), (128, 1, 64, 64, 256), (5, 0, 256, 256, 128),
    (4, 1000, 4096, 2048, 256)])
@pytest.mark.parametrize('psum', [True, False])
def test_m_grouped_fp8_contiguous(num_groups, expected_m, n, k, alignment, psum):
    print(f'm_grouped contiguous G={num_groups} m~{expected_m} n={n} k={k} align={alignment} psum={psum}', flush=True)
    g = gen(8)
    sizes = _group_sizes(num_groups, expected_m, g)
    total, ps = ol.psum_from_sizes(sizes, alignment)
    total = max(total, alignment)
    a, sfa, a_deq = operand(total, k, 'e4m3', (1, 32), g)
    # zero the padding rows of A (ensure_zero_padding); SF padding gets garbage like the reference
    for sl in ol.psum_pad_slices(ps, alignment):
        a.view(torch.uint8)[sl] = 0
        a_deq[sl] = 0
        sfa[sl] = torch.randn(sl.stop - sl.start, sfa.size(1), generator=g)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=num_groups)
    layout_t = torch.tensor(ps, dtype=torch.int32) if psum else ol.m_indices_from_psum(ps, alignment, total)
    ref = og.m_grouped_contiguous(a_deq, b_deq, layout_t, psum, alignment)
    d = torch.full((total, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d,
                                                   layout_t.cuda(), use_psum_layout=psum)
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    torch.cuda.synchronize()
    out = d.cpu()
    assert not torch.isnan(out.float()).any()
    # padding rows are exact zeros, valid rows within tolerance
    valid = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(ps, alignment):
        valid[sl] = True
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid]))
    assert calc_diff(out[valid], ref[valid]) < THRESH


@pytest.mark.parametrize('num_groups,max_m,n,k', [(4, 256, 512, 1024), (32, 256, 4096, 7168), (3, 100, 200, 300)])
def test_m_grouped_fp8_masked(num_groups, max_m, n, k):
    print(f'masked G={num_groups} max_m={max_m} n={n} k={k}', flush=True)
    g = gen(9)
    a, sfa, a_deq = operand(max_m, k, 'e4m3', (1, 32), g, batch=num_groups)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=num_groups)
    masked = torch.randint(0, max_m + 1, (num_groups,), generator=g, dtype=torch.int32)
    masked[0] = max_m
    d = torch.zeros(num_groups, max_m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.m_grouped_fp8_gemm_nt_masked((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, masked.cuda(), max_m)
    torch.cuda.synchronize()
    ref = og.m_grouped_masked(a_deq, b_deq, masked)
    out = d.cpu()
    for i in range(num_groups):
        mg = int(masked[i])
        if mg:
            assert calc_diff(out[i, :mg], ref[i, :mg]) < THRESH, i


@pytest.mark.parametrize('m,n,k', [(128, 7168, 2048), (4096, 7168, 2048), (256, 512, 1024), (130, 250, 320)])
def test_fp8_fp4_gemm(m, n, k):
    print(f'fp8xfp4 m={m} n={n} k={k}', flush=True)
    g = gen(10)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g)
    b, sfb, b_deq = operand(n, k, 'e2m1', (1, 32), g)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), _ref_nt(a_deq, b_deq)) < THRESH


def test_fp8_fp4_gemm_deepseek_recipe():
    """N(0,1) weights quantised to e2m1 with 1x32 scales, A 1x128."""
    m, n, k = 4096, 7168, 2048
    g = gen(11)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, mode='randn')
    b, sfb, b_deq = operand(n, k, 'e2m1', (1, 32), g, mode='randn')
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, recipe_a=(1, 128), recipe_b=(1, 32))
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), _ref_nt(a_deq, b_deq)) < THRESH


@pytest.mark.parametrize('m,n,k', [(256, 512, 1024), (100, 200, 256)])
def test_fp4_fp4_gemm(m, n, k):
    g = gen(12)
    a, sfa, a_deq = operand(m, k, 'e2m1', (1, 32), g)
    b, sfb, b_deq = operand(n, k, 'e2m1', (1, 32), g)
    d = torch.empty(m, n, dtype=torch.float32, device='cuda')
    deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), _ref_nt(a_deq, b_deq, torch.float32)) < THRESH


def test_fp8_fp4_mn_major_b():
    """FP4 B packed along N (MN-major) goes through the re-pack path."""
    m, n, k = 128, 256, 512
    g = gen(13)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g)
    from oracle import quant
    b_codes, sfb, b_deq = quant.random_codes((n, k), 'e2m1', 0, g, (1, 32))   # packed along N
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b_codes.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), _ref_nt(a_deq, b_deq)) < THRESH
