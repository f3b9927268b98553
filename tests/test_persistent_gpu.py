"""GPU parity of the persistent tile kernel (csrc/gemm_persistent.hpp) and the set_num_sms cap.

With set_num_sms below the device's CU count at most num_sms workgroups run: the 128-K-stage
tiles with a persistent kernel walk the tiles with min(tiles, num_sms) workgroups (the reference's persistent block walk,
deep_gemm/include/deep_gemm/scheduler.hpp:141-196, launched with num_cores blocks,
csrc/jit_kernels/heuristics.hpp:98).  Checked against the oracle (calc_diff < 1e-5) and, where the
tile shape matches the uncapped launch, bit for bit against it (same MFMAs in the same K order).
"""
import pytest
import torch

import deep_gemm
from oracle import gemm as og, layout as ol, quant
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


@pytest.fixture
def num_sms():
    """set_num_sms for the test, restored to the device's CU count afterwards."""
    full = deep_gemm.get_num_sms()
    yield deep_gemm.set_num_sms
    deep_gemm.set_num_sms(full)


def _fp8_nt(m, n, k, seed, d_dtype=torch.bfloat16, bias=False):
    g = gen(seed)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    c = torch.randn(1, n, generator=g).to(torch.bfloat16) if bias else None
    args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()))
    ref = og.gemm_nt(a_deq, b_deq, d_dtype, bias=c)

    def run():
        d = torch.empty(m, n, dtype=d_dtype, device='cuda')
        deep_gemm.fp8_gemm_nt(*args, d, c=None if c is None else c.cuda(), recipe_a=(1, 128), recipe_b=(128, 128))
        torch.cuda.synchronize()
        return d.cpu()
    return run, ref


def test_set_num_sms_caps_the_grid(num_sms):
    m, n, k = 4096, 7168, 2048
    full = deep_gemm.launch_plan(m, n, k)
    assert full['persistent'] == 0 and full['grid'] == full['tiles']
    run, ref = _fp8_nt(m, n, k, seed=1)
    d_full = run()
    num_sms(64)
    capped = deep_gemm.launch_plan(m, n, k)
    print('full plan', full, 'capped plan', capped, flush=True)
    assert capped['grid'] == 64 < capped['tiles']
    d_cap = run()
    assert calc_diff(d_cap, ref) < THRESH
    if (capped['block_m'], capped['block_n']) == (full['block_m'], full['block_n']):
        assert torch.equal(d_cap, d_full)


@pytest.mark.parametrize('m,n,k,bias,d_dtype', [
    (4096, 7168, 2048, False, torch.bfloat16),     # the north-star shape, 512 tiles over 255 workgroups
    (1000, 1000, 1000, False, torch.bfloat16),     # ragged edges and a K tail
    (777, 2112, 7168, True, torch.bfloat16),       # bias
    (512, 640, 384, False, torch.float32),         # fp32 out, a single tile column
])
def test_persistent_dense(num_sms, m, n, k, bias, d_dtype):
    num_sms(255)
    plan = deep_gemm.launch_plan(m, n, k)
    print(f'persistent dense m={m} n={n} k={k} plan={plan}', flush=True)
    run, ref = _fp8_nt(m, n, k, seed=2, d_dtype=d_dtype, bias=bias)
    out = run()
    assert calc_diff(out, ref) < THRESH
    assert plan['grid'] <= 255
    if plan['persistent']:
        assert plan['grid'] == min(plan['tiles'], 255)


def test_persistent_bf16_and_fp8_fp4(num_sms):
    num_sms(200)
    m, n, k = 1024, 1792, 1024
    g = gen(3)
    a = (torch.randn(m, k, generator=g) * 0.1).to(torch.bfloat16)
    b = (torch.randn(n, k, generator=g) * 0.1).to(torch.bfloat16)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    print('persistent bf16 plan', deep_gemm.launch_plan(m, n, k, kind=3), flush=True)
    deep_gemm.bf16_gemm_nt(a.cuda(), b.cuda(), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a.float(), b.float())) < THRESH
    a8, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g)
    b4, sfb, b_deq = operand(n, k, 'e2m1', (1, 32), g)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_fp4_gemm_nt((a8.cuda(), sfa.cuda()), (b4.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq)) < THRESH


@pytest.mark.parametrize('psum', [True, False])
def test_persistent_m_grouped(num_sms, psum):
    """Padding-only tiles are written as zeros, valid rows match the oracle (alignment 256 lets
    the 256-row tiles serve the contiguous layout)."""
    num_sms(128)
    alignment = 256
    sizes = [700, 0, 256, 1, 513, 300]
    total, ps = ol.psum_from_sizes(sizes, alignment)
    total += 256                                    # trailing rows past the last group
    n, k = 1792, 1024
    g = gen(4)
    a, sfa, a_deq = operand(total, k, 'e4m3', (1, 32), g)
    for sl in ol.psum_pad_slices(ps, alignment):
        a.view(torch.uint8)[sl] = 0
        a_deq[sl] = 0
    a.view(torch.uint8)[-256:] = 0
    a_deq[-256:] = 0
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=len(sizes))
    if psum:
        layout_t = torch.tensor(ps, dtype=torch.int32)
    else:
        layout_t = ol.m_indices_from_psum(ps, alignment, total)
    d = torch.full((total, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        plan = deep_gemm.launch_plan(total, n, k, gemm_type=2 if psum else 3, num_groups=len(sizes))
        print(f'persistent m_grouped psum={psum} plan={plan}', flush=True)
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, layout_t.cuda(),
                                                   use_psum_layout=psum)
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    torch.cuda.synchronize()
    out = d.cpu()
    valid = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(ps, alignment):
        valid[sl] = True
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid]))
    ref = og.m_grouped_contiguous(a_deq, b_deq, layout_t, psum, alignment)
    assert calc_diff(out[valid], ref[valid]) < THRESH


def test_persistent_masked(num_sms):
    num_sms(96)
    gnum, max_m, n, k = 6, 512, 1792, 768
    g = gen(5)
    a, sfa, a_deq = operand(max_m, k, 'e4m3', (1, 32), g, batch=gnum)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=gnum)
    masked = torch.tensor([512, 0, 1, 300, 257, 256], dtype=torch.int32)
    d = torch.full((gnum, max_m, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    deep_gemm.m_grouped_fp8_gemm_nt_masked((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, masked.cuda(), 256)
    torch.cuda.synchronize()
    out = d.cpu()
    ref = og.m_grouped_masked(a_deq, b_deq, masked)
    for i in range(gnum):
        mg = int(masked[i])
        if mg:
            assert calc_diff(out[i, :mg], ref[i, :mg]) < THRESH, i
        assert torch.isnan(out[i, mg:].float()).all(), i


def test_persistent_batched(num_sms):
    num_sms(100)
    bsz, m, n, k = 3, 600, 1000, 512
    g = gen(6)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g, batch=bsz)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=bsz)
    d = torch.empty(bsz, m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_bmm((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.batched_nt(a_deq, b_deq)) < THRESH
