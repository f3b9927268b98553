"""set_num_sms as a CU cap on every kernel family: under set_num_sms(n) the launch holds at most n
workgroups (the reference launches num_cores blocks, csrc/jit_kernels/heuristics.hpp:98, and
csrc/apis/runtime.hpp:17-19 sets that count), each serving the plan's workgroups b, b + grid, ...
in turn, and D matches the CPU oracle (calc_diff < 1e-5, the reference's bar,
tests/test_fp8_gemm.py:21; padding rows of grouped layouts exact zeros).

Families: the 128-K-stage tiles (256x224 persistent, 256x256 and 256x160 walking the virtual grid),
the 64-K-stage tiles (128x128, 64x128), split-K tile launches, the decode kernels (skinny,
shared-ring, GEMV), the anchored M-grouped tiles (psum and m_indices), masked, batched,
MN-major operands read in place and K-grouped."""
import os

import pytest
import torch

import deep_gemm
from deep_gemm import _lib
from oracle import gemm as og, layout as ol
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


@pytest.fixture
def cap():
    """set_num_sms(n) for the test; the device's CU count and the tuning variables restored after."""
    full = deep_gemm.get_num_sms()
    saved = {k: os.environ.get(k) for k in ('DG_FORCE_BLOCK', 'DG_SPLIT_K')}

    def set_cap(n, block=None, split=None):
        deep_gemm.set_num_sms(n)
        for key, val in (('DG_FORCE_BLOCK', block), ('DG_SPLIT_K', split)):
            if val is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = str(val)
    yield set_cap
    deep_gemm.set_num_sms(full)
    for key, val in saved.items():
        if val is None:
            os.environ.pop(key, None)
        else:
            os.environ[key] = val


def _dense(m, n, k, seed, b_kind='e4m3'):
    g = gen(seed)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g)
    b, sfb, b_deq = operand(n, k, b_kind, (1, 32), g)
    return (a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), og.gemm_nt(a_deq, b_deq)


@pytest.mark.parametrize('n_cus,m,n,k,block,split,kind', [
    (64, 4096, 7168, 2048, None, None, 'tile 256x224 (persistent)'),
    (48, 2048, 2048, 1024, '256x256', None, 'tile 256x256'),
    (40, 1024, 2112, 1024, '256x160', None, 'tile 256x160'),
    (32, 1000, 1000, 1000, '128x128', None, 'tile 128x128'),
    (30, 300, 1000, 640, '64x128', None, 'tile 64x128'),
    (24, 256, 1024, 4096, '64x128', 4, 'tile 64x128 split 4'),
    (16, 16, 7168, 2048, None, None, 'skinny'),
    (40, 128, 2112, 7168, None, None, 'shared-ring decode'),
    (100, 128, 1024, 7168, None, None, 'shared-ring two-launch 64x64'),
    (160, 128, 3072, 7168, None, None, 'shared-ring two-launch 128x64'),
    (20, 1, 2112, 7168, None, None, 'decode GEMV'),
    (12, 1, 4096, 4096, None, 3, 'skinny split 3'),
])
def test_cap_dense_families(cap, n_cus, m, n, k, block, split, kind):
    cap(n_cus, block, split)
    plan = deep_gemm.launch_plan(m, n, k, split_k=split or 0)
    print(f'cu cap {n_cus} {kind} m={m} n={n} k={k} plan={plan}', flush=True)
    assert plan['grid'] <= n_cus
    assert plan['plan_workgroups'] >= plan['grid']
    if kind == 'decode GEMV':
        assert plan['skinny'] == 3
    elif kind == 'shared-ring decode':
        assert plan['skinny'] == 2
    elif kind.startswith('shared-ring two-launch'):
        # (the second launch's workgroups go out in chunks of at most n_cus as well)
        assert plan['skinny'] == 2 and plan['split_reduce'] == 1 and plan['split_k'] >= 3, plan
    elif kind.startswith('skinny'):
        assert plan['skinny'] == 1
    elif block is not None:
        assert f"{plan['block_m']}x{plan['block_n']}" == block
    if split:
        assert plan['split_k'] == split
    a, b, ref = _dense(m, n, k, seed=m + n + k)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt(a, b, d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), ref) < THRESH


def test_cap_bf16_and_fp8_fp4(cap):
    cap(50)
    m, n, k = 1024, 1792, 1024
    g = gen(11)
    a = (torch.randn(m, k, generator=g) * 0.1).to(torch.bfloat16)
    b = (torch.randn(n, k, generator=g) * 0.1).to(torch.bfloat16)
    for kind in (3, 1):
        plan = deep_gemm.launch_plan(m, n, k, kind=kind)
        print('cu cap 50 kind', kind, plan, flush=True)
        assert plan['grid'] <= 50
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.bf16_gemm_nt(a.cuda(), b.cuda(), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a.float(), b.float())) < THRESH
    a8, b4, ref = _dense(m, n, k, seed=12, b_kind='e2m1')
    deep_gemm.fp8_fp4_gemm_nt(a8, b4, d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), ref) < THRESH


@pytest.mark.parametrize('psum', [True, False])
def test_cap_anchored_m_grouped(cap, psum):
    """Alignment 128: 384x192 tiles anchored at each group's (run's) first row; the plan's upper
    bound of workgroups is walked by at most n_cus of them."""
    cap(36)
    alignment, n, k = 128, 576, 512
    sizes = [257, 0, 130, 400, 5]
    total, ps = ol.psum_from_sizes(sizes, alignment)
    g = gen(13)
    a, sfa, a_deq = operand(total, k, 'e4m3', (1, 32), g)
    for sl in ol.psum_pad_slices(ps, alignment):
        a.view(torch.uint8)[sl] = 0
        a_deq[sl] = 0
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=len(sizes))
    layout_t = torch.tensor(ps, dtype=torch.int32) if psum else ol.m_indices_from_psum(ps, alignment, total)
    d = torch.full((total, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        plan = deep_gemm.launch_plan(total, n, k, gemm_type=2 if psum else 3, num_groups=len(sizes))
        print(f'cu cap 36 anchored psum={psum} plan={plan}', flush=True)
        assert (plan['block_m'], plan['block_n']) == (384, 192) and plan['grid'] <= 36
        assert plan['persistent'] == 1   # the anchored tiles' walk kernel
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, layout_t.cuda(),
                                                   use_psum_layout=psum)
        torch.cuda.synchronize()
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    out = d.cpu()
    valid = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(ps, alignment):
        valid[sl] = True
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid]))
    ref = og.m_grouped_contiguous(a_deq, b_deq, layout_t, psum, alignment)
    assert calc_diff(out[valid], ref[valid]) < THRESH


@pytest.mark.parametrize('psum', [True, False])
def test_cap_anchored_m_grouped_bf16(cap, psum):
    """The bf16 anchored tiles' walk kernel under a cap (psum and m_indices, an empty group)."""
    cap(44)
    alignment, n, k = 128, 768, 1024
    sizes = [300, 0, 129, 77, 512, 1]
    total, ps = ol.psum_from_sizes(sizes, alignment)
    g = gen(17)
    a = (torch.randn(total, k, generator=g) * 0.1).to(torch.bfloat16)
    for sl in ol.psum_pad_slices(ps, alignment):
        a[sl] = 0
    b = (torch.randn(len(sizes), n, k, generator=g) * 0.1).to(torch.bfloat16)
    layout_t = torch.tensor(ps, dtype=torch.int32) if psum else ol.m_indices_from_psum(ps, alignment, total)
    d = torch.full((total, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        plan = deep_gemm.launch_plan(total, n, k, kind=3, gemm_type=2 if psum else 3, num_groups=len(sizes))
        print(f'cu cap 44 anchored bf16 psum={psum} plan={plan}', flush=True)
        assert plan['grid'] <= 44
        deep_gemm.m_grouped_bf16_gemm_nt_contiguous(a.cuda(), b.cuda(), d, layout_t.cuda(), use_psum_layout=psum)
        torch.cuda.synchronize()
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    out = d.cpu()
    valid = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(ps, alignment):
        valid[sl] = True
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid]))
    ref = og.m_grouped_contiguous(a.float(), b.float(), layout_t, psum, alignment)
    assert calc_diff(out[valid], ref[valid]) < THRESH


def test_cap_masked_and_batched(cap):
    cap(20)
    gnum, max_m, n, k = 4, 256, 640, 512
    g = gen(14)
    a, sfa, a_deq = operand(max_m, k, 'e4m3', (1, 32), g, batch=gnum)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=gnum)
    masked = torch.tensor([256, 0, 17, 129], dtype=torch.int32)
    plan = deep_gemm.launch_plan(max_m, n, k, gemm_type=4, num_groups=gnum)
    print('cu cap 20 masked', plan, flush=True)
    assert plan['grid'] <= 20
    d = torch.full((gnum, max_m, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    deep_gemm.m_grouped_fp8_gemm_nt_masked((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, masked.cuda(), 128)
    torch.cuda.synchronize()
    out = d.cpu()
    ref = og.m_grouped_masked(a_deq, b_deq, masked)
    for i in range(gnum):
        mg = int(masked[i])
        if mg:
            assert calc_diff(out[i, :mg], ref[i, :mg]) < THRESH, i
    plan = deep_gemm.launch_plan(max_m, n, k, gemm_type=1, num_groups=gnum)
    print('cu cap 20 batched', plan, flush=True)
    assert plan['grid'] <= 20
    d = torch.empty(gnum, max_m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_bmm((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.batched_nt(a_deq, b_deq)) < THRESH


def test_cap_mn_major_in_place(cap):
    """fp8_gemm_tn: MN-major A and B read in place by the 128-K-stage tiles (no copy), capped."""
    cap(28)
    m, n, k = 1024, 1536, 1024
    g = gen(15)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    a_t = a.view(torch.uint8).t().contiguous().view(torch.float8_e4m3fn).cuda()   # [K, M], M contiguous
    b_t = b.view(torch.uint8).t().contiguous().view(torch.float8_e4m3fn).cuda()   # [K, N], N contiguous
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_tn((a_t, sfa.cuda().t()), (b_t, sfb.cuda().t()), d, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq)) < THRESH


def test_cap_k_grouped(cap):
    """K-grouped wgrad (MN-major A and B read in place), capped."""
    from test_batched_kgrouped_gpu import _k_grouped_case
    cap(24)
    g_, m, n, ks = 3, 512, 768, [384, 0, 700]
    psum, a_tn, sfa, a_deq, b_tn, sfb, b_deq = _k_grouped_case(m, n, ks, seed=16)
    print(f'cu cap 24 k-grouped G={g_} m={m} n={n} ks={ks}', flush=True)
    d = torch.full((g_, m, n), float('nan'), dtype=torch.float32, device='cuda')
    layout = torch.tensor(psum, dtype=torch.int32, device='cuda')
    deep_gemm.k_grouped_fp8_gemm_tn_contiguous((a_tn.cuda(), sfa.cuda()), (b_tn.cuda(), sfb.cuda()), d, ks, layout)
    torch.cuda.synchronize()
    ref = og.k_grouped_tn(a_deq, b_deq, psum, 256, None, torch.float32)
    dc = d.cpu()
    for gi in range(g_):
        if ks[gi] == 0:
            assert torch.equal(dc[gi], ref[gi]), gi
        else:
            assert calc_diff(dc[gi], ref[gi]) < THRESH, gi
