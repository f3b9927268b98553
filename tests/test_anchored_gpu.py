"""GPU parity of the anchored tiles of M-grouped GEMMs (csrc/gemm_kernel.hpp, anchored_tile):
tiles of 384 rows that start at each group's (psum) or run's (m_indices) first row, so the tile
height need not divide the alignment.  Valid rows match the oracle (calc_diff < 1e-5, the reference's bar,
tests/test_fp8_gemm.py:21), the padding rows of every group and the rows past the last group are
exact zeros, and nothing outside D's rows is written (a NaN canary row after D)."""
import os

import pytest
import torch

import deep_gemm
from oracle import gemm as og, layout as ol
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


@pytest.mark.parametrize('block', ['384x192', '384x128'])
@pytest.mark.parametrize('sizes,alignment,trailing', [
    ([257, 240, 0, 272, 1, 384, 385, 900], 128, 0),     # typical MoE counts, an empty group, multi-chunk groups
    ([100, 50, 300], 32, 64),                            # alignment 32, rows past the last group
    ([700, 0, 256, 1, 513, 300], 256, 256),             # alignment 256
    ([5], 128, 0),                                       # one tiny group
])
def test_anchored_m_grouped(monkeypatch, block, sizes, alignment, trailing):
    print(f'anchored {block} sizes={sizes} alignment={alignment} trailing={trailing}', flush=True)
    monkeypatch.setenv('DG_FORCE_BLOCK', block)
    total, ps = ol.psum_from_sizes(sizes, alignment)
    total += trailing
    n, k = 448, 1024
    g = gen(sum(sizes) + alignment)
    a, sfa, a_deq = operand(total, k, 'e4m3', (1, 32), g)
    for sl in ol.psum_pad_slices(ps, alignment):
        a.view(torch.uint8)[sl] = 0
        a_deq[sl] = 0
    if trailing:
        a.view(torch.uint8)[-trailing:] = 0
        a_deq[-trailing:] = 0
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=len(sizes))
    layout_t = torch.tensor(ps, dtype=torch.int32)
    out_full = torch.full((total + 1, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    d = out_full[:total]
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        plan = deep_gemm.launch_plan(total, n, k, gemm_type=2, num_groups=len(sizes))
        print('plan', plan, flush=True)
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, layout_t.cuda())
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    torch.cuda.synchronize()
    res = out_full.cpu()
    assert torch.isnan(res[total].float()).all(), 'wrote past D'
    out = res[:total]
    valid = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(ps, alignment):
        valid[sl] = True
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid])), 'padding rows must be exact zeros'
    ref = og.m_grouped_contiguous(a_deq, b_deq, layout_t, True, alignment)
    assert calc_diff(out[valid], ref[valid]) < THRESH


def test_anchored_m_grouped_bf16():
    """bf16 operands take the same anchored tiles (the default plan at alignment 128)."""
    alignment = 128
    sizes = [257, 0, 130, 400, 1]
    total, ps = ol.psum_from_sizes(sizes, alignment)
    n, k = 320, 512
    g = gen(11)
    a = (torch.randn(total, k, generator=g) * 0.1).to(torch.bfloat16)
    for sl in ol.psum_pad_slices(ps, alignment):
        a[sl] = 0
    b = (torch.randn(len(sizes), n, k, generator=g) * 0.1).to(torch.bfloat16)
    layout_t = torch.tensor(ps, dtype=torch.int32)
    d = torch.full((total, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        plan = deep_gemm.launch_plan(total, n, k, kind=3, gemm_type=2, num_groups=len(sizes))
        print('bf16 anchored plan', plan, flush=True)
        assert (plan['block_m'], plan['block_n']) == (384, 192)
        deep_gemm.m_grouped_bf16_gemm_nt_contiguous(a.cuda(), b.cuda(), d, layout_t.cuda())
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    torch.cuda.synchronize()
    out = d.cpu()
    valid = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(ps, alignment):
        valid[sl] = True
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid]))
    ref = og.m_grouped_contiguous(a.float(), b.float(), layout_t, True, alignment)
    assert calc_diff(out[valid], ref[valid]) < THRESH


def _runs_layout(blocks, alignment, fill):
    """m_indices from a list of (group, rows) alignment blocks in the given order (rows < alignment:
    the rest of the block is -1 padding)."""
    idx = []
    for grp, rows in blocks:
        idx += [grp] * rows + [-1] * (alignment - rows)
    return torch.tensor(idx, dtype=torch.int32)


@pytest.mark.parametrize('case', ['sorted', 'unsorted', 'split_group', 'padding_blocks'])
def test_anchored_m_indices(case):
    """m_indices layouts: the run table (csrc/status.hip) drives the anchored tiles whether groups
    are sorted, out of order, split into several runs, or separated by padding-only blocks."""
    alignment, g_num = 128, 4
    if case == 'sorted':
        blocks = [(0, 128), (0, 128), (0, 1), (1, 100), (2, 128), (2, 128), (2, 128), (2, 128), (3, 5)]
    elif case == 'unsorted':
        blocks = [(3, 128), (3, 7), (0, 128), (2, 64), (1, 128), (1, 128), (1, 128), (1, 2)]
    elif case == 'split_group':
        blocks = [(1, 128), (1, 30), (0, 128), (1, 128), (1, 128), (1, 128), (1, 17), (2, 90)]
    else:
        blocks = [(-1, 0), (0, 128), (0, 60), (-1, 0), (-1, 0), (3, 128), (3, 128), (3, 128), (3, 128), (-1, 0)]
    idx = _runs_layout(blocks, alignment, -1)
    total = idx.numel()
    n, k = 448, 512
    g = gen(len(blocks) * 7 + alignment)
    a, sfa, a_deq = operand(total, k, 'e4m3', (1, 32), g)
    pad = idx < 0
    a.view(torch.uint8)[pad] = 0
    a_deq[pad] = 0
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=g_num)
    d = torch.full((total, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        plan = deep_gemm.launch_plan(total, n, k, gemm_type=3, num_groups=g_num)
        print(f'anchored m_indices {case} plan={plan}', flush=True)
        assert (plan['block_m'], plan['block_n']) == (384, 192)
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, idx.cuda(),
                                                   use_psum_layout=False)
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    torch.cuda.synchronize()
    from deep_gemm import _lib
    assert _lib.load().dg_take_errors() == 0, 'a valid m_indices layout must not be reported'
    out = d.cpu()
    assert torch.equal(out[pad], torch.zeros_like(out[pad])), 'padding rows must be exact zeros'
    ref = og.m_grouped_contiguous(a_deq, b_deq, idx, False, alignment)
    assert calc_diff(out[~pad], ref[~pad]) < THRESH



@pytest.mark.parametrize('psum', [True, False])
def test_anchored_m_grouped_fp8_fp4(psum):
    """FP8 x FP4 (e2m1 B, 1x32 scales) M-grouped layouts below alignment 256 take the 384x128 anchored tiles on
    their default plan: valid rows match the oracle, padding rows are exact zeros, nothing is written past D."""
    sizes, alignment = [257, 240, 0, 272, 1, 384, 385, 900], 128
    total, ps = ol.psum_from_sizes(sizes, alignment)
    n, k = 448, 1024
    g = gen(81 + psum)
    a, sfa, a_deq = operand(total, k, 'e4m3', (1, 32), g)
    for sl in ol.psum_pad_slices(ps, alignment):
        a.view(torch.uint8)[sl] = 0
        a_deq[sl] = 0
    b, sfb, b_deq = operand(n, k, 'e2m1', (1, 32), g, batch=len(sizes))
    layout_t = torch.tensor(ps, dtype=torch.int32)
    idx = ol.m_indices_from_psum(ps, alignment, total)
    out_full = torch.full((total + 1, n), float('nan'), dtype=torch.bfloat16, device='cuda')
    d = out_full[:total]
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(alignment)
    try:
        plan = deep_gemm.launch_plan(total, n, k, kind=1, gemm_type=2 if psum else 3, num_groups=len(sizes))
        print(f'anchored fp8xfp4 psum={psum} plan={plan}', flush=True)
        assert (plan['block_m'], plan['block_n']) == (384, 128), plan
        deep_gemm.m_grouped_fp8_fp4_gemm_nt_contiguous((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d,
                                                       (layout_t if psum else idx).cuda(), use_psum_layout=psum)
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    torch.cuda.synchronize()
    res = out_full.cpu()
    assert torch.isnan(res[total].float()).all(), 'wrote past D'
    out = res[:total]
    valid = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(ps, alignment):
        valid[sl] = True
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid])), 'padding rows must be exact zeros'
    ref = og.m_grouped_contiguous(a_deq, b_deq, layout_t, True, alignment)
    assert calc_diff(out[valid], ref[valid]) < THRESH
