"""Every tile shape of the kernel menu, forced through the DG_FORCE_BLOCK tuning override, on
ragged problems (M, N not multiples of the tile, K ending inside a 128-K stage) for every operand
kind, against the CPU oracle (calc_diff < 1e-5; M-grouped padding rows bit-exact 0).  The
heuristic alone would only ever reach the large tiles on large problems."""
import pytest
import torch

import deep_gemm
from oracle import gemm as og, layout as ol
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5
# the menu compiled into libdeep_gemm_amd.so (csrc/gemm_tiles.hpp)
TILES = ['256x256', '256x224', '256x160', '256x128', '128x256', '128x128', '64x128', '32x128']


@pytest.fixture
def force(monkeypatch):
    def _set(tile):
        monkeypatch.setenv('DG_FORCE_BLOCK', tile)
    return _set


@pytest.mark.parametrize('tile', TILES)
@pytest.mark.parametrize('kinds', [('e4m3', 'e4m3'), ('e4m3', 'e2m1'), ('e2m1', 'e2m1')])
def test_tile_fp8_fp4(force, tile, kinds):
    m, n, k = 300, 500, 832
    print(f'tile {tile} {kinds} m={m} n={n} k={k}', flush=True)
    force(tile)
    g = gen(21)
    a, sfa, a_deq = operand(m, k, kinds[0], (1, 32), g)
    b, sfb, b_deq = operand(n, k, kinds[1], (1, 32), g)
    out = torch.float32 if kinds[0] == 'e2m1' else torch.bfloat16
    d = torch.empty(m, n, dtype=out, device='cuda')
    deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq, out)) < THRESH


@pytest.mark.parametrize('tile', TILES)
def test_tile_fp8_accumulate(force, tile):
    """fp32 D += A . B^T (c aliases d) with a K of one 64-K step past a 128-K stage."""
    m, n, k = 257, 230, 192
    print(f'tile {tile} fp8 accumulate m={m} n={n} k={k}', flush=True)
    force(tile)
    g = gen(22)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, mode='randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, mode='randn')
    c = torch.randn(m, n, generator=g)
    d = c.clone().cuda()
    deep_gemm.fp8_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, c=d, recipe_a=(1, 128),
                          recipe_b=(128, 128))
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq, torch.float32) + c) < THRESH


@pytest.mark.parametrize('tile', TILES)
def test_tile_bf16(force, tile):
    m, n, k = 300, 500, 200
    print(f'tile {tile} bf16 m={m} n={n} k={k}', flush=True)
    force(tile)
    g = gen(23)
    a = (torch.randn(m, k, generator=g) * 0.1).to(torch.bfloat16)
    b = (torch.randn(n, k, generator=g) * 0.1).to(torch.bfloat16)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.bf16_gemm_nt(a.cuda(), b.cuda(), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a.float(), b.float())) < THRESH


@pytest.mark.parametrize('tile', ['256x256', '256x224', '256x160', '256x128', '128x128'])
def test_tile_m_grouped(force, tile):
    """psum layout, alignment 256: padding rows exact zeros, valid rows per group's B."""
    counts, n, k = [300, 0, 129], 448, 640
    print(f'tile {tile} m-grouped counts={counts} n={n} k={k}', flush=True)
    force(tile)
    align = 256
    psum, total = [], 0
    for cnt in counts:
        psum.append(total + cnt)
        total = -(-(total + cnt) // align) * align
    g = gen(24)
    a, sfa, a_deq = operand(total, k, 'e4m3', (1, 32), g)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=len(counts))
    layout = torch.tensor(psum, dtype=torch.int32)
    d = torch.empty(total, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.set_mk_alignment_for_contiguous_layout(align)
    try:
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d,
                                                   layout.cuda())
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(256)
    torch.cuda.synchronize()
    out = d.cpu()
    start = 0
    for gi, end in enumerate(psum):
        if end > start:
            ref = og.gemm_nt(a_deq[start:end], b_deq[gi])
            assert calc_diff(out[start:end], ref) < THRESH
        nxt = -(-end // align) * align
        assert torch.count_nonzero(out[end:nxt]) == 0
        start = nxt
