"""The shared-ring decode kernel (csrc/skinny_kernel.hpp, skinny_rows_kernel) on every configuration
of its menu, forced through the DG_SKINNY_ROWS tuning override ("mt,nb,d[,split[,reduce]]"; reduce = 1:
the split-K partials are summed by the second launch, split_reduce_kernel), against the CPU
oracle (calc_diff < 1e-5): ragged N (a partial last strip), K ending inside a 64-K block and inside
a group, K split across workgroups, every operand kind, fp32 accumulate and bias, batched and
masked launches, odd M / N (the scale rows are fetched as row-pair dwords), and the bit-exact
epilogues (stochastic rounding, FP8 output) against the same plan's fp32 / bf16 output.  The
heuristic picks this kernel by default for 64 < M <= 128 and K <= 8192; the default-path test
checks that choice against the tile kernel."""
import pytest
import torch

import deep_gemm
from oracle import gemm as og, epilogue as oe
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5
# the kSkinnyRows menu of csrc/gemm_tiles.hpp, plus forced K splits
CONFIGS = ['4,1,3', '4,1,4', '4,1,5', '4,2,4', '4,4,4', '2,1,4', '2,2,4', '2,4,4', '4,1,4,3', '2,2,4,5',
           '4,1,4,3,1', '4,2,4,6,1', '4,4,4,9,1', '2,4,4,4,1', '2,2,4,3,1']


def _ms(cfg):
    """M values for a configuration: one tile's rows and, below 128 rows a tile, M held in several
    tiles per strip (a ragged last one included)."""
    rows = 32 * int(cfg.split(',')[0])
    return sorted({1, rows - 3, rows} | ({rows + 37, 128} if rows < 128 else set()))


@pytest.fixture
def rows(monkeypatch):
    def _set(cfg):
        monkeypatch.setenv('DG_SKINNY_ROWS', cfg)
    return _set




@pytest.mark.parametrize('cfg', CONFIGS)
@pytest.mark.parametrize('kinds', [('e4m3', 'e4m3'), ('e4m3', 'e2m1'), ('e2m1', 'e2m1')])
def test_rows_kinds(rows, cfg, kinds):
    n, k = 500, 1040   # N: a partial last strip; K: 16 64-K blocks and a 16-element tail
    rows(cfg)
    g = gen(61)
    b, sfb, b_deq = operand(n, k, kinds[1], (1, 32), g)
    for m in _ms(cfg):
        print(f'rows {cfg} {kinds} m={m} n={n} k={k}', flush=True)
        a, sfa, a_deq = operand(m, k, kinds[0], (1, 32), g)
        out = torch.float32 if kinds[0] == 'e2m1' else torch.bfloat16
        d = torch.empty(m, n, dtype=out, device='cuda')
        deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
        torch.cuda.synchronize()
        assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq, out)) < THRESH


@pytest.mark.parametrize('cfg', CONFIGS)
@pytest.mark.parametrize('k', [64, 192, 7168])
def test_rows_fp8_accumulate_bias(rows, cfg, k):
    """fp32 D += A . B^T (c aliases d), then bf16 D with a bias row; the 1x128 / 128x128 recipe."""
    m, n = 32 * int(cfg.split(',')[0]) - 1, 230
    print(f'rows {cfg} fp8 accumulate/bias m={m} n={n} k={k}', flush=True)
    rows(cfg)
    g = gen(62)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, mode='randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, mode='randn')
    args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()))
    ref = og.gemm_nt(a_deq, b_deq, torch.float32)
    c = torch.randn(m, n, generator=g)
    d = c.clone().cuda()
    deep_gemm.fp8_gemm_nt(*args, d, c=d, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), ref + c) < THRESH
    bias = torch.randn(1, n, generator=g).bfloat16()
    d16 = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt(*args, d16, c=bias.cuda(), recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    assert calc_diff(d16.cpu(), ref + bias.float()) < THRESH


@pytest.mark.parametrize('cfg', CONFIGS)
def test_rows_bf16(rows, cfg):
    n, k = 300, 1000
    rows(cfg)
    g = gen(63)
    b = (torch.randn(n, k, generator=g) * 0.1).to(torch.bfloat16)
    for m in _ms(cfg):
        print(f'rows {cfg} bf16 m={m} n={n} k={k}', flush=True)
        a = (torch.randn(m, k, generator=g) * 0.1).to(torch.bfloat16)
        d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
        deep_gemm.bf16_gemm_nt(a.cuda(), b.cuda(), d)
        torch.cuda.synchronize()
        assert calc_diff(d.cpu(), og.gemm_nt(a.float(), b.float())) < THRESH


@pytest.mark.parametrize('cfg', ['4,1,4', '2,2,4,2', '4,4,4,3,1'])
def test_rows_bmm(rows, cfg):
    bs, m, n, k = 3, 57, 192, 640
    print(f'rows {cfg} bmm bs={bs} m={m} n={n} k={k}', flush=True)
    rows(cfg)
    g = gen(64)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g, 'randn', batch=bs)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, 'randn', batch=bs)
    d = torch.empty(bs, m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_bmm((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    for i in range(bs):
        assert calc_diff(d[i].cpu(), og.gemm_nt(a_deq[i], b_deq[i])) < THRESH


@pytest.mark.parametrize('cfg', ['4,1,4', '4,2,4,2', '4,4,4,5,1'])
def test_rows_epilogues_bit_exact(rows, cfg):
    """Stochastic rounding: bit-exact against the hash of the same plan's fp32 output; FP8 output:
    bit-exact against quantising its bf16 output per (row, 32 columns)."""
    bs, m, n, k = 2, 77, 256, 512
    print(f'rows {cfg} SR / FP8 output bs={bs} m={m} n={n} k={k}', flush=True)
    rows(cfg)
    g = gen(65)
    a, sfa, _ = operand(m, k, 'e4m3', (1, 32), g, 'randn')
    b, sfb, _ = operand(n, k, 'e4m3', (1, 32), g, 'randn')
    args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()))
    f32 = torch.empty(m, n, device='cuda')
    deep_gemm.fp8_gemm_nt(*args, f32)
    out = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt(*args, out, epilogue=deep_gemm.epilogue.BF16StochasticRounding())
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().view(torch.int16), oe.stochastic_round_bf16(f32).cpu().view(torch.int16))

    a3, sfa3, _ = operand(m, k, 'e4m3', (1, 32), g, 'randn', batch=bs)
    b3, sfb3, _ = operand(n, k, 'e4m3', (1, 32), g, 'randn', batch=bs)
    args3 = ((a3.cuda(), sfa3.cuda()), (b3.cuda(), sfb3.cuda()))
    d_bf16 = torch.empty(m, bs, n, dtype=torch.bfloat16, device='cuda').transpose(0, 1)
    deep_gemm.fp8_bmm(*args3, d_bf16)
    fp8 = torch.empty(m, bs, n, dtype=torch.float8_e4m3fn, device='cuda').transpose(0, 1)
    sfd = torch.empty_strided((m, bs * n // 64), (1, m), device='cuda', dtype=torch.int16)
    deep_gemm.fp8_bmm(*args3, fp8, epilogue=deep_gemm.epilogue.FP8Quantization(sfd))
    torch.cuda.synchronize()
    ref_fp8, ref_sfd = oe.quantize_fp8_output(d_bf16.transpose(0, 1).cpu().reshape(m, bs * n))
    assert torch.equal(fp8.transpose(0, 1).cpu().view(torch.uint8).reshape(m, bs * n), ref_fp8.view(torch.uint8))
    assert torch.equal(sfd.cpu(), ref_sfd)


@pytest.mark.parametrize('m,n,k', [(128, 2112, 7168), (128, 4096, 7168), (128, 7168, 2048), (65, 4096, 1024),
                                   (100, 300, 7168), (128, 24576, 1536), (96, 3072, 7168), (128, 7168, 7168),
                                   (128, 7168, 16384), (96, 3072, 12288)])
def test_rows_default_plan_vs_tile_kernel(monkeypatch, m, n, k):
    """The heuristic's decode plans for 64 < M <= 128 agree with the tile kernel (DG_SKINNY=0) and
    with the oracle; the BASELINE decode shapes take the shared-ring kernel."""
    print(f'rows default plan m={m} n={n} k={k}', flush=True)
    g = gen(66)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()))
    if n <= 8192:
        info = deep_gemm.launch_plan(m, n, k)
        wide = k > 4096 and n >= 3072   # 64-column strips, partials summed by the second launch
        wide128 = wide and k >= 8192 and n >= 7168   # (e4m3: 128-column strips from K = 8192 over N >= 7168)
        # (64 x 64 tiles from M = 81 on, else 128-row strips: 128 x 64 where wide, 128 x 32 otherwise)
        bm, bn = (128, 128) if wide128 else (128, 64) if wide else (64, 64) if m > 80 else (128, 32)
        assert info['skinny'] == 2 and (info['block_m'], info['block_n']) == (bm, bn), info
        assert info['split_reduce'] == int(wide or (m > 80 and info['split_k'] > 2)), info
        assert info['split_k'] > 1 or not wide, info
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt(*args, d, recipe_a=(1, 128), recipe_b=(128, 128))
    monkeypatch.setenv('DG_SKINNY', '0')
    d0 = torch.empty_like(d)
    deep_gemm.fp8_gemm_nt(*args, d0, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq)) < THRESH
    assert calc_diff(d.cpu(), d0.cpu()) < 1e-6


@pytest.mark.parametrize('cfg', ['4,1,4', '2,1,4', '4,2,4,2', '4,4,4,3,1'])
@pytest.mark.parametrize('max_m,n,k', [(128, 384, 1024), (64, 300, 1040)])
def test_rows_masked(monkeypatch, cfg, max_m, n, k):
    """M-grouped masked launches on forced configurations: valid rows match the oracle, rows past
    masked_m keep their previous contents, empty groups write nothing."""
    if max_m > 32 * int(cfg.split(',')[0]):
        pytest.skip('configuration holds fewer rows than max_m')
    monkeypatch.setenv('DG_SKINNY_ROWS', cfg)
    print(f'rows masked {cfg} max_m={max_m} n={n} k={k}', flush=True)
    groups = 6
    g = gen(67)
    a, sfa, a_deq = operand(max_m, k, 'e4m3', (1, 32), g, batch=groups)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=groups)
    masked = torch.tensor([max_m, 0, 1, max_m // 2, 3, max_m - 1], dtype=torch.int32)
    sentinel = torch.full((groups, max_m, n), 7.0).bfloat16()
    d = sentinel.clone().cuda()
    deep_gemm.m_grouped_fp8_gemm_nt_masked((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, masked.cuda(), max_m)
    torch.cuda.synchronize()
    out = d.cpu()
    for i in range(groups):
        mg = int(masked[i])
        if mg:
            assert calc_diff(out[i, :mg], og.gemm_nt(a_deq[i, :mg], b_deq[i])) < THRESH, i
        assert torch.equal(out[i, mg:], sentinel[i, mg:]), i


@pytest.mark.parametrize('cfg', ['4,1,4', '2,2,4', '4,1,3,3'])
@pytest.mark.parametrize('m,n,k', [(3, 257, 320), (33, 99, 1088), (127, 501, 64), (97, 33, 4160)])
def test_rows_odd_shapes(rows, cfg, m, n, k):
    """Odd M and N: the packed scale rows are fetched as row-pair dwords, so the last row's pair
    partner lies past the operand (inside the even SF leading dimension) and must not leak in."""
    if m > 32 * int(cfg.split(',')[0]):
        pytest.skip('configuration holds fewer rows than M')
    print(f'rows {cfg} odd m={m} n={n} k={k}', flush=True)
    rows(cfg)
    g = gen(68)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g, 'randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, 'randn')
    d = torch.empty(m, n, dtype=torch.float32, device='cuda')
    deep_gemm.fp8_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq, torch.float32)) < THRESH


def test_rows_split_back_to_back_bit_exact(monkeypatch):
    """A split-K launch repeated back to back (the arrival counters reset by each launch) gives the
    same bits as an isolated one."""
    m, n, k = 128, 2112, 7168
    monkeypatch.setenv('DG_SKINNY_ROWS', '4,1,4,3')
    g = gen(69)
    a, sfa, _ = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, _ = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()))
    d0 = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt(*args, d0, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    outs = [torch.empty_like(d0) for _ in range(8)]
    for o in outs:
        deep_gemm.fp8_gemm_nt(*args, o, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), d0.view(torch.int16))


@pytest.mark.parametrize('cfg', ['4,1,4,3', '4,2,4,6', '4,4,4,9', '2,4,4,4'])
@pytest.mark.parametrize('out', [torch.float32, torch.bfloat16])
def test_rows_split_reduce_launch_bit_exact(monkeypatch, cfg, out):
    """The second-launch reduction (split_reduce_kernel) sums the same partials in the same split
    order as the first launch's last-arriving workgroup: bit-identical D, fp32 and bf16, on a
    ragged N and a K that ends inside a 64-K block; launch_plan reports which path runs."""
    mt = int(cfg.split(',')[0])
    m, n, k = 32 * mt - 5, 1000, 7000
    print(f'rows split reduce {cfg} m={m} n={n} k={k} {out}', flush=True)
    g = gen(70)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()))
    res = {}
    for reduce in (0, 1):
        monkeypatch.setenv('DG_SKINNY_ROWS', f'{cfg},{reduce}')
        info = deep_gemm.launch_plan(m, n, k)
        assert info['split_k'] == int(cfg.split(',')[3]) and info['split_reduce'] == reduce, info
        d = torch.empty(m, n, dtype=out, device='cuda')
        deep_gemm.fp8_gemm_nt(*args, d, recipe_a=(1, 128), recipe_b=(128, 128))
        torch.cuda.synchronize()
        res[reduce] = d.cpu()
    bits = torch.int32 if out == torch.float32 else torch.int16
    assert torch.equal(res[0].view(bits), res[1].view(bits))
    assert calc_diff(res[1], og.gemm_nt(a_deq, b_deq, out)) < THRESH


@pytest.mark.parametrize('kind', ['bf16', 'fp4'])
@pytest.mark.parametrize('m,n,k', [(128, 2112, 7168), (128, 4096, 7168), (128, 7168, 2048), (96, 7168, 4096), (72, 1000, 2048),
                                   (96, 7168, 12288), (128, 3072, 8192), (128, 7168, 16384)])
def test_rows_default_plan_bf16_fp4(monkeypatch, kind, m, n, k):
    """bf16 and FP8 x FP4 decode shapes on their default plans (the shared-ring kernel where it measured
    ahead, the skinny kernel elsewhere) agree with the oracle and with the tile kernel."""
    g = gen(73)
    if kind == 'bf16':
        a = (torch.randn(m, k, generator=g) * 0.1).bfloat16()
        b = (torch.randn(n, k, generator=g) * 0.1).bfloat16()
        ref = og.gemm_nt(a.float(), b.float())
        call = lambda d: deep_gemm.bf16_gemm_nt(a.cuda(), b.cuda(), d)
        info = deep_gemm.launch_plan(m, n, k, kind=deep_gemm._lib.DG_KIND_BF16)
    else:
        a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g, 'randn')
        b, sfb, b_deq = operand(n, k, 'e2m1', (1, 32), g)
        ref = og.gemm_nt(a_deq, b_deq)
        call = lambda d: deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
        info = deep_gemm.launch_plan(m, n, k, kind=deep_gemm._lib.DG_KIND_FP8_FP4)
    print(f'rows default {kind} m={m} n={n} k={k} plan={info}', flush=True)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    call(d)
    monkeypatch.setenv('DG_SKINNY', '0')
    d0 = torch.empty_like(d)
    call(d0)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), ref) < THRESH
    assert calc_diff(d.cpu(), d0.cpu()) < 1e-6


@pytest.mark.parametrize('m,n,k', [(100, 2112, 2048), (128, 4096, 7168), (97, 3000, 5000), (128, 7168, 8192)])
def test_rows_default_plan_bmm(m, n, k):
    """Batched launches on the default decode plans (64 x 64 tiles with M in two row blocks, or the 128 x 64
    two-launch plan): every batch against the oracle."""
    bs = 3
    print(f'rows default bmm bs={bs} m={m} n={n} k={k}', flush=True)
    g = gen(74)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g, 'randn', batch=bs)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, 'randn', batch=bs)
    d = torch.empty(bs, m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_bmm((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    for i in range(bs):
        assert calc_diff(d[i].cpu(), og.gemm_nt(a_deq[i], b_deq[i])) < THRESH, i
