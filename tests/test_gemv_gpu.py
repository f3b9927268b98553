"""The decode GEMV kernel (csrc/gemv_kernel.hip: e4m3 x e4m3, M <= 4, whole rows of B per wave)
against the CPU oracle (calc_diff < 1e-5): the plan it takes at the BASELINE decode shapes, every
M it serves (1..4), ragged N (a workgroup's last rows past N), K ending inside a 1024-K step and
inside a 64-K block, rows per wave forced through DG_GEMV, fp32 accumulate and bias, batched
launches, both scale recipes, and agreement with the MFMA decode kernel (DG_GEMV=0) on the same
inputs."""
import pytest
import torch

import deep_gemm
from oracle import gemm as og
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


@pytest.mark.parametrize('m,n,k,ks', [(1, 2112, 7168, ''), (1, 7168, 16384, '8'), (1, 4096, 7168, ''),
                                      (1, 24576, 1536, '2'), (1, 7168, 2048, '2'), (2, 4096, 7168, '4'),
                                      (4, 7168, 2048, '2')])
def test_gemv_plan_and_parity_baseline_shapes(monkeypatch, m, n, k, ks):
    """BASELINE config-2 decode shapes through the GEMV kernel (the default plan at M = 1, 4096 <= K <= 8192;
    forced with DG_GEMV elsewhere), D against the oracle (N(0,1) data, 1x128 / 128x128 recipe)."""
    monkeypatch.setenv('DG_GEMV', ks)
    plan = deep_gemm.launch_plan(m, n, k)
    print(f'gemv baseline m={m} n={n} k={k} ks={ks!r} plan={plan}', flush=True)
    assert plan['skinny'] == 3 and plan['split_k'] == 1
    g = gen(m * 7 + n + k)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, mode='randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, mode='randn')
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq, torch.bfloat16)) < THRESH


@pytest.mark.parametrize('ks', ['', '1', '2', '8', '2,4', '4,4'])
@pytest.mark.parametrize('n,k', [(500, 1040), (130, 64), (77, 3000), (1000, 9216)])
def test_gemv_ragged_codes(monkeypatch, ks, n, k):
    """Random e4m3 codes with per-32 power-of-two scales; every M the kernel serves; the K split
    between a workgroup's waves forced to 1, 2 and 8 (DG_GEMV; "2,4" and "4,4" with four-wave workgroups) or
    the heuristic's."""
    if ks:
        monkeypatch.setenv('DG_GEMV', ks)
    else:
        monkeypatch.delenv('DG_GEMV', raising=False)
    g = gen(n + k)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g)
    for m in (1, 2, 3, 4):
        plan = deep_gemm.launch_plan(m, n, k)
        print(f'gemv ks={ks!r} m={m} n={n} k={k} plan={plan}', flush=True)
        # LDS of a workgroup (A as f16, its scale bytes, 64 row sums per row of A) is at most 64 KB
        mr, kp = (1 if m == 1 else 2 if m == 2 else 4), -(-k // 128) * 128
        lds = mr * kp * 2 + mr * kp // 32 + mr * 64 * 4
        assert (plan['skinny'] == 3) == (lds <= 64 * 1024 and (ks != '' or (m == 1 and 4096 <= k <= 8192)))
        a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g)
        d = torch.empty(m, n, dtype=torch.float32, device='cuda')
        deep_gemm.fp8_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
        torch.cuda.synchronize()
        assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq, torch.float32)) < THRESH


@pytest.mark.parametrize('m', [1, 3])
def test_gemv_accumulate_bias(monkeypatch, m):
    """fp32 D += A . B^T (c aliases d), then bf16 D with a bias row."""
    monkeypatch.setenv('DG_GEMV', '4')
    n, k = 700, 4096
    print(f'gemv accumulate/bias m={m} n={n} k={k}', flush=True)
    g = gen(40 + m)
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


def test_gemv_default_plan_bias_and_accumulate(monkeypatch):
    """The default GEMV plan (M = 1, 4096 <= K <= 8192, no DG_GEMV): fp32 D accumulate (c is d),
    bf16 D accumulate (the kernel reads the bf16 D back, adds, rounds once), and a bf16 bias row."""
    monkeypatch.delenv('DG_GEMV', raising=False)
    m, n, k = 1, 2112, 7168
    assert deep_gemm.launch_plan(m, n, k)['skinny'] == 3
    g = gen(45)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, mode='randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, mode='randn')
    args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()))
    rec = dict(recipe_a=(1, 128), recipe_b=(128, 128))
    ref = og.gemm_nt(a_deq, b_deq, torch.float32)
    c = torch.randn(m, n, generator=g) * 4
    d = c.clone().cuda()
    deep_gemm.fp8_gemm_nt(*args, d, c=d, **rec)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), ref + c) < THRESH
    c16 = c.bfloat16()
    d16 = c16.clone().cuda()
    deep_gemm.fp8_gemm_nt(*args, d16, c=d16, **rec)
    torch.cuda.synchronize()
    assert calc_diff(d16.cpu().float(), (ref + c16.float()).bfloat16().float()) < THRESH
    bias = torch.randn(1, n, generator=g).bfloat16()
    d16b = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt(*args, d16b, c=bias.cuda(), **rec)
    torch.cuda.synchronize()
    assert calc_diff(d16b.cpu().float(), ref + bias.float()) < THRESH


def test_gemv_bmm(monkeypatch):
    monkeypatch.setenv('DG_GEMV', '2')
    bs, m, n, k = 5, 2, 300, 2000
    print(f'gemv bmm bs={bs} m={m} n={n} k={k}', flush=True)
    g = gen(44)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g, 'randn', batch=bs)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, 'randn', batch=bs)
    d = torch.empty(bs, m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_bmm((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    for i in range(bs):
        assert calc_diff(d[i].cpu(), og.gemm_nt(a_deq[i], b_deq[i], torch.bfloat16)) < THRESH


def test_gemv_matches_mfma_decode_kernel(monkeypatch):
    """The same inputs through the GEMV kernel and through the MFMA decode kernel (DG_GEMV=0):
    fp32 outputs agree to summation-order rounding (calc_diff < 1e-9), and the GEMV kernel's largest
    error against the fp64 product is within twice the MFMA kernel's."""
    m, n, k = 1, 2112, 7168
    g = gen(45)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, mode='randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, mode='randn')
    args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()))
    out = {}
    for env in ('', '0'):
        monkeypatch.setenv('DG_GEMV', env)
        print(f'gemv vs mfma DG_GEMV={env!r} plan={deep_gemm.launch_plan(m, n, k)}', flush=True)
        d = torch.empty(m, n, dtype=torch.float32, device='cuda')
        deep_gemm.fp8_gemm_nt(*args, d, recipe_a=(1, 128), recipe_b=(128, 128))
        torch.cuda.synchronize()
        out[env] = d.cpu()
    assert deep_gemm.launch_plan(m, n, k)['skinny'] != 3   # (DG_GEMV=0 still set)
    # (|D| up to ~300 here: fp32 sums of 7168 products in two orders differ by a few 1e-3)
    assert calc_diff(out[''], out['0']) < 1e-9
    exact = a_deq.double() @ b_deq.double().t()
    err = {e: (o.double() - exact).abs().max().item() for e, o in out.items()}
    print('max |error| vs fp64', err, 'max |D|', exact.abs().max().item(), flush=True)
    assert err[''] <= 2 * err['0'] + 1e-6 * exact.abs().max().item()
