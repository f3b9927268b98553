"""Seeded random decode shapes (65 <= M <= 128, ragged N, K any multiple of 16 up to 8192; and M from 1, K up
to 16384 with B stored [K, N]) on the default
plans -- the shared-ring kernel's 64 x 64 tiles with M in row blocks, its 128 x 64 two-launch plan, the
skinny-M kernel elsewhere -- for e4m3, bf16 and FP8 x FP4 operands, against the CPU oracle
(calc_diff < 1e-5), the plan each shape took printed with it."""
import random

import pytest
import torch

import deep_gemm
from deep_gemm import _lib
from oracle import gemm as og
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


def _shapes(seed, count):
    rnd = random.Random(seed)
    out = []
    for _ in range(count):
        m = rnd.randint(65, 128)
        n = rnd.choice([rnd.randint(1, 700), rnd.randint(700, 4500)])
        k = 16 * rnd.randint(1, 512)
        out.append((m, n, k))
    return out


@pytest.mark.parametrize('kind', ['e4m3', 'bf16', 'fp4'])
@pytest.mark.parametrize('m,n,k', _shapes(2026, 8))
def test_decode_fuzz(kind, m, n, k):
    g = gen(m * 7919 + n * 31 + k)
    if kind == 'bf16':
        a = (torch.randn(m, k, generator=g) * 0.1).bfloat16()
        b = (torch.randn(n, k, generator=g) * 0.1).bfloat16()
        ref = og.gemm_nt(a.float(), b.float())
        plan = deep_gemm.launch_plan(m, n, k, kind=_lib.DG_KIND_BF16)
        d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
        print(f'decode fuzz {kind} m={m} n={n} k={k} plan={plan}', flush=True)
        deep_gemm.bf16_gemm_nt(a.cuda(), b.cuda(), d)
    else:
        if kind == 'fp4' and k % 32:
            k += 16   # (packed e2m1 rows: K a multiple of 32)
        a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g, 'randn')
        b, sfb, b_deq = operand(n, k, 'e2m1' if kind == 'fp4' else 'e4m3', (1, 32), g, 'randn')
        ref = og.gemm_nt(a_deq, b_deq)
        plan = deep_gemm.launch_plan(m, n, k, kind=_lib.DG_KIND_FP8_FP4 if kind == 'fp4' else _lib.DG_KIND_FP8_FP8)
        d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
        print(f'decode fuzz {kind} m={m} n={n} k={k} plan={plan}', flush=True)
        deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), ref) < THRESH


def _shapes_all_m(seed, count):
    rnd = random.Random(seed)
    out = []
    for _ in range(count):
        m = rnd.choice([rnd.randint(1, 16), rnd.randint(17, 64), rnd.randint(65, 128)])
        n = rnd.choice([rnd.randint(1, 700), rnd.randint(700, 7200)])
        k = 16 * rnd.randint(1, 1024)
        out.append((m, n, k))
    return out


@pytest.mark.parametrize('kind', ['e4m3', 'bf16'])
@pytest.mark.parametrize('m,n,k', _shapes_all_m(2027, 8))
def test_decode_fuzz_mn_major_b(kind, m, n, k):
    """The same for B stored [K, N] (the nn layout: the skinny-M kernel reads it in place), M from 1 to 128,
    K up to 16384."""
    g = gen(m * 104729 + n * 17 + k)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    print(f'decode fuzz nn {kind} m={m} n={n} k={k}', flush=True)
    if kind == 'bf16':
        a = (torch.randn(m, k, generator=g) * 0.1).bfloat16()
        b = (torch.randn(n, k, generator=g) * 0.1).bfloat16()
        ref = og.gemm_nt(a.float(), b.float())
        buf = torch.zeros(k, -(-n // 8) * 8, dtype=torch.bfloat16, device='cuda')
        buf[:, :n] = b.cuda().t()
        deep_gemm.bf16_gemm_nn(a.cuda(), buf[:, :n], d)
    else:
        a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
        b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
        ref = og.gemm_nt(a_deq, b_deq)
        buf = torch.zeros(k, -(-n // 16) * 16, dtype=torch.uint8, device='cuda')
        buf[:, :n] = b.cuda().view(torch.uint8).t()
        deep_gemm.fp8_gemm_nn((a.cuda(), sfa.cuda()), (buf[:, :n].view(torch.float8_e4m3fn), sfb.cuda().t()), d,
                              recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), ref) < THRESH
