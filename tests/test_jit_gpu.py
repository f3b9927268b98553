"""Kernels compiled at run time (set_jit(True): hipRTC, GEMM type / K split / compiled_dims sizes
as compile-time constants, launched through hipModuleLaunchKernel) give bit-identical results to
the ahead-of-time kernels of the same plan, for every GEMM type, and match the CPU oracle."""
import os

import pytest
import torch

import deep_gemm
from deep_gemm import _lib
from oracle import gemm as og
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


@pytest.fixture(autouse=True)
def jit_cache(tmp_path, monkeypatch):
    monkeypatch.setenv('DG_JIT_CACHE_DIR', str(tmp_path / 'jit'))
    # (the skinny-M kernel that decode shapes take is ahead-of-time only: keep the tile kernel)
    monkeypatch.setenv('DG_SKINNY', '0')
    yield
    deep_gemm.set_jit(False)


def _both(fn):
    """fn() with AOT kernels, then with run-time compiled kernels; both outputs."""
    deep_gemm.set_jit(False)
    aot = fn()
    torch.cuda.synchronize()
    compiled0 = _lib.jit_stats()[0]
    deep_gemm.set_jit(True)
    jit = fn()
    torch.cuda.synchronize()
    deep_gemm.set_jit(False)
    assert _lib.jit_stats()[0] > compiled0, 'the run-time compiler was not used'
    return aot, jit


@pytest.mark.parametrize('m,n,k,dims', [(4096, 7168, 2048, 'nk'), (300, 500, 832, 'nk'), (300, 500, 832, 'mnk'),
                                        (128, 7168, 4096, 'nk'), (77, 130, 200, '')])
def test_jit_dense(m, n, k, dims):
    print(f'jit dense m={m} n={n} k={k} dims={dims!r}', flush=True)
    g = gen(31)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g)
    b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g)
    a, sfa, b, sfb = a.cuda(), sfa.cuda(), b.cuda(), sfb.cuda()

    def run():
        d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
        deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, compiled_dims=dims)
        return d
    aot, jit = _both(run)
    assert torch.equal(aot, jit)
    assert calc_diff(jit.cpu(), og.gemm_nt(a_deq, b_deq)) < THRESH


def test_jit_fp8_fp4_and_bf16():
    print('jit fp8xfp4 / bf16', flush=True)
    g = gen(32)
    m, n, k = 256, 384, 512
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g)
    b, sfb, b_deq = operand(n, k, 'e2m1', (1, 32), g)
    a, sfa, b, sfb = a.cuda(), sfa.cuda(), b.cuda(), sfb.cuda()

    def run():
        d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
        deep_gemm.fp8_fp4_gemm_nt((a, sfa), (b, sfb), d)
        return d
    aot, jit = _both(run)
    assert torch.equal(aot, jit)
    x = (torch.randn(m, k, generator=g) * 0.1).bfloat16().cuda()
    y = (torch.randn(n, k, generator=g) * 0.1).bfloat16().cuda()

    def run_bf16():
        d = torch.empty(m, n, dtype=torch.float32, device='cuda')
        deep_gemm.bf16_gemm_nt(x, y, d)
        return d
    aot, jit = _both(run_bf16)
    assert torch.equal(aot, jit)


def test_jit_m_grouped_and_masked():
    print('jit m-grouped / masked', flush=True)
    g = gen(33)
    counts, n, k, align = [300, 0, 129, 256], 448, 640, 128
    psum, total = [], 0
    for c in counts:
        psum.append(total + c)
        total = -(-(total + c) // align) * align
    a, sfa, _ = operand(total, k, 'e4m3', (1, 32), g)
    b, sfb, _ = operand(n, k, 'e4m3', (1, 32), g, batch=len(counts))
    a, sfa, b, sfb = a.cuda(), sfa.cuda(), b.cuda(), sfb.cuda()
    layout = torch.tensor(psum, dtype=torch.int32, device='cuda')

    def run():
        d = torch.empty(total, n, dtype=torch.bfloat16, device='cuda')
        deep_gemm.set_mk_alignment_for_contiguous_layout(align)
        try:
            deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a, sfa), (b, sfb), d, layout)
        finally:
            deep_gemm.set_mk_alignment_for_contiguous_layout(256)
        return d
    aot, jit = _both(run)
    assert torch.equal(aot, jit)
    am, sfam, _ = operand(256, k, 'e4m3', (1, 32), g, batch=len(counts))
    am, sfam = am.cuda(), sfam.cuda()
    masked = torch.tensor([min(c, 256) for c in counts], dtype=torch.int32, device='cuda')

    def run_masked():
        d = torch.zeros(len(counts), 256, n, dtype=torch.bfloat16, device='cuda')
        deep_gemm.m_grouped_fp8_gemm_nt_masked((am, sfam), (b, sfb), d, masked, 256)
        return d
    aot, jit = _both(run_masked)
    assert torch.equal(aot, jit)


def test_jit_batched_and_split(monkeypatch):
    print('jit bmm / split-K', flush=True)
    g = gen(34)
    bsz, m, n, k = 3, 200, 256, 512
    a, sfa, _ = operand(m, k, 'e4m3', (1, 32), g, batch=bsz)
    b, sfb, _ = operand(n, k, 'e4m3', (1, 32), g, batch=bsz)
    a, sfa, b, sfb = a.cuda(), sfa.cuda(), b.cuda(), sfb.cuda()

    def run():
        d = torch.empty(bsz, m, n, dtype=torch.bfloat16, device='cuda')
        deep_gemm.fp8_bmm((a, sfa), (b, sfb), d)
        return d
    aot, jit = _both(run)
    assert torch.equal(aot, jit)
    monkeypatch.setenv('DG_SPLIT_K', '3')
    a2, sfa2, a_deq = operand(64, 4096, 'e4m3', (1, 32), g)
    b2, sfb2, b_deq = operand(2112, 4096, 'e4m3', (1, 32), g)
    a2, sfa2, b2, sfb2 = a2.cuda(), sfa2.cuda(), b2.cuda(), sfb2.cuda()

    def run_split():
        d = torch.empty(64, 2112, dtype=torch.bfloat16, device='cuda')
        deep_gemm.fp8_gemm_nt((a2, sfa2), (b2, sfb2), d)
        return d
    aot, jit = _both(run_split)
    assert torch.equal(aot, jit)
    assert calc_diff(jit.cpu(), og.gemm_nt(a_deq, b_deq)) < THRESH


def test_jit_dry_run_compiles_without_launch():
    print('jit dry run', flush=True)
    g = gen(35)
    m, n, k = 128, 256, 384
    a, sfa, _ = operand(m, k, 'e4m3', (1, 32), g)
    b, sfb, _ = operand(n, k, 'e4m3', (1, 32), g)
    a, sfa, b, sfb = a.cuda(), sfa.cuda(), b.cuda(), sfb.cuda()
    d = torch.full((m, n), 7.0, dtype=torch.bfloat16, device='cuda')
    before = _lib.jit_stats()[0]
    deep_gemm.set_jit(True)
    deep_gemm.set_dry_run(True)
    try:
        deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d)
    finally:
        deep_gemm.set_dry_run(False)
        deep_gemm.set_jit(False)
    torch.cuda.synchronize()
    assert _lib.jit_stats()[0] == before + 1
    assert torch.all(d == 7.0), 'a dry run must not launch'
