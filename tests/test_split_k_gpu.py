"""GPU parity of split-K launches (K cut into ranges, fp32 partial tiles reduced by the last
workgroup of each tile) against the CPU oracle, through libdeep_gemm_amd.so.  Split-K has no
counterpart in the reference; its results are pinned by the same oracle and calc_diff bar
(1e-5, tests/test_fp8_gemm.py:21 of the reference) as the unsplit path."""
import os

import pytest
import torch

import deep_gemm
from oracle import gemm as og
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


@pytest.fixture
def split_env():
    old = os.environ.get('DG_SPLIT_K')
    yield
    if old is None:
        os.environ.pop('DG_SPLIT_K', None)
    else:
        os.environ['DG_SPLIT_K'] = old


def _case(m, n, k, seed, b_kind='e4m3'):
    g = gen(seed)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 32), g, 'codes')
    b, sfb, b_deq = operand(n, k, b_kind, (1, 32), g, 'codes')
    return a.cuda(), sfa.cuda(), a_deq, b.cuda(), sfb.cuda(), b_deq


def _counters_zero(m, n, k, kind=0):
    """The tile counters (first align(tiles * 4, 256) bytes of the workspace) are back at zero."""
    import ctypes
    from deep_gemm import _lib
    args = _lib.GemmArgs()
    args.kind, args.gemm_type, args.m, args.n, args.k, args.num_groups = kind, 0, m, n, k, 1
    args.num_cus = deep_gemm.get_num_sms()
    args.alignment = 256
    args.split_k = int(os.environ.get('DG_SPLIT_K', '0'))
    args.workspace = 1   # any non-NULL value: ask for the split plan
    bm, bn = ctypes.c_int32(), ctypes.c_int32()
    lib = _lib.load()
    _lib.check(lib.dg_select_config(ctypes.byref(args), ctypes.byref(bm), ctypes.byref(bn)), lib)
    tiles = -(-m // bm.value) * -(-n // bn.value)
    nbytes = -(-tiles * 4 // 256) * 256
    ptr, size = ctypes.c_void_p(), ctypes.c_int64()
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.dg_stream_workspace(stream, ctypes.byref(ptr), ctypes.byref(size)), lib)
    assert ptr.value and size.value >= nbytes
    host = (ctypes.c_uint8 * nbytes)()
    hip = ctypes.CDLL('libamdhip64.so')
    assert hip.hipMemcpy(host, ptr, ctypes.c_size_t(nbytes), 2) == 0   # hipMemcpyDeviceToHost
    return not any(host)


@pytest.mark.parametrize('split', [2, 3, 5, 8])
@pytest.mark.parametrize('m,n,k', [(128, 2112, 2048), (1, 7168, 1024), (64, 512, 4096), (130, 257, 1984)])
def test_split_k_forced(split_env, split, m, n, k):
    print(f'split_k={split} m={m} n={n} k={k}', flush=True)
    os.environ['DG_SPLIT_K'] = str(split)
    a, sfa, a_deq, b, sfb, b_deq = _case(m, n, k, seed=split + m)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq)) < THRESH
    assert _counters_zero(m, n, k), 'split-K counters must be left at zero'


def test_split_k_fp32_accumulate_bias(split_env):
    print('split_k fp32 accumulate', flush=True)
    os.environ['DG_SPLIT_K'] = '4'
    m, n, k = 96, 640, 2048
    a, sfa, a_deq, b, sfb, b_deq = _case(m, n, k, seed=7)
    g = gen(8)
    c = torch.randn(m, n, generator=g)
    d = c.clone().cuda()
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d, c=d)
    torch.cuda.synchronize()
    ref = og.gemm_nt(a_deq, b_deq, torch.float32, c=c)
    assert calc_diff(d.cpu(), ref) < THRESH
    bias = torch.randn(1, n, generator=g).to(torch.bfloat16)
    d2 = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d2, c=bias.cuda())
    torch.cuda.synchronize()
    ref2 = og.gemm_nt(a_deq, b_deq, bias=bias)
    assert calc_diff(d2.cpu(), ref2) < THRESH
    assert _counters_zero(m, n, k)


def test_split_k_heuristic_skinny_shapes(split_env):
    """The heuristic splits skinny shapes on its own; repeated calls reuse the workspace."""
    os.environ.pop('DG_SPLIT_K', None)
    for (m, n, k) in [(128, 2112, 7168), (1, 7168, 2048), (64, 4096, 7168)]:
        print(f'split_k heuristic m={m} n={n} k={k}', flush=True)
        a, sfa, a_deq, b, sfb, b_deq = _case(m, n, k, seed=m + n)
        ref = og.gemm_nt(a_deq, b_deq)
        for _ in range(3):
            d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
            deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d)
            torch.cuda.synchronize()
            assert calc_diff(d.cpu(), ref) < THRESH
        assert _counters_zero(m, n, k)


def test_split_k_fp8_fp4(split_env):
    print('split_k fp8 x fp4', flush=True)
    os.environ['DG_SPLIT_K'] = '3'
    m, n, k = 128, 1024, 3072
    a, sfa, a_deq, b, sfb, b_deq = _case(m, n, k, seed=11, b_kind='e2m1')
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_fp4_gemm_nt((a, sfa), (b, sfb), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq)) < THRESH


@pytest.mark.parametrize('tile', ['256x256', '128x256', '128x128', '64x128'])
@pytest.mark.parametrize('split', [2, 3])
def test_split_k_tiles(split_env, monkeypatch, tile, split):
    """Forced split on every splittable tile shape, including the 128-K-stage two-slot ring, with a
    K that ends inside a stage."""
    m, n, k = 300, 512, 1984
    print(f'split_k={split} tile={tile} m={m} n={n} k={k}', flush=True)
    monkeypatch.setenv('DG_FORCE_BLOCK', tile)
    os.environ['DG_SPLIT_K'] = str(split)
    a, sfa, a_deq, b, sfb, b_deq = _case(m, n, k, seed=40 + split)
    d = torch.empty(m, n, dtype=torch.float32, device='cuda')
    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d)
    torch.cuda.synchronize()
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq, torch.float32)) < THRESH


def test_split_back_to_back_matches_isolated():
    """Split-K launches issued back to back on one stream with no sync between them (skinny-M kernel
    with its K split, and a tile-kernel split): workgroups of one tile may then sit on different
    XCDs.  Each output equals the same GEMM launched alone, bit for bit, on every repetition."""
    print('split back to back', flush=True)
    shapes = [(1, 2112, 7168, None), (16, 4096, 7168, None), (128, 2112, 7168, None), (64, 2112, 4096, '3')]
    cases = []
    for i, (m, n, k, split) in enumerate(shapes):
        a, sfa, _, b, sfb, _ = _case(m, n, k, seed=60 + i)
        if split is not None:
            os.environ['DG_SKINNY'], os.environ['DG_SPLIT_K'] = '0', split
        try:
            d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
            deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d)
            torch.cuda.synchronize()
        finally:
            os.environ.pop('DG_SKINNY', None)
            os.environ.pop('DG_SPLIT_K', None)
        cases.append((a, sfa, b, sfb, d.clone(), split))
    outs = [torch.empty_like(c[4]) for c in cases]
    for rep in range(3):
        for _ in range(8):
            for (a, sfa, b, sfb, _, split), d in zip(cases, outs):
                if split is not None:
                    os.environ['DG_SKINNY'], os.environ['DG_SPLIT_K'] = '0', split
                try:
                    deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d)
                finally:
                    os.environ.pop('DG_SKINNY', None)
                    os.environ.pop('DG_SPLIT_K', None)
        torch.cuda.synchronize()
        for i, (c, d) in enumerate(zip(cases, outs)):
            assert torch.equal(d.view(torch.int16), c[4].view(torch.int16)), (rep, shapes[i])


@pytest.mark.parametrize('m,n,k,split', [(64, 2112, 7168, 4), (130, 257, 1984, 3), (256, 1024, 4096, 5)])
def test_split_k_across_xcds(split_env, m, n, k, split):
    """The splits of one tile on different XCDs (DG_SPLIT_SPREAD=1 hands them to consecutive
    workgroups, which the dispatcher places round-robin over the 8 XCDs): the device-scope partial
    stores and loads must still meet, on every one of three back-to-back calls."""
    print(f'split_k across XCDs m={m} n={n} k={k} split={split}', flush=True)
    os.environ['DG_SPLIT_K'] = str(split)
    os.environ['DG_SPLIT_SPREAD'] = '1'
    try:
        plan = deep_gemm.launch_plan(m, n, k, split_k=split)
        print('plan', plan, flush=True)
        assert plan['split_k'] == split
        a, sfa, a_deq, b, sfb, b_deq = _case(m, n, k, seed=m + split)
        ref = og.gemm_nt(a_deq, b_deq)
        for _ in range(3):
            d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
            deep_gemm.fp8_gemm_nt((a, sfa), (b, sfb), d)
            torch.cuda.synchronize()
            assert calc_diff(d.cpu(), ref) < THRESH
        assert _counters_zero(m, n, k)
    finally:
        os.environ.pop('DG_SPLIT_SPREAD', None)
