"""MN-major B (stored [K][N], N contiguous: the `nn` layouts) read in place by the skinny-M decode kernel
(csrc/skinny_kernel.hpp, BMN: the strip's K rows straight to LDS, fragments through ds_read_b64_tr_b8 /
ds_read_b64_tr_b16).  Every case checks that B was not copied to K-major and that the result matches the CPU
oracle (calc_diff < 1e-5); on a forced skinny configuration (DG_SKINNY, optionally split across workgroups)
it is also bit-identical to the copy path (DG_MN_COPY=1) on the same configuration, whose MFMA operands are
the same bytes.  Covers e4m3 and bf16, every 32-column configuration, ragged N and K, and the default plans
of config-2 decode shapes."""
import pytest
import torch

import deep_gemm
import deep_gemm.gemm as dg_gemm_mod
from oracle import gemm as og
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu
THRESH = 1e-5


@pytest.fixture
def no_copy(monkeypatch):
    """Fail the test if any operand goes through the MN-major -> K-major copy."""
    def _forbid(*args, **kwargs):
        raise AssertionError('an MN-major operand was copied to K-major')
    def _set(on):
        if on:
            monkeypatch.setattr(dg_gemm_mod, '_transpose_to_k_major', _forbid)
        else:
            monkeypatch.undo()
    return _set


def _mn_major(x, align):
    """[rows, K] -> [K, rows] view over a buffer whose K rows are 16-byte aligned."""
    rows = x.size(0)
    buf = torch.zeros(x.size(1), -(-rows // align) * align, dtype=x.dtype, device='cuda')
    buf[:, :rows] = x.t()
    return buf[:, :rows]


def _case(kind, m, n, k, seed):
    g = gen(seed)
    if kind == 'fp8':
        a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
        b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
        b_kn = _mn_major(b.cuda().view(torch.uint8), 16).view(torch.float8_e4m3fn)
        fn = lambda d: deep_gemm.fp8_gemm_nn((a.cuda(), sfa.cuda()), (b_kn, sfb.cuda().t()), d,
                                             recipe_a=(1, 128), recipe_b=(128, 128))
        return fn, og.gemm_nt(a_deq, b_deq)
    a = (torch.randn(m, k, generator=g) * 0.1).bfloat16()
    b = (torch.randn(n, k, generator=g) * 0.1).bfloat16()
    a_c, b_kn = a.cuda(), _mn_major(b.cuda(), 8)
    return (lambda d: deep_gemm.bf16_gemm_nn(a_c, b_kn, d)), og.gemm_nt(a.float(), b.float())


@pytest.mark.parametrize('kind', ['fp8', 'bf16'])
@pytest.mark.parametrize('cfg,m', [('1,1,4,2,16', 1), ('1,1,4,2,16', 16), ('1,1,8,2,16', 7), ('1,1,4,3,16', 5),
                                   ('1,1,4,2,32', 32), ('1,1,4,3,32', 20), ('2,1,4,2,64', 64), ('2,1,4,2,64', 40),
                                   ('4,1,4,2,128', 128), ('4,1,4,2,128', 100), ('1,1,4,2,16,3', 3),
                                   ('2,1,4,2,64,4', 64), ('4,1,4,2,128,2', 96)])
@pytest.mark.parametrize('n,k', [(512, 256), (200, 1984), (2112, 7168)])
def test_mn_major_b_decode_forced(monkeypatch, no_copy, kind, cfg, m, n, k):
    print(f'mn-major B decode {kind} DG_SKINNY={cfg} m={m} n={n} k={k}', flush=True)
    fn, ref = _case(kind, m, n, k, 91)
    monkeypatch.setenv('DG_SKINNY', cfg)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    no_copy(True)
    fn(d)
    torch.cuda.synchronize()
    no_copy(False)
    monkeypatch.setenv('DG_SKINNY', cfg)
    monkeypatch.setenv('DG_MN_COPY', '1')
    d_copy = torch.empty_like(d)
    fn(d_copy)
    torch.cuda.synchronize()
    assert torch.equal(d.cpu().view(torch.int16), d_copy.cpu().view(torch.int16))
    assert calc_diff(d.cpu(), ref) < THRESH


@pytest.mark.parametrize('kind', ['fp8', 'bf16'])
@pytest.mark.parametrize('m,n,k', [(1, 2112, 7168), (128, 4096, 7168), (128, 7168, 16384), (96, 3072, 7168), (1, 7168, 2048), (64, 4096, 7168), (100, 2112, 7168),
                                   (128, 7168, 2048), (128, 2112, 7168), (33, 7168, 16384)])
def test_mn_major_b_decode_default_plan(no_copy, kind, m, n, k):
    """config-2 / config-3 decode shapes in the nn layout on their default plans: B read in place."""
    print(f'mn-major B decode {kind} default plan m={m} n={n} k={k}', flush=True)
    fn, ref = _case(kind, m, n, k, 92)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    no_copy(True)
    fn(d)
    torch.cuda.synchronize()
    no_copy(False)
    assert calc_diff(d.cpu(), ref) < THRESH


def test_mn_major_b_decode_fp32_accumulate(no_copy):
    """fp32 D accumulated in place (c = d) through the MN-major decode path, ragged N."""
    m, n, k = 16, 1000, 1024
    g = gen(93)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    b_kn = _mn_major(b.cuda().view(torch.uint8), 16).view(torch.float8_e4m3fn)
    ref = og.gemm_nt(a_deq, b_deq)
    c = torch.randn(m, n, generator=g).cuda()
    d = c.clone()
    no_copy(True)
    deep_gemm.fp8_gemm_nn((a.cuda(), sfa.cuda()), (b_kn, sfb.cuda().t()), d, c=d, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    no_copy(False)
    assert calc_diff(d.cpu(), ref + c.cpu()) < THRESH


@pytest.mark.parametrize('kind', ['fp8', 'bf16'])
def test_mn_major_tn_decode_copies_only_a(monkeypatch, kind):
    """tn at a decode shape (A [K, M] and B [K, N] both MN-major): the decode kernels read A K-major, so only
    A is copied; B is read in place."""
    m, n, k = 64, 2112, 1024
    g = gen(94)
    copied = []
    orig = dg_gemm_mod._transpose_to_k_major
    monkeypatch.setattr(dg_gemm_mod, '_transpose_to_k_major',
                        lambda t, *args, **kw: copied.append(tuple(t.shape)) or orig(t, *args, **kw))
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    if kind == 'fp8':
        a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
        b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
        a_km = _mn_major(a.cuda().view(torch.uint8), 16).view(torch.float8_e4m3fn)
        b_kn = _mn_major(b.cuda().view(torch.uint8), 16).view(torch.float8_e4m3fn)
        deep_gemm.fp8_gemm_tn((a_km, sfa.cuda().t()), (b_kn, sfb.cuda().t()), d, recipe_a=(1, 128), recipe_b=(128, 128))
        ref = og.gemm_nt(a_deq, b_deq)
    else:
        a = (torch.randn(m, k, generator=g) * 0.1).bfloat16()
        b = (torch.randn(n, k, generator=g) * 0.1).bfloat16()
        deep_gemm.bf16_gemm_tn(_mn_major(a.cuda(), 8), _mn_major(b.cuda(), 8), d)
        ref = og.gemm_nt(a.float(), b.float())
    torch.cuda.synchronize()
    assert len(copied) == 1 and sorted(copied[0]) == sorted((m, k)), copied
    assert calc_diff(d.cpu(), ref) < THRESH


@pytest.mark.parametrize('kind', ['fp8', 'bf16'])
@pytest.mark.parametrize('cus,m,n,k', [(100, 64, 2112, 7168), (64, 1, 4096, 4096), (40, 128, 1000, 2048)])
def test_mn_major_b_decode_under_cu_cap(no_copy, kind, cus, m, n, k):
    """set_num_sms(n) below the CU count: the MN-major decode launch (padded and remapped so that strips
    sharing a line of B run on one XCD) goes out in chunks of at most n workgroups; D matches the oracle."""
    print(f'mn-major B decode {kind} set_num_sms({cus}) m={m} n={n} k={k}', flush=True)
    full = deep_gemm.get_num_sms()
    fn, ref = _case(kind, m, n, k, 96)
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    try:
        deep_gemm.set_num_sms(cus)
        no_copy(True)
        fn(d)
        torch.cuda.synchronize()
        no_copy(False)
    finally:
        deep_gemm.set_num_sms(full)
    assert calc_diff(d.cpu(), ref) < THRESH
