"""e4m3 MN-major operands read in place by the 128-K-stage tile kernels (csrc/gemm_kernel.hpp, AMN / BMN:
[K][MN] rows straight to LDS, fragments through ds_read_b64_tr_b8).  Every case checks that no operand
was copied to K-major, that the result is bit-identical to the copy path (DG_MN_COPY=1, whose MFMA
operands are the same bytes) and that it matches the CPU oracle (calc_diff < 1e-5): the four
layouts on every 128-K-stage tile shape, ragged M / N edges, K ending inside a stage, the
north-star shape on its default plan, and K-grouped wgrad with empty and unaligned groups."""
import pytest
import torch

import deep_gemm
import deep_gemm.gemm as dg_gemm_mod
from oracle import gemm as og, layout as ol
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


def _layout_call(layout, m, n, k, seed, block, monkeypatch, no_copy):
    g = gen(seed)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    a, sfa, b, sfb = a.cuda(), sfa.cuda(), b.cuda(), sfb.cuda()
    # logical shapes: A [M,K] (n*) or [K,M] (t*); B [N,K] (*t) or [K,N] (*n).  MN-major storage keeps
    # its K rows 16-byte aligned: an MN extent off the multiple lives in a wider buffer.
    def mn_major(x):
        rows = x.size(0)
        buf = torch.zeros(x.size(1), -(-rows // 16) * 16, dtype=torch.uint8, device='cuda')
        buf[:, :rows] = x.view(torch.uint8).t()
        return buf[:, :rows].view(torch.float8_e4m3fn)
    if layout[0] == 't':
        a, sfa = mn_major(a), sfa.t()
    if layout[1] == 'n':
        b, sfb = mn_major(b), sfb.t()
    if block:
        monkeypatch.setenv('DG_FORCE_BLOCK', block)
    fn = getattr(deep_gemm, f'fp8_gemm_{layout}')
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    no_copy(layout != 'nt')
    fn((a, sfa), (b, sfb), d, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    no_copy(False)
    if block:
        monkeypatch.setenv('DG_FORCE_BLOCK', block)
    monkeypatch.setenv('DG_MN_COPY', '1')
    d_copy = torch.empty_like(d)
    fn((a, sfa), (b, sfb), d_copy, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    return d.cpu(), d_copy.cpu(), og.gemm_nt(a_deq, b_deq)


@pytest.mark.parametrize('layout', ['nn', 'tn', 'tt'])
@pytest.mark.parametrize('block', ['256x256', '256x224', '256x160'])
@pytest.mark.parametrize('m,n,k', [(512, 448, 512), (300, 200, 384), (260, 500, 320)])
def test_mn_major_layouts(monkeypatch, no_copy, layout, block, m, n, k):
    print(f'mn-major fp8_gemm_{layout} {block} m={m} n={n} k={k}', flush=True)
    d, d_copy, ref = _layout_call(layout, m, n, k, 71, block, monkeypatch, no_copy)
    assert torch.equal(d.view(torch.int16), d_copy.view(torch.int16))
    assert calc_diff(d, ref) < THRESH


@pytest.mark.parametrize('layout', ['nn', 'tn', 'tt'])
def test_mn_major_north_star_default_plan(monkeypatch, no_copy, layout):
    m, n, k = 4096, 7168, 2048
    print(f'mn-major fp8_gemm_{layout} default plan m={m} n={n} k={k}', flush=True)
    d, d_copy, ref = _layout_call(layout, m, n, k, 72, None, monkeypatch, no_copy)
    assert torch.equal(d.view(torch.int16), d_copy.view(torch.int16))
    assert calc_diff(d, ref) < THRESH


def test_mn_major_small_plan_falls_back_to_copy(monkeypatch):
    """A plan that cannot read an MN-major operand in place (here MN-major A at a decode shape: the
    decode kernels read A K-major) copies it."""
    m, n, k = 64, 512, 256
    calls = []
    orig = dg_gemm_mod._transpose_to_k_major
    monkeypatch.setattr(dg_gemm_mod, '_transpose_to_k_major', lambda *a, **kw: calls.append(1) or orig(*a, **kw))
    g = gen(73)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    a_km = a.cuda().view(torch.uint8).t().contiguous().view(torch.float8_e4m3fn)   # [K, M]
    deep_gemm.fp8_gemm_tt((a_km, sfa.cuda().t()), (b.cuda(), sfb.cuda()), d, recipe_a=(1, 128), recipe_b=(128, 128))
    torch.cuda.synchronize()
    assert calls, 'the decode plan was expected to copy A'
    assert calc_diff(d.cpu(), og.gemm_nt(a_deq, b_deq)) < THRESH


def _k_grouped_case(m, n, ks, seed, alignment=256):
    total, psum = ol.psum_from_sizes(ks, alignment)
    g = gen(seed)
    keep = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(psum, alignment):
        keep[sl] = True
    out = [psum]
    for rows in (m, n):
        x, sf, deq = operand(rows, total, 'e4m3', (1, 32), g, 'codes')     # [rows, Ktot] K-major
        raw = x.view(torch.uint8).clone()
        raw[:, ~keep] = 0x7f   # padding K rows hold NaN codes: an in-place read must not touch them
        x_tn = raw.t().contiguous().view(torch.float8_e4m3fn)              # [Ktot, rows]
        out += [x_tn, sf.t(), (deq * keep).t()]
    return out


@pytest.mark.parametrize('block', ['256x256', '256x224', '256x160'])
@pytest.mark.parametrize('g_,m,n,ks', [(4, 512, 384, [512, 320, 0, 1000]), (3, 304, 528, [128, 640, 64])])
def test_mn_major_k_grouped(monkeypatch, no_copy, block, g_, m, n, ks):
    print(f'mn-major k_grouped {block} G={g_} m={m} n={n} ks={ks}', flush=True)
    psum, a_tn, sfa, a_deq, b_tn, sfb, b_deq = _k_grouped_case(m, n, ks, seed=74 + g_)
    layout = torch.tensor(psum, dtype=torch.int32, device='cuda')
    if block:
        monkeypatch.setenv('DG_FORCE_BLOCK', block)
    d = torch.empty(g_, m, n, dtype=torch.float32, device='cuda')
    no_copy(True)
    deep_gemm.k_grouped_fp8_gemm_tn_contiguous((a_tn.cuda(), sfa.cuda()), (b_tn.cuda(), sfb.cuda()), d, ks, layout)
    torch.cuda.synchronize()
    no_copy(False)
    ref = og.k_grouped_tn(a_deq, b_deq, psum, 256, None, torch.float32)
    dc = d.cpu()
    for gi in range(g_):
        if ks[gi] == 0:
            assert torch.equal(dc[gi], torch.zeros_like(dc[gi])), gi
        else:
            assert calc_diff(dc[gi], ref[gi]) < THRESH, gi


def _bf16_layout_call(layout, m, n, k, seed, block, monkeypatch, no_copy):
    g = gen(seed)
    a = (torch.randn(m, k, generator=g) * 0.1).bfloat16()
    b = (torch.randn(n, k, generator=g) * 0.1).bfloat16()
    ref = og.gemm_nt(a.float(), b.float())
    a, b = a.cuda(), b.cuda()

    def mn_major(x):   # [rows, K] -> [K, rows] view over a buffer whose K rows are 16-byte aligned
        rows = x.size(0)
        buf = torch.zeros(x.size(1), -(-rows // 8) * 8, dtype=torch.bfloat16, device='cuda')
        buf[:, :rows] = x.t()
        return buf[:, :rows]
    if layout[0] == 't':
        a = mn_major(a)
    if layout[1] == 'n':
        b = mn_major(b)
    if block:
        monkeypatch.setenv('DG_FORCE_BLOCK', block)
    fn = getattr(deep_gemm, f'bf16_gemm_{layout}')
    d = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    # (bf16 nn at M > 128 copies B by design: only A MN-major operands are read in place there)
    no_copy(layout in ('tn', 'tt'))
    fn(a, b, d)
    torch.cuda.synchronize()
    no_copy(False)
    if block:
        monkeypatch.setenv('DG_FORCE_BLOCK', block)
    monkeypatch.setenv('DG_MN_COPY', '1')
    d_copy = torch.empty_like(d)
    fn(a, b, d_copy)
    torch.cuda.synchronize()
    return d.cpu(), d_copy.cpu(), ref


@pytest.mark.parametrize('layout', ['nn', 'tn', 'tt'])
@pytest.mark.parametrize('block', ['256x256', '256x224', '256x160'])
@pytest.mark.parametrize('m,n,k', [(512, 448, 512), (300, 200, 384), (260, 500, 320)])
def test_mn_major_bf16_layouts(monkeypatch, no_copy, layout, block, m, n, k):
    print(f'mn-major bf16_gemm_{layout} {block} m={m} n={n} k={k}', flush=True)
    d, d_copy, ref = _bf16_layout_call(layout, m, n, k, 81, block, monkeypatch, no_copy)
    assert torch.equal(d.view(torch.int16), d_copy.view(torch.int16))
    assert calc_diff(d, ref) < THRESH


@pytest.mark.parametrize('layout', ['nn', 'tn'])
def test_mn_major_bf16_baseline_shape(monkeypatch, no_copy, layout):
    """BASELINE config 3's M=4096 shape on its default plan (nn: B copied, tn: both in place)."""
    m, n, k = 4096, 7168, 2048
    print(f'mn-major bf16_gemm_{layout} default plan m={m} n={n} k={k}', flush=True)
    d, d_copy, ref = _bf16_layout_call(layout, m, n, k, 82, None, monkeypatch, no_copy)
    assert torch.equal(d.view(torch.int16), d_copy.view(torch.int16))
    assert calc_diff(d, ref) < THRESH


@pytest.mark.parametrize('block', ['256x256', '256x224'])
def test_mn_major_bf16_k_grouped(monkeypatch, no_copy, block):
    m, n, ks = 304, 528, [700, 0, 256, 96]
    print(f'mn-major k_grouped bf16 {block} m={m} n={n} ks={ks}', flush=True)
    total, psum = ol.psum_from_sizes(ks, 256)
    g = gen(83)
    keep = torch.zeros(total, 1)
    for sl in ol.psum_slices(psum, 256):
        keep[sl] = 1
    a = (torch.randn(total, m, generator=g) * keep).bfloat16()
    b = (torch.randn(total, n, generator=g) * keep).bfloat16()
    a_dev, b_dev = a.cuda(), b.cuda()
    a_dev[keep.squeeze(1) == 0] = float('nan')   # padding K rows: never read in place
    b_dev[keep.squeeze(1) == 0] = float('nan')
    c = torch.randn(len(ks), m, n, generator=g)
    d = c.clone().cuda()
    monkeypatch.setenv('DG_FORCE_BLOCK', block)
    no_copy(True)
    deep_gemm.k_grouped_bf16_gemm_tn_contiguous(a_dev, b_dev, d, ks, torch.tensor(psum, dtype=torch.int32, device='cuda'), c=d)
    torch.cuda.synchronize()
    no_copy(False)
    ref = og.k_grouped_tn(a.float(), b.float(), psum, 256, c, torch.float32)
    assert torch.equal(d[1].cpu(), c[1])
    assert calc_diff(d.cpu(), ref) < THRESH


@pytest.mark.parametrize('psum', [True, False])
@pytest.mark.parametrize('dtype', ['e4m3', 'bf16'])
def test_mn_major_m_grouped_nn(monkeypatch, no_copy, psum, dtype):
    """m_grouped_*_gemm_nn_contiguous at alignment 256 (256-row tiles): B [G, K, N] read in place;
    padding rows exact zeros, bit-identical to the copy path, oracle parity."""
    sizes, n, k, alignment = [200, 512, 0, 300], 384, 512, 256
    print(f'mn-major m_grouped nn {dtype} psum={psum} sizes={sizes} n={n} k={k}', flush=True)
    g = gen(91)
    total, ps = ol.psum_from_sizes(sizes, alignment)
    if dtype == 'e4m3':
        a, sfa, a_deq = operand(total, k, 'e4m3', (1, 128), g, 'randn')
        b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn', batch=len(sizes))
    else:
        a_deq = (torch.randn(total, k, generator=g) * 0.1).bfloat16().float()
        b_deq = (torch.randn(len(sizes), n, k, generator=g) * 0.1).bfloat16().float()
        a, b = a_deq.bfloat16(), b_deq.bfloat16()
    for sl in ol.psum_pad_slices(ps, alignment):
        a.view(torch.uint8 if dtype == 'e4m3' else torch.int16)[sl] = 0
        a_deq[sl] = 0
    layout_t = torch.tensor(ps, dtype=torch.int32) if psum else ol.m_indices_from_psum(ps, alignment, total)
    ref = og.m_grouped_contiguous(a_deq, b_deq, layout_t, psum, alignment)
    b_kn = b.cuda().transpose(1, 2).contiguous()   # [G, K, N] storage: N contiguous
    b_view = b_kn.transpose(1, 2)                   # logical [G, N, K], MN-major

    def run(copy):
        d = torch.full((total, n), float('nan'), dtype=torch.bfloat16, device='cuda')
        no_copy(not copy)
        # the problem is small enough to plan 128-row tiles; force a 256x256 tile (alignment 256)
        monkeypatch.setenv('DG_FORCE_BLOCK', '256x256')
        if copy:
            monkeypatch.setenv('DG_MN_COPY', '1')
        if dtype == 'e4m3':
            deep_gemm.m_grouped_fp8_gemm_nn_contiguous((a.cuda(), sfa.cuda()), (b_kn, sfb.cuda().transpose(1, 2)), d,
                                                       layout_t.cuda(), recipe_a=(1, 128), recipe_b=(128, 128),
                                                       use_psum_layout=psum)
        else:
            deep_gemm.m_grouped_bf16_gemm_nn_contiguous(a.cuda(), b_kn, d, layout_t.cuda(), use_psum_layout=psum)
        torch.cuda.synchronize()
        no_copy(False)
        return d.cpu()
    out = run(False)
    out_copy = run(True)
    assert torch.equal(out.view(torch.int16), out_copy.view(torch.int16))
    valid = torch.zeros(total, dtype=torch.bool)
    for sl in ol.psum_slices(ps, alignment):
        valid[sl] = True
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid]))
    assert calc_diff(out[valid], ref[valid]) < THRESH
