"""Committed fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
the CPU oracle must reproduce them bit-exactly; the GPU kernels must match them
(bit-exact for the SF layout and grouped padding rows, calc_diff < 1e-5 for GEMM values).
tests/golden/sr_bf16_reference.npz (written by tests/golden/make_sr_golden.py) holds stochastic-rounding
outputs that the reference's own check (tests/utils.py:70-92 of the reference) accepted: the oracle's
rounding must reproduce them bit for bit."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import epilogue as oe, gemm as og, layout as ol, quant

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def _load(name):
    z = np.load(os.path.join(GOLD, name + '.npz'), allow_pickle=False)
    return {k: z[k] for k in z.files}, json.loads(str(z['meta']))


def _fp8(arr):
    return torch.from_numpy(arr).view(torch.float8_e4m3fn)


def _operands(z, meta):
    a = _fp8(z['a'])
    b = _fp8(z['b']) if meta.get('kind_b', 'e4m3') == 'e4m3' else torch.from_numpy(z['b']).view(torch.int8)
    return a, torch.from_numpy(z['sfa']), b, torch.from_numpy(z['sfb'])


def _expected(z):
    return torch.from_numpy(z['d_bits']).view(torch.bfloat16)


GEMM_CASES = ['fp8_nt_codes_96x160x384', 'fp8_nt_randn_128x256x512_1x128_128x128', 'fp8_fp4_nt_codes_64x128x256']


@pytest.mark.parametrize('name', GEMM_CASES)
def test_oracle_reproduces_gemm_fixture(name):
    z, meta = _load(name)
    a, sfa, b, sfb = _operands(z, meta)
    m, n, k = meta['m'], meta['n'], meta['k']
    pa = ol.transform_sf(sfa, m, k, meta['gran_a'][0], meta['gran_a'][1])
    pb = ol.transform_sf(sfb, n, k, meta['gran_b'][0], meta['gran_b'][1])
    d = og.gemm_nt(og.dequant_operand(a, pa, k), og.dequant_operand(b, pb, k))
    assert torch.equal(d.view(torch.int16), _expected(z).view(torch.int16))


@pytest.mark.parametrize('name', ['transform_sf_300x1000_g1', 'transform_sf_300x1000_g128_k128', 'transform_sf_psum_640x512'])
def test_oracle_reproduces_transform_fixture(name):
    z, meta = _load(name)
    out = ol.transform_sf(torch.from_numpy(z['sf']), meta['mn'], meta['k'], meta['gran_mn'], meta['gran_k'],
                          psum=meta['psum'], alignment=meta['alignment'])
    assert np.array_equal(out.contiguous().numpy(), z['out'])


def test_oracle_reproduces_grouped_and_bf16_fixtures():
    z, meta = _load('m_grouped_psum_3g_64x128')
    a, b = _fp8(z['a']), _fp8(z['b'])
    total, k = a.shape
    pa = ol.transform_sf(torch.from_numpy(z['sfa']), total, k, 1, 32)
    a_deq = og.dequant_operand(a, pa, k)
    b_deq = quant.decode(b) * quant.expand_sf(torch.from_numpy(z['sfb']), b.shape, (1, 1, 32))
    d = og.m_grouped_contiguous(a_deq, b_deq, torch.from_numpy(z['psum']), True, meta['alignment'])
    assert torch.equal(d.view(torch.int16), _expected(z).view(torch.int16))
    z, meta = _load('bf16_nt_64x96x128')
    a = torch.from_numpy(z['a']).view(torch.bfloat16)
    b = torch.from_numpy(z['b']).view(torch.bfloat16)
    assert torch.equal(og.gemm_nt(a.float(), b.float()).view(torch.int16), _expected(z).view(torch.int16))


# ----------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize('name', GEMM_CASES)
def test_kernel_matches_gemm_fixture(name):
    import deep_gemm
    z, meta = _load(name)
    a, sfa, b, sfb = _operands(z, meta)
    d = torch.empty(meta['m'], meta['n'], dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()), d,
                              recipe_a=tuple(meta['gran_a']), recipe_b=tuple(meta['gran_b']))
    torch.cuda.synchronize()
    assert og.calc_diff(d.cpu(), _expected(z)) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize('name', ['transform_sf_300x1000_g1', 'transform_sf_300x1000_g128_k128', 'transform_sf_psum_640x512'])
def test_kernel_matches_transform_fixture(name):
    import deep_gemm
    z, meta = _load(name)
    psum = torch.tensor(meta['psum'], dtype=torch.int32).cuda() if meta['psum'] else None
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(meta['alignment'])
    try:
        out = deep_gemm.transform_sf_into_required_layout(torch.from_numpy(z['sf']).cuda(), meta['mn'], meta['k'],
                                                          (meta['gran_mn'], meta['gran_k']), is_sfa=True,
                                                          psum_layout=psum)
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    torch.cuda.synchronize()
    assert out.stride(-2) == 1
    assert np.array_equal(out.cpu().contiguous().numpy(), z['out'])


@pytest.mark.gpu
def test_kernel_matches_grouped_fixture():
    import deep_gemm
    z, meta = _load('m_grouped_psum_3g_64x128')
    a, b = _fp8(z['a']).cuda(), _fp8(z['b']).cuda()
    d = torch.full((a.shape[0], meta['n']), float('nan'), dtype=torch.bfloat16, device='cuda')
    old = deep_gemm.get_mk_alignment_for_contiguous_layout()
    deep_gemm.set_mk_alignment_for_contiguous_layout(meta['alignment'])
    try:
        deep_gemm.m_grouped_fp8_gemm_nt_contiguous((a, torch.from_numpy(z['sfa']).cuda()),
                                                   (b, torch.from_numpy(z['sfb']).cuda()), d,
                                                   torch.from_numpy(z['psum']).cuda())
    finally:
        deep_gemm.set_mk_alignment_for_contiguous_layout(old)
    torch.cuda.synchronize()
    exp = _expected(z)
    valid = torch.zeros(exp.shape[0], dtype=torch.bool)
    for sl in ol.psum_slices(z['psum'].tolist(), meta['alignment']):
        valid[sl] = True
    out = d.cpu()
    assert torch.equal(out[~valid].view(torch.int16), torch.zeros_like(out[~valid]).view(torch.int16))
    assert og.calc_diff(out[valid], exp[valid]) < 1e-5


@pytest.mark.gpu
def test_kernel_matches_bf16_fixture():
    import deep_gemm
    z, meta = _load('bf16_nt_64x96x128')
    a = torch.from_numpy(z['a']).view(torch.bfloat16).cuda()
    b = torch.from_numpy(z['b']).view(torch.bfloat16).cuda()
    d = torch.empty(meta['m'], meta['n'], dtype=torch.bfloat16, device='cuda')
    deep_gemm.bf16_gemm_nt(a, b, d)
    torch.cuda.synchronize()
    assert og.calc_diff(d.cpu(), _expected(z)) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize('kind', ['fp8', 'bf16'])
def test_bf16_output_is_fp32_output_rounded(kind):
    """The bf16 epilogue is a single round-to-nearest-even of the fp32 result: a bf16 D must
    equal the same GEMM's fp32 D cast by torch, bit for bit (the reference's
    assert_direct_output_matches_fp32_accumulation, tests/utils.py:58-64)."""
    import deep_gemm
    g = torch.Generator().manual_seed(11)
    m, n, k = 200, 300, 512
    if kind == 'fp8':
        a, sfa, _ = quant.random_codes((m, k), 'e4m3', -1, g, (1, 32))
        b, sfb, _ = quant.random_codes((n, k), 'e4m3', -1, g, (1, 32))
        args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()))
        fn = deep_gemm.fp8_gemm_nt
    else:
        a = torch.randn(m, k, generator=g).to(torch.bfloat16).cuda()
        b = torch.randn(n, k, generator=g).to(torch.bfloat16).cuda()
        args = (a, b)
        fn = deep_gemm.bf16_gemm_nt
    d32 = torch.empty(m, n, dtype=torch.float32, device='cuda')
    d16 = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    fn(*args, d32)
    fn(*args, d16)
    torch.cuda.synchronize()
    assert torch.equal(d16.cpu().view(torch.int16), d32.cpu().to(torch.bfloat16).view(torch.int16))


def test_oracle_stochastic_rounding_matches_reference_vectors():
    """Ragged rows (zero-padded quartets), NaN / inf / signed zero / subnormal / max-finite inputs and
    random bit patterns: the oracle's bf16 bits equal those the reference's check accepted."""
    z = np.load(os.path.join(GOLD, 'sr_bf16_reference.npz'), allow_pickle=False)
    n = len(z.files) // 2
    assert n >= 8
    for i in range(n):
        x = torch.from_numpy(z[f'x{i}'].view(np.float32).copy())
        got = oe.stochastic_round_bf16(x).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, z[f'y{i}']), i
