"""GPU parity of the output epilogues through libdeep_gemm_amd.so.

* BF16StochasticRounding: bit-exact against the hash of the same GEMM's fp32 output
  (the reference's check, tests/utils.py:70-92 and tests/common.py:211-218), for dense,
  M-grouped, K-grouped, batched and einsum launches, aligned and ragged N.
* FP8 output (an (e4m3 D, SFD) pair / FP8Quantization): bit-exact against quantising the
  bf16 D of the same GEMM per (row, 32 columns) (tests/test_einsum.py:70-86).
"""
import pytest
import torch

import deep_gemm
from oracle import epilogue as oe, layout as ol
from helpers import gen, operand

pytestmark = pytest.mark.gpu


def _bits16(t):
    return t.cpu().view(torch.int16)


def _fp8_operands(m, n, k, seed, batch=0):
    g = gen(seed)
    a, sfa, _ = operand(m, k, 'e4m3', (1, 32), g, 'randn', batch=batch)
    b, sfb, _ = operand(n, k, 'e4m3', (1, 32), g, 'randn', batch=batch)
    return (a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda())


@pytest.mark.parametrize('m,n,k', [(256, 384, 512), (130, 250, 640), (4096, 7168, 2048), (64, 2112, 7168)])
def test_sr_dense_fp8(m, n, k):
    print(f'SR dense m={m} n={n} k={k}', flush=True)
    a, b = _fp8_operands(m, n, k, seed=m)
    f32 = torch.empty(m, n, device='cuda')
    deep_gemm.fp8_gemm_nt(a, b, f32)
    out = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_gemm_nt(a, b, out, epilogue=deep_gemm.epilogue.BF16StochasticRounding())
    torch.cuda.synchronize()
    assert torch.equal(_bits16(out), _bits16(oe.stochastic_round_bf16(f32)))


def test_sr_dense_bf16_and_fp4():
    m, n, k = 200, 320, 256
    g = gen(3)
    a = torch.randn(m, k, generator=g).bfloat16().cuda()
    b = torch.randn(n, k, generator=g).bfloat16().cuda()
    f32 = torch.empty(m, n, device='cuda')
    deep_gemm.bf16_gemm_nt(a, b, f32)
    out = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.bf16_gemm_nt(a, b, out, epilogue=deep_gemm.epilogue.BF16StochasticRounding())
    torch.cuda.synchronize()
    assert torch.equal(_bits16(out), _bits16(oe.stochastic_round_bf16(f32)))
    a4, sfa4, _ = operand(m, k, 'e2m1', (1, 32), g, 'codes')
    b4, sfb4, _ = operand(n, k, 'e2m1', (1, 32), g, 'codes')
    args = ((a4.cuda(), sfa4.cuda()), (b4.cuda(), sfb4.cuda()))
    deep_gemm.fp8_fp4_gemm_nt(*args, f32)
    deep_gemm.fp8_fp4_gemm_nt(*args, out, epilogue=deep_gemm.epilogue.BF16StochasticRounding())
    torch.cuda.synchronize()
    assert torch.equal(_bits16(out), _bits16(oe.stochastic_round_bf16(f32)))


def test_sr_m_grouped_contiguous():
    sizes, n, k = [300, 0, 77, 512], 256, 512
    total, psum = ol.psum_from_sizes(sizes, 256)
    g = gen(4)
    a, sfa, _ = operand(total, k, 'e4m3', (1, 32), g, 'randn')
    b, sfb, _ = operand(n, k, 'e4m3', (1, 32), g, 'randn', batch=len(sizes))
    for sl in ol.psum_pad_slices(psum, 256):
        a.view(torch.uint8)[sl] = 0
    layout = torch.tensor(psum, dtype=torch.int32, device='cuda')
    args = ((a.cuda(), sfa.cuda()), (b.cuda(), sfb.cuda()))
    f32 = torch.empty(total, n, device='cuda')
    deep_gemm.m_grouped_fp8_gemm_nt_contiguous(*args, f32, layout)
    out = torch.empty(total, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.m_grouped_fp8_gemm_nt_contiguous(*args, out, layout,
                                               epilogue=deep_gemm.epilogue.BF16StochasticRounding())
    torch.cuda.synchronize()
    assert torch.equal(_bits16(out), _bits16(oe.stochastic_round_bf16(f32)))


def test_sr_k_grouped():
    """The reference compares against an fp32 launch that accumulates into zeros
    (tests/common.py:211-218)."""
    from test_batched_kgrouped_gpu import _k_grouped_case
    m, n, ks = 256, 384, [512, 300, 0, 1000]
    psum, a_tn, sfa, _, b_tn, sfb, _ = _k_grouped_case(m, n, ks, seed=5)
    layout = torch.tensor(psum, dtype=torch.int32, device='cuda')
    args = ((a_tn.cuda(), sfa.cuda()), (b_tn.cuda(), sfb.cuda()))
    f32 = torch.zeros(len(ks), m, n, device='cuda')
    deep_gemm.k_grouped_fp8_gemm_tn_contiguous(*args, f32, ks, layout, c=f32)
    out = torch.empty(len(ks), m, n, dtype=torch.bfloat16, device='cuda')
    deep_gemm.k_grouped_fp8_gemm_tn_contiguous(*args, out, ks, layout,
                                               epilogue=deep_gemm.epilogue.BF16StochasticRounding())
    torch.cuda.synchronize()
    assert torch.equal(_bits16(out), _bits16(oe.stochastic_round_bf16(f32)))


@pytest.mark.parametrize('expr', ['bhd,hdr->bhr', 'bhd,bhr->hdr'])
def test_sr_einsum_bf16(expr):
    """dgrad / wgrad roles (tests/test_einsum.py:90-93)."""
    B, H, D, R = 96, 3, 128, 200
    sizes = {'b': B, 'h': H, 'd': D, 'r': R}
    ins, outs = expr.split('->')
    ta, tb = ins.split(',')
    g = gen(6)
    a = torch.randn([sizes[x] for x in ta], generator=g).bfloat16().cuda()
    b = torch.randn([sizes[x] for x in tb], generator=g).bfloat16().cuda()
    f32 = torch.empty([sizes[x] for x in outs], device='cuda')
    deep_gemm.einsum(expr, a, b, f32)
    out = torch.empty_like(f32, dtype=torch.bfloat16)
    deep_gemm.einsum(expr, a, b, out, epilogue=deep_gemm.epilogue.BF16StochasticRounding())
    torch.cuda.synchronize()
    assert torch.equal(_bits16(out), _bits16(oe.stochastic_round_bf16(f32)))


@pytest.mark.parametrize('b,h,r,d', [(4, 8, 128, 128), (13, 8, 512, 256), (4096, 2, 128, 128),
                                     (1, 3, 128, 128), (13, 3, 128, 384), (257, 2, 128, 128)])
def test_fp8_einsum_fp8_output(b, h, r, d):
    """The reference's own shape list (tests/test_einsum.py:110-112)."""
    print(f'fp8 output einsum b={b} h={h} r={r} d={d}', flush=True)
    g = gen(b + h)
    a_v, sfa_v, _ = operand(b, r, 'e4m3', (1, 32), g, 'randn', batch=h)     # [h, b, r]
    B_, sfb, _ = operand(d, r, 'e4m3', (1, 32), g, 'randn', batch=h)        # [h, d, r]
    A = a_v.permute(1, 0, 2).contiguous().cuda()                             # [b, h, r]
    sfa = sfa_v.permute(1, 0, 2).contiguous().cuda()
    args = ((A, sfa), (B_.cuda(), sfb.cuda()))
    D = torch.empty(b, h, d, dtype=torch.bfloat16, device='cuda')
    deep_gemm.fp8_einsum('bhr,hdr->bhd', *args, D)
    output = torch.empty(b, h, d, dtype=torch.float8_e4m3fn, device='cuda')
    sfd = torch.empty_strided((b, h * d // 64), (1, b), device='cuda', dtype=torch.int16)
    deep_gemm.fp8_einsum('bhr,hdr->bhd', *args, (output, sfd))
    torch.cuda.synchronize()
    ref_fp8, ref_sfd = oe.quantize_fp8_output(D.cpu().reshape(b, h * d))
    assert torch.equal(output.cpu().view(torch.uint8).reshape(b, h * d), ref_fp8.view(torch.uint8))
    assert torch.equal(sfd.cpu(), ref_sfd)


def test_fp8_bmm_fp8quantization_epilogue_class():
    """The same output through fp8_bmm with FP8Quantization(sfd) and D stored [M, B, N]."""
    bs, m, n, k = 3, 192, 256, 384
    a, b = _fp8_operands(m, n, k, seed=9, batch=bs)
    d_bf16 = torch.empty(m, bs, n, dtype=torch.bfloat16, device='cuda').transpose(0, 1)
    deep_gemm.fp8_bmm(a, b, d_bf16)
    out = torch.empty(m, bs, n, dtype=torch.float8_e4m3fn, device='cuda').transpose(0, 1)
    sfd = torch.empty_strided((m, bs * n // 64), (1, m), device='cuda', dtype=torch.int16)
    deep_gemm.fp8_bmm(a, b, out, epilogue=deep_gemm.epilogue.FP8Quantization(sfd))
    torch.cuda.synchronize()
    ref_fp8, ref_sfd = oe.quantize_fp8_output(d_bf16.transpose(0, 1).cpu().reshape(m, bs * n))
    assert torch.equal(out.transpose(0, 1).cpu().view(torch.uint8).reshape(m, bs * n), ref_fp8.view(torch.uint8))
    assert torch.equal(sfd.cpu(), ref_sfd)
