"""Writes the small golden fixtures in this directory from the CPU oracle.

The reference ships no golden vectors for this path, so these fixtures pin the oracle
(and the GPU kernels, through tests/test_golden.py) against regressions: seeded inputs,
the expected outputs as raw bits.  Regenerate with `python tests/golden/make_golden.py`.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import quant, layout as ol, gemm as og  # noqa: E402


def _u8(t):
    return t.contiguous().view(torch.uint8).numpy()


def fp8_gemm_case(name, m, n, k, gran_a, gran_b, kind_b='e4m3', mode='codes', seed=0):
    g = torch.Generator().manual_seed(seed)
    if mode == 'codes':
        a, sfa, a_deq = quant.random_codes((m, k), 'e4m3', -1, g, gran_a)
        b, sfb, b_deq = quant.random_codes((n, k), kind_b, -1, g, gran_b)
    else:
        a, sfa, a_deq = quant.quantize_blockwise(torch.randn(m, k, generator=g), gran_a, 'e4m3')
        b, sfb, b_deq = quant.quantize_blockwise(torch.randn(n, k, generator=g), gran_b, kind_b)
    d = og.gemm_nt(a_deq, b_deq)
    np.savez_compressed(os.path.join(HERE, name + '.npz'), a=_u8(a), sfa=sfa.numpy(), b=_u8(b), sfb=sfb.numpy(),
                        d_bits=d.view(torch.int16).numpy(),
                        meta=json.dumps(dict(m=m, n=n, k=k, gran_a=gran_a, gran_b=gran_b, kind_b=kind_b)))


def transform_case(name, mn, k, gran_mn, gran_k, psum=None, alignment=256, seed=0):
    g = torch.Generator().manual_seed(seed)
    e = torch.randint(1, 255, ((mn + gran_mn - 1) // gran_mn, (k + gran_k - 1) // gran_k), generator=g, dtype=torch.int32)
    sf = (e << 23).view(torch.float32)
    out = ol.transform_sf(sf, mn, k, gran_mn, gran_k, psum=psum, alignment=alignment)
    np.savez_compressed(os.path.join(HERE, name + '.npz'), sf=sf.numpy(), out=out.contiguous().numpy(),
                        meta=json.dumps(dict(mn=mn, k=k, gran_mn=gran_mn, gran_k=gran_k, psum=psum, alignment=alignment)))


def grouped_case(name, sizes, n, k, alignment, seed=0):
    g = torch.Generator().manual_seed(seed)
    total, ps = ol.psum_from_sizes(sizes, alignment)
    a, sfa, a_deq = quant.random_codes((total, k), 'e4m3', -1, g, (1, 32))
    for sl in ol.psum_pad_slices(ps, alignment):
        a.view(torch.uint8)[sl] = 0
        a_deq[sl] = 0
    b, sfb, b_deq = quant.random_codes((len(sizes), n, k), 'e4m3', -1, g, (1, 1, 32))
    d = og.m_grouped_contiguous(a_deq, b_deq, torch.tensor(ps), True, alignment)
    np.savez_compressed(os.path.join(HERE, name + '.npz'), a=_u8(a), sfa=sfa.numpy(), b=_u8(b), sfb=sfb.numpy(),
                        psum=np.array(ps, dtype=np.int32), d_bits=d.view(torch.int16).numpy(),
                        meta=json.dumps(dict(sizes=sizes, n=n, k=k, alignment=alignment)))


def bf16_case(name, m, n, k, seed=0):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(m, k, generator=g) * 0.1).to(torch.bfloat16)
    b = (torch.randn(n, k, generator=g) * 0.1).to(torch.bfloat16)
    d = og.gemm_nt(a.float(), b.float())
    np.savez_compressed(os.path.join(HERE, name + '.npz'), a=a.view(torch.int16).numpy(), b=b.view(torch.int16).numpy(),
                        d_bits=d.view(torch.int16).numpy(), meta=json.dumps(dict(m=m, n=n, k=k)))


if __name__ == '__main__':
    fp8_gemm_case('fp8_nt_codes_96x160x384', 96, 160, 384, (1, 32), (1, 32))
    fp8_gemm_case('fp8_nt_randn_128x256x512_1x128_128x128', 128, 256, 512, (1, 128), (128, 128), mode='randn', seed=1)
    fp8_gemm_case('fp8_fp4_nt_codes_64x128x256', 64, 128, 256, (1, 32), (1, 32), kind_b='e2m1', seed=2)
    transform_case('transform_sf_300x1000_g1', 300, 1000, 1, 32, seed=3)
    transform_case('transform_sf_300x1000_g128_k128', 300, 1000, 128, 128, seed=4)
    transform_case('transform_sf_psum_640x512', 640, 512, 1, 32, psum=[5, 128, 258, 385], alignment=128, seed=5)
    grouped_case('m_grouped_psum_3g_64x128', [50, 0, 130], 64, 128, 128, seed=6)
    bf16_case('bf16_nt_64x96x128', 64, 96, 128, seed=7)
    print('fixtures written to', HERE)
