"""FP4 operands packed along MN: dg_fp4_to_k_major (bit-exact against a numpy re-pack of the same
nibbles, ragged MN / K, padded rows, batches) and the GEMMs that take such operands (bit-identical to
the same codes packed along K)."""
import ctypes

import numpy as np
import pytest
import torch

import deep_gemm
from deep_gemm import _lib
from oracle import quant
from helpers import gen, operand

pytestmark = pytest.mark.gpu


def _expected(codes: np.ndarray, kpad: int) -> np.ndarray:
    """codes [B, K, MN] (0..15) -> [B, MN, kpad / 2] bytes packed along K, zero past K."""
    b, k, mn = codes.shape
    c = np.zeros((b, mn, kpad), dtype=np.uint8)
    c[:, :, :k] = codes.transpose(0, 2, 1)
    return (c[:, :, 0::2] | (c[:, :, 1::2] << 4)).astype(np.uint8)


@pytest.mark.parametrize('batches,k,mn,ld_pad', [(1, 64, 128, 0), (1, 100, 250, 0), (3, 130, 257, 7),
                                                 (2, 7, 2, 16), (1, 512, 4096, 0), (4, 33, 384, 32)])
def test_fp4_to_k_major_bit_exact(batches, k, mn, ld_pad):
    print(f'dg_fp4_to_k_major batches={batches} k={k} mn={mn} ld_pad={ld_pad}', flush=True)
    rng = np.random.default_rng(k * 1000 + mn)
    codes = rng.integers(0, 16, size=(batches, k, mn), dtype=np.uint8)
    mnb = (mn + 1) // 2
    cpad = np.zeros((batches, k, mnb * 2), dtype=np.uint8)
    cpad[:, :, :mn] = codes
    packed = (cpad[:, :, 0::2] | (cpad[:, :, 1::2] << 4)).astype(np.uint8)   # [B, K, MN/2]
    ld = mnb + ld_pad
    src_np = np.full((batches, k, ld), 0xAB, dtype=np.uint8)                  # padding bytes never read
    src_np[:, :, :mnb] = packed
    src = torch.from_numpy(src_np).cuda()
    kpad = (k + 31) // 32 * 32
    dst = torch.full((batches, mn, kpad // 2), 0x55, dtype=torch.uint8, device='cuda')
    lib = _lib.load()
    rc = lib.dg_fp4_to_k_major(src.data_ptr(), batches, k * ld, ld, k, mn, dst.data_ptr(), mn * kpad // 2,
                               kpad // 2, kpad, None)
    assert rc == 0, lib.dg_last_error()
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), _expected(codes, kpad))


def test_fp4_to_k_major_rejects_bad_arguments():
    lib = _lib.load()
    buf = torch.zeros(4096, dtype=torch.uint8, device='cuda')
    # destination rows not 16-byte aligned
    assert lib.dg_fp4_to_k_major(buf.data_ptr(), 1, 0, 64, 64, 128, buf.data_ptr(), 0, 40, 64, None) != 0
    assert b'16-byte' in lib.dg_last_error()
    # odd k_padded
    assert lib.dg_fp4_to_k_major(buf.data_ptr(), 1, 0, 64, 63, 128, buf.data_ptr(), 0, 48, 63, None) != 0


@pytest.mark.parametrize('m,n,k', [(128, 256, 512), (64, 384, 4096), (300, 130, 2048)])
def test_fp8_fp4_gemm_b_packed_along_n_matches_k_packed(m, n, k):
    """The same e2m1 codes of B, packed along N (re-packed by the kernel above) or along K: the
    GEMM results are bit-identical."""
    print(f'fp8_fp4 B packed along N m={m} n={n} k={k}', flush=True)
    g = gen(m + n + k)
    a, sfa, _ = operand(m, k, 'e4m3', (1, 32), g)
    b_mn, sfb, _ = quant.random_codes((n, k), 'e2m1', 0, g, (1, 32))   # [N/2 packed, K] view, N-major
    u = b_mn.transpose(0, 1).contiguous().view(torch.uint8)            # [K, N/2] bytes
    codes = torch.stack((u & 0x0f, u >> 4), dim=-1).reshape(k, n).t()   # nibble codes [N, K]
    b_k = quant.pack_fp4(codes, 1)                                      # the same codes packed along K
    d_mn = torch.empty(m, n, dtype=torch.bfloat16, device='cuda')
    d_k = torch.empty_like(d_mn)
    deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b_mn.cuda(), sfb.cuda()), d_mn)
    deep_gemm.fp8_fp4_gemm_nt((a.cuda(), sfa.cuda()), (b_k.cuda(), sfb.cuda()), d_k)
    torch.cuda.synchronize()
    assert torch.equal(d_mn.view(torch.int16), d_k.view(torch.int16))
