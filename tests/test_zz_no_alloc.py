"""dg_gemm_noalloc (the allocation-free dg_gemm: split-K scratch in a fixed device array) against
dg_gemm with a caller workspace, through the C ABI: the same plan, bit-identical D, on two calls in
a row (the second smaller), plus the oracle and the over-size rejection."""
import ctypes

import pytest
import torch

import deep_gemm
from deep_gemm import _lib
from oracle import gemm as og
from helpers import gen, operand, calc_diff

pytestmark = pytest.mark.gpu


def _args(m, n, k, seed):
    """Filled dg_gemm_args (K-major e4m3 A / B, packed SF) and the tensors it points at."""
    g = gen(seed)
    a, sfa, a_deq = operand(m, k, 'e4m3', (1, 128), g, 'randn')
    b, sfb, b_deq = operand(n, k, 'e4m3', (128, 128), g, 'randn')
    a, b = a.cuda(), b.cuda()
    sfa_t = deep_gemm.transform_sf_into_required_layout(sfa.cuda(), m, k, (1, 128), is_sfa=True)
    sfb_t = deep_gemm.transform_sf_into_required_layout(sfb.cuda(), n, k, (128, 128), is_sfa=False)
    args = _lib.GemmArgs()
    args.kind, args.gemm_type, args.m, args.n, args.k, args.num_groups = _lib.DG_KIND_FP8_FP8, _lib.DG_GEMM_NORMAL, m, n, k, 1
    args.a, args.b, args.sfa, args.sfb = a.data_ptr(), b.data_ptr(), sfa_t.data_ptr(), sfb_t.data_ptr()
    args.lda, args.ldb, args.ldd = a.stride(0), b.stride(0), n
    args.sfa_ld, args.sfb_ld = sfa_t.stride(-1), sfb_t.stride(-1)
    args.d_dtype, args.alpha, args.alignment = _lib.DG_DTYPE_BF16, 1.0, 256
    keep = (a, b, sfa_t, sfb_t)
    return args, keep, og.gemm_nt(a_deq, b_deq)


def _run(lib, args, noalloc):
    d = torch.empty(args.m, args.n, dtype=torch.bfloat16, device='cuda')
    args.d = d.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        args.workspace, args.workspace_bytes = None, 0
        rc = lib.dg_gemm_noalloc(ctypes.byref(args), ctypes.c_void_p(stream))
        ws = None
    else:
        nbytes = ctypes.c_int64(0)
        _lib.check(lib.dg_gemm_workspace_size(ctypes.byref(args), ctypes.byref(nbytes)), lib)
        ws = torch.zeros(max(nbytes.value, 1), dtype=torch.uint8, device='cuda')
        args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes.value
        rc = lib.dg_gemm(ctypes.byref(args), ctypes.c_void_p(stream))
    _lib.check(rc, lib)
    torch.cuda.synchronize()
    return d.cpu()


def test_noalloc_matches_dg_gemm_on_two_calls():
    lib = _lib.load()
    # a split-K decode plan, then a smaller one (the array keeps the first call's contents)
    # (128 x 2112 x 7168 takes the shared-ring decode kernel, the others the skinny kernel)
    for (m, n, k), seed in (((128, 2112, 7168), 5), ((64, 4096, 7168), 1), ((8, 2112, 4096), 2)):
        args, keep, ref = _args(m, n, k, seed)
        info = _lib.LaunchInfo()
        args.workspace, args.workspace_bytes = 1, 1 << 40   # plan as for a caller with a workspace
        _lib.check(lib.dg_launch_plan(ctypes.byref(args), ctypes.byref(info)), lib)
        args.workspace, args.workspace_bytes = None, 0
        print(f'noalloc m={m} n={n} k={k} split_k={info.split_k} skinny={info.skinny}', flush=True)
        assert info.split_k > 1, 'the case must exercise the split-K scratch'
        d_noalloc = _run(lib, args, True)
        d_ws = _run(lib, args, False)
        assert torch.equal(d_noalloc, d_ws)
        assert calc_diff(d_noalloc, ref) < 1e-5
        # again, now that the array holds this call's counters and partials
        assert torch.equal(_run(lib, args, True), d_ws)


def test_noalloc_gemv_plan():
    """A decode GEMM that plans the GEMV kernel (no scratch at all): dg_gemm_noalloc matches dg_gemm bit for
    bit on two calls in a row (the second with fewer rows of B) and the oracle."""
    lib = _lib.load()
    for (m, n, k), seed in (((1, 2112, 7168), 6), ((1, 1000, 4096), 7)):
        args, keep, ref = _args(m, n, k, seed)
        info = _lib.LaunchInfo()
        _lib.check(lib.dg_launch_plan(ctypes.byref(args), ctypes.byref(info)), lib)
        print(f'noalloc gemv m={m} n={n} k={k} skinny={info.skinny} split_k={info.split_k}', flush=True)
        assert info.skinny == 3 and info.split_k == 1
        d_noalloc = _run(lib, args, True)
        d_ws = _run(lib, args, False)
        assert torch.equal(d_noalloc.view(torch.int16), d_ws.view(torch.int16))
        assert calc_diff(d_noalloc, ref) < 1e-5


def test_noalloc_rejects_oversize_and_a_workspace():
    lib = _lib.load()
    args, keep, _ = _args(128, 8192, 16384, 3)
    d = torch.empty(128, 8192, dtype=torch.bfloat16, device='cuda')
    args.d = d.data_ptr()
    args.split_k = 16   # forced: 16 K ranges of every strip need more than the fixed array
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.dg_gemm_noalloc(ctypes.byref(args), ctypes.c_void_p(stream)) != 0
    assert b'maximum' in lib.dg_last_error()
    args.split_k = 0
    args.workspace, args.workspace_bytes = d.data_ptr(), 16
    assert lib.dg_gemm_noalloc(ctypes.byref(args), ctypes.c_void_p(stream)) != 0
    assert b'library provides the workspace' in lib.dg_last_error()


def test_noalloc_m_indices_run_table_in_scratch():
    _check_m_indices_noalloc()


def _check_m_indices_noalloc():
    """M-grouped m_indices GEMMs below alignment 256 take the anchored tiles, whose run table
    dg_gemm_noalloc keeps in its scratch array: bit-identical to dg_gemm (which keeps it in the
    library's per-stream buffer), on two calls in a row, the second with fewer rows."""
    from oracle import layout as ol
    lib = _lib.load()
    alignment, g_num, n, k = 128, 4, 320, 512
    keep_alive = []
    for sizes, seed in (([257, 0, 130, 400], 3), ([5, 128], 4)):
        total, ps = ol.psum_from_sizes(sizes, alignment)
        idx = ol.m_indices_from_psum(ps, alignment, total).cuda()
        g = gen(seed)
        a, sfa, a_deq = operand(total, k, 'e4m3', (1, 32), g)
        b, sfb, b_deq = operand(n, k, 'e4m3', (1, 32), g, batch=g_num)
        a, b = a.cuda(), b.cuda()
        sfa_t = deep_gemm.transform_sf_into_required_layout(sfa.cuda(), total, k, (1, 32), is_sfa=True)
        sfb_t = deep_gemm.transform_sf_into_required_layout(sfb.cuda(), n, k, (1, 32), num_groups=g_num, is_sfa=False)
        args = _lib.GemmArgs()
        args.kind, args.gemm_type = _lib.DG_KIND_FP8_FP8, _lib.DG_GEMM_MGROUPED_IDX
        args.m, args.n, args.k, args.num_groups = total, n, k, g_num
        args.a, args.b, args.sfa, args.sfb = a.data_ptr(), b.data_ptr(), sfa_t.data_ptr(), sfb_t.data_ptr()
        args.lda, args.ldb, args.ldd = a.stride(0), b.stride(1), n
        args.batch_stride_b, args.sfb_batch_stride = b.stride(0), sfb_t.stride(0)
        args.sfa_ld, args.sfb_ld = sfa_t.stride(-1), sfb_t.stride(-1)
        args.grouped_layout = idx.data_ptr()
        args.d_dtype, args.alpha, args.alignment = _lib.DG_DTYPE_BF16, 1.0, alignment
        keep_alive.append((a, b, sfa_t, sfb_t, idx))
        info = _lib.LaunchInfo()
        _lib.check(lib.dg_launch_plan(ctypes.byref(args), ctypes.byref(info)), lib)
        print(f'noalloc m_indices sizes={sizes} block={info.block_m}x{info.block_n}', flush=True)
        assert (info.block_m, info.block_n) == (384, 192)
        d_noalloc = _run(lib, args, True)
        d_lib = _run(lib, args, False)
        assert torch.equal(d_noalloc, d_lib)
        valid = idx.cpu() >= 0
        ref = og.m_grouped_contiguous(a_deq, b_deq, idx.cpu(), False, alignment)
        assert calc_diff(d_noalloc[valid], ref[valid]) < 1e-5
        assert torch.equal(d_noalloc[~valid], torch.zeros_like(d_noalloc[~valid]))
    return keep_alive


def test_noalloc_split_k_after_m_indices():
    """The run table of an m_indices call must not land on the split-K tile counters (which every
    split-K call needs at zero): an anchored m_indices dg_gemm_noalloc call, then the 128x2112x7168
    split-K plan twice, each bit-identical to dg_gemm with its own zeroed workspace."""
    keep = _check_m_indices_noalloc()
    lib = _lib.load()
    args, keep2, ref = _args(128, 2112, 7168, 5)
    info = _lib.LaunchInfo()
    args.workspace, args.workspace_bytes = 1, 1 << 40
    _lib.check(lib.dg_launch_plan(ctypes.byref(args), ctypes.byref(info)), lib)
    args.workspace, args.workspace_bytes = None, 0
    print(f'noalloc split-K after m_indices: split_k={info.split_k}', flush=True)
    assert info.split_k > 1
    d_ws = _run(lib, args, False)
    for _ in range(2):
        assert torch.equal(_run(lib, args, True), d_ws)
    assert calc_diff(d_ws, ref) < 1e-5


def test_noalloc_mn_major_b_decode():
    """A split-K decode plan with MN-major B ([K][N], read in place by the skinny kernel): dg_gemm_noalloc
    matches dg_gemm bit for bit on two calls in a row (the second smaller) and the oracle."""
    lib = _lib.load()
    for (m, n, k), seed in (((64, 2112, 7168), 8), ((16, 1000, 4096), 9)):
        args, keep, ref = _args(m, n, k, seed)
        ldb = -(-n // 16) * 16   # (K rows of B 16-byte aligned)
        b_kn = torch.zeros(k, ldb, dtype=torch.uint8, device='cuda')   # [K, N] in a wider buffer
        b_kn[:, :n] = keep[1].view(torch.uint8).t()
        args.b, args.ldb, args.b_mn_major = b_kn.data_ptr(), ldb, 1
        info = _lib.LaunchInfo()
        args.workspace, args.workspace_bytes = 1, 1 << 40
        _lib.check(lib.dg_launch_plan(ctypes.byref(args), ctypes.byref(info)), lib)
        args.workspace, args.workspace_bytes = None, 0
        print(f'noalloc mn-major B m={m} n={n} k={k} split_k={info.split_k} skinny={info.skinny}', flush=True)
        assert info.skinny == 1 and info.split_k > 1
        d_noalloc = _run(lib, args, True)
        d_ws = _run(lib, args, False)
        assert torch.equal(d_noalloc, d_ws)
        assert calc_diff(d_noalloc, ref) < 1e-5
        assert torch.equal(_run(lib, args, True), d_ws)
