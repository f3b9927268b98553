"""C ABI of libdeep_gemm_amd.so: loads without a GPU, exports every symbol the header
declares, and rejects bad arguments with error codes (no kernel is launched here)."""
import ctypes
import re
from pathlib import Path

import pytest

from deep_gemm import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / 'include' / 'deep_gemm_amd.h'


@pytest.fixture(scope='module')
def lib():
    path = _lib.library_path()
    if not path.exists():
        import importlib.util
        spec = importlib.util.spec_from_file_location('dg_build', ROOT / 'deepgemm-ascend_amd' / 'build.py')
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return _lib.load()


def _declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r'^\s*(?:int|uint32_t|const char \*|const uint32_t \*)\s*(dg_\w+)\s*\(', text, re.M)))


def test_header_declares_the_binding_table():
    assert _declared_symbols() == sorted(_lib.EXPORTED_SYMBOLS)


def test_every_declared_symbol_is_exported(lib):
    for name in _declared_symbols():
        assert hasattr(lib, name), name


def test_version_and_empty_error(lib):
    assert b'gfx950' in lib.dg_version()
    assert lib.dg_last_error() is not None


def test_gemm_rejects_null_and_bad_kind(lib):
    assert lib.dg_gemm(None, None) == -1
    assert b'null args' in lib.dg_last_error()
    args = _lib.GemmArgs()
    args.kind = 9
    assert lib.dg_gemm(ctypes.byref(args), None) == -1
    assert b'unknown kind' in lib.dg_last_error()


def test_gemm_rejects_misaligned_rows(lib):
    args = _lib.GemmArgs()
    args.kind, args.gemm_type, args.m, args.n, args.k = 0, 0, 64, 64, 100   # K=100 bytes: not 16-aligned
    args.a = args.b = args.d = 4096
    args.sfa = args.sfb = 4096
    args.lda = args.ldb = 100
    args.ldd = 64
    assert lib.dg_gemm(ctypes.byref(args), None) == -1
    assert b'16-byte aligned' in lib.dg_last_error()


def test_gemm_zero_size_is_a_noop(lib):
    args = _lib.GemmArgs()
    args.kind, args.m, args.n, args.k = 0, 0, 64, 128
    assert lib.dg_gemm(ctypes.byref(args), None) == 0


def test_grouped_requires_layout(lib):
    args = _lib.GemmArgs()
    args.kind, args.gemm_type, args.m, args.n, args.k, args.num_groups = 0, 2, 256, 256, 128, 4
    args.a = args.b = args.d = args.sfa = args.sfb = 4096
    args.lda = args.ldb = 128
    args.ldd = 256
    args.alignment = 256
    assert lib.dg_gemm(ctypes.byref(args), None) == -1
    assert b'grouped_layout required' in lib.dg_last_error()


def test_select_config_respects_grouped_alignment(lib):
    """M-grouped layouts take a block_m dividing the alignment, except the tiles anchored at each
    group's or run's first row (384 rows), taken when the alignment rules out 256-row tiles."""
    for gemm_type in (2, 3):
        for align in (256, 128, 64, 32):
            args = _lib.GemmArgs()
            args.kind, args.gemm_type, args.m, args.n, args.k, args.num_groups = 0, gemm_type, 8192, 4096, 7168, 32
            args.alignment, args.num_cus = align, 256
            bm, bn = ctypes.c_int32(), ctypes.c_int32()
            assert lib.dg_select_config(ctypes.byref(args), ctypes.byref(bm), ctypes.byref(bn)) == 0
            if align < 256:
                assert (bm.value, bn.value) == (384, 192)
            else:
                assert align % bm.value == 0 and bn.value > 0


def test_fp4_grouped_plans_skip_anchored_tiles(lib):
    """M-grouped FP8 x FP4 / FP4 x FP4 layouts below alignment 256 take the 384x128 anchored tiles (the 384x192
    build spills for e2m1 B), at alignment 256 scored tiles whose block_m divides it; no layout scores an
    anchored tile at alignment 256."""
    for kind in (1, 2):
        for align in (128, 256):
            args = _lib.GemmArgs()
            args.kind, args.gemm_type, args.m, args.n, args.k, args.num_groups = kind, 2, 8192, 4096, 7168, 32
            args.alignment, args.num_cus = align, 256
            bm, bn = ctypes.c_int32(), ctypes.c_int32()
            assert lib.dg_select_config(ctypes.byref(args), ctypes.byref(bm), ctypes.byref(bn)) == 0
            if align == 128:
                assert (bm.value, bn.value) == (384, 128), (kind, align, bm.value, bn.value)
            else:
                assert bm.value <= 256 and align % bm.value == 0, (kind, align, bm.value, bn.value)
    args = _lib.GemmArgs()
    args.kind, args.gemm_type, args.m, args.n, args.k, args.num_groups = 0, 2, 32768, 7168, 3072, 8
    args.alignment, args.num_cus = 256, 256
    bm, bn = ctypes.c_int32(), ctypes.c_int32()
    assert lib.dg_select_config(ctypes.byref(args), ctypes.byref(bm), ctypes.byref(bn)) == 0
    assert bm.value <= 256, (bm.value, bn.value)


def test_transform_sf_argument_checks(lib):
    f = lib.dg_transform_sf
    # gran_mn not a power of two
    assert f(4096, 0, 0, 1, 1, 1, 10, 1, 30, 32, 3, 32, None, 0, 256, 4096, 0, None, None) == -1
    assert b'power of two' in lib.dg_last_error()
    # fp32 SF with gran_k 64
    assert f(4096, 0, 0, 1, 1, 1, 10, 1, 10, 64, 1, 64, None, 0, 256, 4096, 0, None, None) == -1
    # wrong sf_k extent
    assert f(4096, 0, 0, 1, 1, 1, 10, 5, 10, 64, 1, 32, None, 0, 256, 4096, 0, None, None) == -1
    assert b'sf_k' in lib.dg_last_error()
    # psum with an alignment that gran_mn does not divide
    assert f(4096, 0, 0, 1, 1, 1, 1, 2, 128, 64, 128, 32, 4096, 2, 64, 4096, 0, None, None) == -1


def _plan_args(m, n, k, num_cus):
    args = _lib.GemmArgs()
    args.kind, args.gemm_type, args.m, args.n, args.k, args.num_groups = 0, 0, m, n, k, 1
    args.lda, args.ldb, args.ldd = k, k, n
    args.sfa_ld, args.sfb_ld = (m + 1) // 2 * 2, (n + 1) // 2 * 2
    args.alignment, args.num_cus = 256, num_cus
    return args


def test_launch_plan_without_device(lib):
    """dg_launch_plan describes the launch and touches no device: one workgroup per tile at the
    full CU count; under a set_num_sms cap (below the 256 CUs of MI355X the library assumes when it
    cannot query a device) at most num_cus workgroups, each serving plan workgroups in turn."""
    full = _lib.LaunchInfo()
    assert lib.dg_launch_plan(_plan_args(4096, 7168, 2048, 0), ctypes.byref(full)) == 0, lib.dg_last_error()
    assert full.persistent == 0 and full.grid == full.tiles == full.plan_workgroups and full.block_m == 256
    capped = _lib.LaunchInfo()
    assert lib.dg_launch_plan(_plan_args(4096, 7168, 2048, 64), ctypes.byref(capped)) == 0, lib.dg_last_error()
    assert capped.grid == 64 and capped.tiles > 64 and capped.plan_workgroups >= capped.grid
    small = _lib.LaunchInfo()
    assert lib.dg_launch_plan(_plan_args(1, 2112, 7168, 64), ctypes.byref(small)) == 0, lib.dg_last_error()
    assert small.skinny in (1, 3) and small.persistent == 0 and small.grid <= 64
    # decode shapes with 64 < M <= 128 and K <= 8192 take the shared-ring decode kernel
    mid = _lib.LaunchInfo()
    assert lib.dg_launch_plan(_plan_args(128, 2112, 7168, 0), ctypes.byref(mid)) == 0, lib.dg_last_error()
    assert mid.skinny == 2 and mid.threads == 256 and mid.block_m == 64 and mid.block_n == 64
    assert mid.split_reduce == 0
    # long K over many columns: 64-column strips, the split-K partials summed by a second launch
    # (only where the call can split K: here with the library's per-stream workspace)
    wide = _lib.LaunchInfo()
    wide_args = _plan_args(128, 4096, 7168, 0)
    wide_args.library_workspace = 1
    assert lib.dg_launch_plan(wide_args, ctypes.byref(wide)) == 0, lib.dg_last_error()
    assert wide.skinny == 2 and wide.threads == 512 and wide.block_n == 64 and wide.split_reduce == 1
    assert 2 <= wide.split_k <= 4
    long_k = _lib.LaunchInfo()
    assert lib.dg_launch_plan(_plan_args(128, 7168, 16384, 0), ctypes.byref(long_k)) == 0, lib.dg_last_error()
    assert long_k.skinny == 1
    # (with a workspace the wide two-launch plan takes it, up to K = 16384; from K = 8192 over N >= 7168 with
    # 128-column strips)
    long_args = _plan_args(128, 7168, 16384, 0)
    long_args.library_workspace = 1
    assert lib.dg_launch_plan(long_args, ctypes.byref(long_k)) == 0, lib.dg_last_error()
    assert long_k.skinny == 2 and long_k.block_n == 128 and long_k.split_reduce == 1   # (128-column strips)
    # e4m3 M <= 64 with K > 8192 over many columns: 64 x 128 shared-ring tiles, two launches
    m64 = _lib.LaunchInfo()
    m64_args = _plan_args(64, 7168, 16384, 0)
    m64_args.library_workspace = 1
    assert lib.dg_launch_plan(m64_args, ctypes.byref(m64)) == 0, lib.dg_last_error()
    assert m64.skinny == 2 and (m64.block_m, m64.block_n) == (64, 128) and m64.split_reduce == 1 and m64.split_k > 1
    assert lib.dg_launch_plan(_plan_args(64, 7168, 7168, 0), ctypes.byref(m64)) == 0, lib.dg_last_error()
    assert m64.skinny == 1
    # bf16 from K > 4096: 64 x 128 tiles from N >= 6144, 64 x 64 below, the skinny kernel under N = 3072
    for (n, k), want in (((7168, 16384), (2, 64, 128)), ((4096, 7168), (2, 64, 64)), ((2112, 7168), (1, None, None))):
        bf = _plan_args(64, n, k, 0)
        bf.kind, bf.library_workspace = _lib.DG_KIND_BF16, 1
        assert lib.dg_launch_plan(bf, ctypes.byref(m64)) == 0, lib.dg_last_error()
        assert m64.skinny == want[0], (n, k, m64.skinny)
        if want[1] is not None:
            assert (m64.block_m, m64.block_n, m64.split_reduce) == (want[1], want[2], 1), (n, k)
    assert lib.dg_launch_plan(None, None) == -1


def test_gemv_plan_splits_k_within_one_round(lib):
    """M = 1 decode GEMV: the K split between a workgroup's waves doubles while each range keeps 16 steps
    of 128 bytes and the workgroups (64 / ks rows of B each) still fit one round on the 256 CUs."""
    for (n, k), rows in (((2112, 7168), 16), ((4096, 7168), 16), ((7168, 7168), 32), ((7168, 4096), 32),
                         ((3072, 7168), 16)):
        info = _lib.LaunchInfo()
        assert lib.dg_launch_plan(_plan_args(1, n, k, 0), ctypes.byref(info)) == 0, lib.dg_last_error()
        assert info.skinny == 3 and info.block_n == rows, (n, k, info.skinny, info.block_n)
        assert info.grid <= 256


def test_workspace_size_of_decode_plans(lib):
    """dg_gemm_workspace_size covers the shared-ring plans' partial tiles as their kernels number them: with M
    in two 64-row blocks the strips are padded to whole groups of eight (128x2112x7168: 33 strips -> 40, two
    row blocks, split 3, 64x64 fp32 partials), plus the 64 KiB counter area; the wide 128x64 plan has no row
    blocks (128x4096x7168: 64 strips, split 4)."""
    def size(m, n, k):
        args = _plan_args(m, n, k, 256)
        nbytes = ctypes.c_int64(0)
        assert lib.dg_gemm_workspace_size(ctypes.byref(args), ctypes.byref(nbytes)) == 0, lib.dg_last_error()
        info = _lib.LaunchInfo()
        args.library_workspace = 1
        assert lib.dg_launch_plan(args, ctypes.byref(info)) == 0, lib.dg_last_error()
        return nbytes.value, info
    ws, info = size(128, 2112, 7168)
    assert (info.block_m, info.block_n, info.split_k, info.tiles) == (64, 64, 3, 80), (info.block_m, info.block_n, info.split_k, info.tiles)
    assert ws == 64 * 1024 + 80 * 3 * 64 * 64 * 4
    ws, info = size(128, 4096, 7168)
    assert (info.block_m, info.block_n, info.split_k, info.tiles) == (128, 64, 4, 64)
    assert ws == 64 * 1024 + 64 * 4 * 128 * 64 * 4


def test_error_words_and_stream_workspace_without_device(lib):
    # no kernel has run: nothing pending; the workspace query rejects null outputs
    assert lib.dg_take_errors() == 0
    assert lib.dg_stream_workspace(None, None, None) == -1
    assert b'null argument' in lib.dg_last_error()


def test_error_message_words():
    msg = _lib.error_message(_lib.DG_ERR_SF_INVALID | _lib.DG_ERR_M_INDICES)
    assert 'Invalid float32 SF' in msg and 'm_indices is not padded' in msg


def test_host_extension_loads_and_binds(lib):
    """The C++ host path (deep_gemm_C.so) imports and takes the library's entry points; with no
    device the error words are unavailable and it still binds."""
    path = Path(_lib.__file__).resolve().parent / 'deep_gemm_C.so'
    if not path.exists():
        pytest.skip('host extension not built')
    mod = _lib.ext()
    assert mod is not None and hasattr(mod, 'gemm') and hasattr(mod, 'init')
