"""The run-time compiler (dg_jit_compile, hipRTC for gfx950) on the CPU: a GEMM plan compiles
without a GPU, lands in the DG_JIT_CACHE_DIR cache, is served from memory on the next call and from
disk in a fresh process, and a header-text change gives a different cache key."""
import ctypes
import os
import subprocess
import sys
import textwrap

import pytest

from deep_gemm import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _args(m=4096, n=7168, k=2048, gemm_type=_lib.DG_GEMM_NORMAL, dims=_lib.DG_COMPILED_N | _lib.DG_COMPILED_K):
    a = _lib.GemmArgs()
    a.kind, a.gemm_type, a.m, a.n, a.k, a.num_groups = _lib.DG_KIND_FP8_FP8, gemm_type, m, n, k, 1
    a.a, a.b, a.d, a.sfa, a.sfb = 0x100000, 0x200000, 0x300000, 0x400000, 0x500000
    a.lda, a.ldb, a.ldd = k, k, n
    a.sfa_ld, a.sfb_ld = m + (m & 1), n + (n & 1)
    a.d_dtype, a.alpha, a.alignment, a.num_cus, a.split_k = _lib.DG_DTYPE_BF16, 1.0, 256, 256, 1
    a.jit, a.compiled_dims = 1, dims
    return a


def test_jit_compile_and_cache(tmp_path, monkeypatch):
    monkeypatch.setenv('DG_JIT_CACHE_DIR', str(tmp_path / 'c1') + ':' + str(tmp_path / 'c2'))
    lib = _lib.load()
    before = _lib.jit_stats(lib)
    _lib.check(lib.dg_jit_compile(ctypes.byref(_args())), lib)
    after = _lib.jit_stats(lib)
    assert after[0] == before[0] + 1, 'one hipRTC compilation'
    files = os.listdir(tmp_path / 'c1')
    assert len(files) == 1 and files[0].endswith('.hsaco'), files
    assert os.path.getsize(tmp_path / 'c1' / files[0]) > 4096
    # same plan again: served from memory, nothing compiled
    _lib.check(lib.dg_jit_compile(ctypes.byref(_args())), lib)
    assert _lib.jit_stats(lib)[0] == after[0]
    # another compile-time K is another kernel
    _lib.check(lib.dg_jit_compile(ctypes.byref(_args(k=1024))), lib)
    assert _lib.jit_stats(lib)[0] == after[0] + 1
    assert len(os.listdir(tmp_path / 'c1')) == 2


def test_jit_disk_cache_in_fresh_process(tmp_path):
    """A second process finds the code object in the second directory of the search list."""
    code = textwrap.dedent(f'''
        import ctypes, sys
        sys.path[:0] = [{ROOT!r}, {os.path.join(ROOT, 'deepgemm-ascend_amd')!r}, {os.path.join(ROOT, 'tests')!r}]
        from deep_gemm import _lib
        from test_jit import _args
        lib = _lib.load()
        _lib.check(lib.dg_jit_compile(ctypes.byref(_args(k=512))), lib)
        print(*_lib.jit_stats(lib))
    ''')
    env = dict(os.environ, DG_JIT_CACHE_DIR=str(tmp_path / 'c1'))
    out1 = subprocess.run([sys.executable, '-c', code], env=env, capture_output=True, text=True, timeout=300)
    assert out1.returncode == 0, out1.stderr[-2000:]
    assert out1.stdout.split()[:2] == ['1', '0']
    env['DG_JIT_CACHE_DIR'] = str(tmp_path / 'empty') + ':' + str(tmp_path / 'c1')
    out2 = subprocess.run([sys.executable, '-c', code], env=env, capture_output=True, text=True, timeout=300)
    assert out2.returncode == 0, out2.stderr[-2000:]
    assert out2.stdout.split()[:2] == ['0', '1'], 'read from the disk cache, not recompiled'


def test_jit_header_change_changes_key(tmp_path, monkeypatch):
    """Editing a kernel header must never reuse a stale code object."""
    monkeypatch.setenv('DG_JIT_CACHE_DIR', str(tmp_path / 'c'))
    src = os.path.join(ROOT, 'deepgemm-ascend_amd', 'csrc')
    hdr = tmp_path / 'hdr'
    hdr.mkdir()
    for f in ('gemm_kernel.hpp', 'dg_common.hpp'):
        (hdr / f).write_text(open(os.path.join(src, f)).read())
    lib = _lib.load()
    try:
        _lib.check(lib.dg_jit_set_include_dir(str(hdr).encode()), lib)
        _lib.check(lib.dg_jit_compile(ctypes.byref(_args(k=256))), lib)
        (hdr / 'dg_common.hpp').write_text((hdr / 'dg_common.hpp').read_text() + '\n// edited\n')
        _lib.check(lib.dg_jit_set_include_dir(str(hdr).encode()), lib)
        _lib.check(lib.dg_jit_compile(ctypes.byref(_args(k=256))), lib)
        assert len(os.listdir(tmp_path / 'c')) == 2
    finally:
        _lib.check(lib.dg_jit_set_include_dir(src.encode()), lib)


def test_jit_compile_error_is_reported(tmp_path, monkeypatch):
    monkeypatch.setenv('DG_JIT_CACHE_DIR', str(tmp_path / 'c'))
    hdr = tmp_path / 'bad'
    hdr.mkdir()
    (hdr / 'gemm_kernel.hpp').write_text('#error broken header\n')
    (hdr / 'dg_common.hpp').write_text('\n')
    lib = _lib.load()
    src = os.path.join(ROOT, 'deepgemm-ascend_amd', 'csrc')
    try:
        _lib.check(lib.dg_jit_set_include_dir(str(hdr).encode()), lib)
        with pytest.raises(RuntimeError, match='hipRTC compilation failed'):
            _lib.check(lib.dg_jit_compile(ctypes.byref(_args(k=128))), lib)
    finally:
        _lib.check(lib.dg_jit_set_include_dir(src.encode()), lib)
