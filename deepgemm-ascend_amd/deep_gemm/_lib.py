"""ctypes binding of libdeep_gemm_amd.so (the C ABI declared in include/deep_gemm_amd.h).

The library is loaded lazily on the first kernel call, so ``import deep_gemm`` touches
neither the HIP runtime nor the GPU (the reference keeps import fork-safe the same way,
csrc/apis/runtime.hpp:41-44).  There is no CPU fallback: a missing library raises.
"""
import ctypes
import os
import threading
from pathlib import Path

_LIB_NAME = 'libdeep_gemm_amd.so'
_lock = threading.Lock()
_lib = None

DG_KIND_FP8_FP8, DG_KIND_FP8_FP4, DG_KIND_FP4_FP4, DG_KIND_BF16 = 0, 1, 2, 3
DG_GEMM_NORMAL, DG_GEMM_BATCHED, DG_GEMM_MGROUPED_PSUM, DG_GEMM_MGROUPED_IDX, DG_GEMM_MASKED, DG_GEMM_KGROUPED = 0, 1, 2, 3, 4, 5
DG_DTYPE_BF16, DG_DTYPE_F32, DG_DTYPE_FP8_E4M3 = 0, 1, 2
DG_EPI_DEFAULT, DG_EPI_BF16_SR = 0, 1
DG_SF_F32, DG_SF_I16 = 0, 1
DG_COMPILED_M, DG_COMPILED_N, DG_COMPILED_K = 1, 2, 4

# Every symbol include/deep_gemm_amd.h declares.
EXPORTED_SYMBOLS = ('dg_gemm', 'dg_transform_sf', 'dg_transform_k_grouped_sf', 'dg_transpose_to_k_major', 'dg_fp4_to_k_major', 'dg_device_num_cus', 'dg_select_config',
                    'dg_gemm_workspace_size', 'dg_last_error', 'dg_version', 'dg_jit_compile', 'dg_jit_set_include_dir',
                    'dg_jit_stats', 'dg_launch_plan', 'dg_gemm_noalloc', 'dg_take_errors', 'dg_error_words',
                    'dg_stream_workspace')

# Sticky error bits kernels report through host-mapped words (DG_ERR_* in the header)
DG_ERR_SF_INVALID, DG_ERR_M_INDICES = 1, 2
DG_ENOKERNEL = -3   # dg_gemm: no compiled kernel for the requested configuration


class GemmArgs(ctypes.Structure):
    """Mirror of ``dg_gemm_args`` (include/deep_gemm_amd.h)."""
    _fields_ = [
        ('kind', ctypes.c_int32), ('gemm_type', ctypes.c_int32),
        ('a', ctypes.c_void_p), ('b', ctypes.c_void_p), ('d', ctypes.c_void_p),
        ('sfa', ctypes.c_void_p), ('sfb', ctypes.c_void_p),
        ('bias', ctypes.c_void_p), ('grouped_layout', ctypes.c_void_p),
        ('m', ctypes.c_int32), ('n', ctypes.c_int32), ('k', ctypes.c_int32), ('num_groups', ctypes.c_int32),
        ('lda', ctypes.c_int64), ('ldb', ctypes.c_int64), ('ldd', ctypes.c_int64),
        ('batch_stride_a', ctypes.c_int64), ('batch_stride_b', ctypes.c_int64), ('batch_stride_d', ctypes.c_int64),
        ('sfa_ld', ctypes.c_int64), ('sfb_ld', ctypes.c_int64),
        ('sfa_batch_stride', ctypes.c_int64), ('sfb_batch_stride', ctypes.c_int64),
        ('d_dtype', ctypes.c_int32), ('accumulate', ctypes.c_int32), ('alpha', ctypes.c_float),
        ('alignment', ctypes.c_int32), ('block_m', ctypes.c_int32), ('block_n', ctypes.c_int32),
        ('num_cus', ctypes.c_int32), ('split_k', ctypes.c_int32),
        ('workspace', ctypes.c_void_p), ('workspace_bytes', ctypes.c_int64),
        ('epilogue', ctypes.c_int32), ('sfd', ctypes.c_void_p), ('sfd_ld', ctypes.c_int64),
        ('jit', ctypes.c_int32), ('compiled_dims', ctypes.c_int32), ('library_workspace', ctypes.c_int32),
        ('a_mn_major', ctypes.c_int32), ('b_mn_major', ctypes.c_int32),
    ]


class LaunchInfo(ctypes.Structure):
    """Mirror of ``dg_launch_info`` (include/deep_gemm_amd.h)."""
    _fields_ = [
        ('block_m', ctypes.c_int32), ('block_n', ctypes.c_int32), ('grid', ctypes.c_int64),
        ('threads', ctypes.c_int32), ('tiles', ctypes.c_int64), ('split_k', ctypes.c_int32),
        ('persistent', ctypes.c_int32), ('skinny', ctypes.c_int32), ('plan_workgroups', ctypes.c_int64),
        ('split_reduce', ctypes.c_int32),
    ]


def library_path() -> Path:
    override = os.environ.get('DG_LIBRARY_PATH')
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / _LIB_NAME


def load(path=None) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else library_path()
        if not p.exists():
            raise RuntimeError(f'deep_gemm HIP library not found at {p}; build it with '
                               f'`python deepgemm-ascend_amd/build.py` (there is no CPU fallback)')
        lib = ctypes.CDLL(str(p))
        lib.dg_gemm.argtypes = [ctypes.POINTER(GemmArgs), ctypes.c_void_p]
        lib.dg_gemm.restype = ctypes.c_int
        lib.dg_transform_sf.argtypes = [
            ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        lib.dg_transform_sf.restype = ctypes.c_int
        lib.dg_transform_k_grouped_sf.argtypes = [
            ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.dg_transform_k_grouped_sf.restype = ctypes.c_int
        lib.dg_transpose_to_k_major.argtypes = [
            ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
            ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
        lib.dg_transpose_to_k_major.restype = ctypes.c_int
        lib.dg_fp4_to_k_major.argtypes = [
            ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
        lib.dg_fp4_to_k_major.restype = ctypes.c_int
        lib.dg_device_num_cus.argtypes = [ctypes.c_int32]
        lib.dg_device_num_cus.restype = ctypes.c_int
        lib.dg_select_config.argtypes = [ctypes.POINTER(GemmArgs), ctypes.POINTER(ctypes.c_int32),
                                         ctypes.POINTER(ctypes.c_int32)]
        lib.dg_select_config.restype = ctypes.c_int
        lib.dg_gemm_noalloc.argtypes = [ctypes.POINTER(GemmArgs), ctypes.c_void_p]
        lib.dg_gemm_noalloc.restype = ctypes.c_int
        lib.dg_launch_plan.argtypes = [ctypes.POINTER(GemmArgs), ctypes.POINTER(LaunchInfo)]
        lib.dg_launch_plan.restype = ctypes.c_int
        lib.dg_gemm_workspace_size.argtypes = [ctypes.POINTER(GemmArgs), ctypes.POINTER(ctypes.c_int64)]
        lib.dg_gemm_workspace_size.restype = ctypes.c_int
        lib.dg_jit_compile.argtypes = [ctypes.POINTER(GemmArgs)]
        lib.dg_jit_compile.restype = ctypes.c_int
        lib.dg_jit_set_include_dir.argtypes = [ctypes.c_char_p]
        lib.dg_jit_set_include_dir.restype = ctypes.c_int
        lib.dg_jit_stats.argtypes = [ctypes.POINTER(ctypes.c_int64)] * 3
        lib.dg_jit_stats.restype = ctypes.c_int
        # kernel headers the run-time compiler reads: csrc/ beside this package
        lib.dg_jit_set_include_dir(str(Path(__file__).resolve().parent.parent / 'csrc').encode())
        lib.dg_stream_workspace.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64)]
        lib.dg_stream_workspace.restype = ctypes.c_int
        lib.dg_take_errors.restype = ctypes.c_uint32
        lib.dg_take_errors.argtypes = []
        lib.dg_error_words.restype = ctypes.c_void_p
        lib.dg_error_words.argtypes = []
        lib.dg_last_error.restype = ctypes.c_char_p
        lib.dg_version.restype = ctypes.c_char_p
        if path is None:
            _lib = lib
        return lib


def error_message(bits: int, where: str = 'an earlier deep_gemm call') -> str:
    """Text of the sticky error bits (the C++ host path words it the same way, csrc/torch_ext.cpp)."""
    parts = []
    if bits & DG_ERR_SF_INVALID:
        parts.append('Invalid float32 SF: only the 8-bit exponent may be set (sign and mantissa must be 0)')
    if bits & DG_ERR_M_INDICES:
        parts.append('m_indices is not padded to the M-grouped alignment (every alignment-row block must hold one '
                     'group id < num_groups followed only by -1 padding)')
    return '; '.join(parts) + f' [reported by a kernel of {where}]'


def raise_pending() -> None:
    """Raise the errors kernels of earlier calls reported (no synchronisation: what has not
    completed yet is reported by a later call)."""
    if _lib is None:
        return
    bits = _lib.dg_take_errors()
    if bits:
        raise RuntimeError(error_message(bits))


def check_errors(synchronize: bool = True) -> None:
    """Raise the errors that kernels of deep_gemm calls have reported (invalid float32 scale
    factors, unpadded m_indices), at a point the caller chooses.  With `synchronize` the current
    device is synchronised first, so every call issued before this one is covered and the error
    is raised for it, not by a later call; the words are cleared either way."""
    lib = load()
    if synchronize:
        import torch
        if torch.cuda.is_available():
            torch.cuda.synchronize()
    bits = lib.dg_take_errors()
    if bits:
        raise RuntimeError(error_message(bits, 'a deep_gemm call issued before check_errors()'))


_EXT_NAME = 'deep_gemm_C'
_ext = None
_ext_tried = False


def ext():
    """The C++ host-path extension (deep_gemm_C.so beside this file), bound to the loaded
    library's entry points; None when it has not been built (the Python path then serves every
    call)."""
    global _ext, _ext_tried
    if _ext_tried:
        return _ext
    lib = load()
    with _lock:
        if _ext_tried:
            return _ext
        path = Path(__file__).resolve().parent / f'{_EXT_NAME}.so'
        mod = None
        if path.exists() and not os.environ.get('DG_DISABLE_EXT'):
            import importlib.util
            import torch  # noqa: F401  (the extension links torch's libraries)
            spec = importlib.util.spec_from_file_location(_EXT_NAME, str(path))
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            addr = lambda f: ctypes.cast(f, ctypes.c_void_p).value
            mod.init(addr(lib.dg_gemm), addr(lib.dg_transform_sf), addr(lib.dg_take_errors), addr(lib.dg_last_error),
                     lib.dg_error_words() or 0)
        _ext = mod
        _ext_tried = True
        return _ext


def jit_stats(lib=None):
    """(hipRTC compilations, disk-cache reads, launches of an already loaded kernel) since load."""
    lib = lib or load()
    vals = [ctypes.c_int64() for _ in range(3)]
    check(lib.dg_jit_stats(*[ctypes.byref(v) for v in vals]), lib)
    return tuple(v.value for v in vals)


def check(rc: int, lib=None) -> None:
    if rc != 0:
        lib = lib or load()
        msg = lib.dg_last_error().decode(errors='replace')
        raise RuntimeError(msg or f'deep_gemm error {rc}')
