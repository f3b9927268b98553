"""Runtime knobs (the reference's csrc/apis/runtime.hpp:13-79 and csrc/jit/jit.hpp:18-74).

``set_num_sms`` maps to the number of CUs the tile heuristic plans for (MI355X: 256).
The M-grouped contiguous alignment defaults to 256 like the reference and may be set to
any positive multiple of 32 (128 is the common MoE choice); the grouped kernels then use a
block_m that divides it.
"""
import os
import threading

_state = threading.local()
_lock = threading.Lock()
_num_sms = 0
_mk_alignment = 256
_dry_run = False
_jit = os.environ.get('DG_JIT', '0') not in ('', '0')
_deterministic = False
_device_cus = {}

DEFAULT_MK_ALIGNMENT = 256


def _device_num_cus() -> int:
    import torch
    from . import _lib
    dev = torch.cuda.current_device()
    if dev not in _device_cus:
        n = _lib.load().dg_device_num_cus(dev)
        if n <= 0:
            _lib.check(n)
        _device_cus[dev] = n
    return _device_cus[dev]


def get_num_sms() -> int:
    return _num_sms if _num_sms else _device_num_cus()


def set_num_sms(n: int) -> None:
    global _num_sms
    if not (0 < n <= _device_num_cus()):
        raise RuntimeError(f'Assertion error: n > 0 and n <= device CU count ({n})')
    _num_sms = int(n)


def get_mk_alignment_for_contiguous_layout() -> int:
    return _mk_alignment


def set_mk_alignment_for_contiguous_layout(value: int) -> None:
    global _mk_alignment
    if value <= 0 or value % 32 != 0:
        raise RuntimeError(f'mk_alignment must be a positive multiple of 32, got {value}')
    _mk_alignment = int(value)


def get_theoretical_mk_alignment_for_contiguous_layout() -> int:
    return DEFAULT_MK_ALIGNMENT


def set_dry_run(value: bool) -> None:
    global _dry_run
    _dry_run = bool(value)


def get_dry_run() -> bool:
    return _dry_run


def set_jit(enabled: bool) -> None:
    """Launch kernels compiled at run time for each problem (hipRTC, cached under DG_JIT_CACHE_DIR)
    instead of the ahead-of-time tile menu; the initial value comes from DG_JIT (default off)."""
    global _jit
    _jit = bool(enabled)


def get_jit() -> bool:
    return _jit


def use_deterministic_algorithms(enabled: bool) -> None:
    # Every kernel here is deterministic (no split-K atomics); the flag is kept for API parity.
    global _deterministic
    _deterministic = bool(enabled)


def get_deterministic_algorithms() -> bool:
    return _deterministic


def get_npu_arch() -> int:
    return 950


def set_npu_arch(arch: int) -> None:
    if arch != 950:
        raise RuntimeError('this build targets gfx950 only')


def init(version: str = '', library_root_path: str = '') -> None:
    """Lazy init: nothing touches the device here (fork safety, tests/test_lazy_init.py)."""
    return None
