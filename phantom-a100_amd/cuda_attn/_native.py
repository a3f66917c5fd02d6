"""ctypes binding of libphantom_attn.so (declarations: include/phantom_attn.h).

Replaces the reference's pybind11 module cuda_attn._C and its JIT fallback
(/root/reference/cuda_attn/__init__.py:18-37, /root/reference/csrc/bindings.cpp:40-54). There is
no fallback here: if the HIP library is not built, every compute call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libphantom_attn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

# include/phantom_attn.h: enum pa_dtype / pa_status
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
OK, ERR_INVALID, ERR_UNSUPPORTED = 0, -1, -2

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64

# name -> (restype, argtypes); must list every function the header declares.
PROTOTYPES = {
    "pa_naive_fwd": (_i, [_p, _p, _p, _p, _p, _i, _i64, _i64, _i64, _i, _p]),
    "pa_tiled_fwd": (_i, [_p, _p, _p, _p, _p, _i, _i64, _i64, _i64, _i, _p]),
    "pa_tiled_fwd_noalloc": (_i, [_p, _p, _p, _p, _i, _i64, _i64, _i64, _i, _p]),
    "pa_fused_fwd": (_i, [_p, _p, _p, _p, _i, _i, _i64, _i64, _i64, _i, _p]),
    "pa_fused_tuned_fwd": (_i, [_p, _p, _p, _p, _i, _i, _i64, _i64, _i64, _i, _i, _i, _i, _p]),
    "pa_fused_tc_fwd": (_i, [_p, _p, _p, _p, _i, _i, _i64, _i64, _i64, _i, _p]),
    "pa_fused_tc_kernel": (ctypes.c_char_p, [_i, _i, _i64, _i64, _i64, _i]),
    "pa_set_persistent": (_i, [_i]),
    "pa_fused_tuned_lds_bytes": (_i64, [_i, _i, _i, _i64, _i]),
    "pa_fused_tc_lds_bytes": (_i64, [_i64, _i]),
    "pa_device_lds_limit": (_i, [_i, ctypes.POINTER(_i64)]),
    "pa_last_error": (ctypes.c_char_p, []),
    "pa_version": (ctypes.c_char_p, []),
}

_lib = None
_lock = threading.Lock()


class NativeLibraryMissing(RuntimeError):
    """libphantom_attn.so has not been built (run `python __graft_entry__.py` or build_native.py)."""


def lib() -> ctypes.CDLL:
    """Load libphantom_attn.so once and attach the prototypes."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise NativeLibraryMissing(
                        f"cuda_attn: {LIB_NAME} is not built at {LIB_PATH}; build it with "
                        "`python phantom-a100_amd/build_native.py`")
                handle = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in PROTOTYPES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().pa_last_error()
    return msg.decode() if msg else ""


def version() -> str:
    return lib().pa_version().decode()


def check(rc: int, name: str) -> None:
    """Turn a nonzero status into RuntimeError (the reference's ATTN_CHECK, csrc/common.cuh:21-25)."""
    if rc != OK:
        msg = last_error() or f"{name}: error {rc}"
        raise RuntimeError(msg)


def device_lds_limit(device: int) -> int:
    out = ctypes.c_int64(0)
    check(lib().pa_device_lds_limit(int(device), ctypes.byref(out)), "pa_device_lds_limit")
    return int(out.value)


def fused_tc_kernel(dtype: int, out_dtype: int, bh: int, n: int, d: int, causal: bool = False) -> str:
    """The kernel instantiation and launch shape fused_tc would use (pa_fused_tc_kernel)."""
    return lib().pa_fused_tc_kernel(int(dtype), int(out_dtype), int(bh), int(n), int(d), int(bool(causal))).decode()


def set_persistent(enable: bool) -> bool:
    """Switch fused_tc's persistent launch on or off (every shape that would take it: causal calls,
    and non-causal ones with an even number of 64-key tiles or an odd number, above one, of full
    ones, at d = 64 and 128); returns the previous setting. fused_tc_kernel names the launch."""
    return bool(lib().pa_set_persistent(int(bool(enable))))
