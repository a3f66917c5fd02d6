"""ctypes binding of libphantom_attn_tiles.so (include/phantom_attn_tiles.h): the tile and
occupancy alternatives of the fused MFMA kernel, for the tile choice only. cuda_attn never loads
this library; the shipped tiles are measured through cuda_attn.fused_tc itself.

Replaces, for the tile choice, the reference's run-time tile selection through
attn::launch_fused_tuned_cfg (/root/reference/csrc/kernels/fused_tuned.cuh:192-228).
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

from cuda_attn import _native

LIB_PATH = os.path.join(os.path.dirname(_native.LIB_PATH), "libphantom_attn_tiles.so")
DTYPE_CODE = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16}
CODE_DTYPE = {v: k for k, v in DTYPE_CODE.items()}

_p, _i, _i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
_ip = ctypes.POINTER(ctypes.c_int)
PROTOTYPES = {
    "pa_tiles_count": (_i, []),
    "pa_tiles_label": (ctypes.c_char_p, [_i]),
    "pa_tiles_describe": (_i, [_i, _ip, _ip, _ip, _ip, _ip, _ip, _ip]),
    "pa_tiles_fwd": (_i, [_i, _p, _p, _p, _p, _i, _i64, _i64, _i64, _i, _p]),
    "pa_tiles_kernel": (ctypes.c_char_p, [_i, _i64, _i64]),
    "pa_tiles_last_error": (ctypes.c_char_p, []),
}

_lib = None
_lock = threading.Lock()


def available() -> bool:
    return os.path.exists(LIB_PATH)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not available():
                    raise _native.NativeLibraryMissing(
                        f"libphantom_attn_tiles.so is not built at {LIB_PATH}; build it with "
                        "`python phantom-a100_amd/build_native.py`")
                handle = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in PROTOTYPES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def candidates() -> list[dict]:
    """Every compiled alternative: index, label, dtype, d, br, bc, stages, persistent, wgs_per_cu
    (the most workgroups per CU of a persistent launch, 0 for as many as fit)."""
    out = []
    h = lib()
    for i in range(h.pa_tiles_count()):
        vals = [ctypes.c_int(0) for _ in range(7)]
        rc = h.pa_tiles_describe(i, *(ctypes.byref(x) for x in vals))
        if rc != _native.OK:
            raise RuntimeError(h.pa_tiles_last_error().decode())
        dt, d, br, bc, st, pers, cap = (x.value for x in vals)
        out.append({"index": i, "label": h.pa_tiles_label(i).decode(), "dtype": CODE_DTYPE.get(dt), "d": d,
                    "br": br, "bc": bc, "stages": st, "persistent": bool(pers), "wgs_per_cu": cap})
    return out


def forward(index: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False) -> torch.Tensor:
    """Candidate `index` on (B, H, N, d) CUDA tensors; the output has the input dtype."""
    b, h, n, d = q.shape
    o = torch.empty_like(q)
    rc = lib().pa_tiles_fwd(int(index), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), DTYPE_CODE[q.dtype],
                            b * h, n, d, int(bool(causal)), torch.cuda.current_stream(q.device).cuda_stream)
    if rc != _native.OK:
        raise RuntimeError(lib().pa_tiles_last_error().decode() or f"pa_tiles_fwd: error {rc}")
    return o


def kernel(index: int, bh: int, n: int) -> str:
    return lib().pa_tiles_kernel(int(index), int(bh), int(n)).decode()
