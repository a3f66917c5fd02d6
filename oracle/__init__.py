"""CPU oracle for the attention forward path: TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker or as the timed CPU baseline. The shipped library
(phantom-a100_amd/cuda_attn + its HIP .so) never imports it and has no CPU fallback.

Contents:
  online_softmax.py  NumPy restatement of /root/reference/cuda_attn/online_softmax_ref.py,
                     plus a model of the MFMA kernel's own arithmetic (attention_kernel_model)
  attn_ref64.c       float64 brute force restating /root/reference/sim/harness.cu:40-64
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from .online_softmax import (LOG2E, attention_f64_rows, attention_kernel_model, attention_naive,  # noqa: F401
                             attention_online, round_bf16, round_to)

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build_c_oracle() -> str:
    """Compile oracle/attn_ref64.c into oracle/liboracle_ref64.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle_ref64.so"], check=True)
    return os.path.join(_HERE, "liboracle_ref64.so")


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle_ref64.so")
        if not os.path.exists(path):
            path = build_c_oracle()
        lib = ctypes.CDLL(path)
        lib.attn_ref64.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3 + [ctypes.c_int]
        lib.attn_ref64.restype = ctypes.c_int
        _LIB = lib
    return _LIB


def attention_ref64(q: np.ndarray, k: np.ndarray, v: np.ndarray, causal: bool = False) -> np.ndarray:
    """float64 attention from the C brute force; q, k, v are (..., N, d) arrays."""
    q32, k32, v32 = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    if not (q32.shape == k32.shape == v32.shape) or q32.ndim < 2:
        raise ValueError("q, k, v must share a (..., N, d) shape")
    n, d = q32.shape[-2], q32.shape[-1]
    bh = int(np.prod(q32.shape[:-2], dtype=np.int64))
    out = np.empty(q32.shape, dtype=np.float64)
    rc = _lib().attn_ref64(q32.ctypes.data, k32.ctypes.data, v32.ctypes.data, out.ctypes.data,
                           bh, n, d, int(bool(causal)))
    if rc != 0:
        raise RuntimeError("attn_ref64 failed (%d)" % rc)
    return out
