"""Attention forward kernels for AMD MI355X (gfx950), behind the reference's cuda_attn API.

    import cuda_attn
    o = cuda_attn.fused_tc(q, k, v, causal=False)   # q, k, v: (B, H, N, d) tensors on the GPU

Drop-in for the reference package (/root/reference/cuda_attn/__init__.py:40-94): same entry
points, argument defaults, KERNELS ordering and FP16_ONLY set, same argument checks and error
messages. Underneath, every entry point calls hand-written HIP kernels in libphantom_attn.so
through its C ABI (include/phantom_attn.h); there is no CPU or PyTorch fallback.

    naive        3 kernels, fp32 N x N scores in a workspace        any d, fp32/fp16
    tiled        LDS-tiled scores / P.V, one wave per softmax row     any d, fp32/fp16
    fused        fused online softmax, fp32 arithmetic (fp32 MFMA)    d=64, fp32/fp16
    fused_tuned  fp16 MFMA fused kernel at a chosen (br, bc) tile and 1 or 2 LDS stages
    fused_tc     fp16/bf16 MFMA fused kernel                          d=64 or 128

Extensions over the reference: fused_tc accepts bfloat16 and d=128; the fused entry points take
`out_dtype=torch.float32` to return fp32 output from fp16/bf16 inputs.
"""
from __future__ import annotations

import torch

from . import _checks, _native

__version__ = "0.1.0"

_DTYPE_CODE = {torch.float32: _native.DTYPE_F32, torch.float16: _native.DTYPE_F16,
               torch.bfloat16: _native.DTYPE_BF16}


_LDS_LIMIT: dict = {}
_LDS_NEED: dict = {}
# Raw handle of the current stream of a device index; torch's private accessor is ~10x cheaper
# than building a torch.cuda.Stream object per call.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        idx = t.device.index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(t.device).cuda_stream


def _lds_need(key, fn, *args) -> int:
    """LDS bytes a compiled tile needs (constant per configuration, queried once)."""
    need = _LDS_NEED.get(key)
    if need is None:
        need = _LDS_NEED[key] = fn(*args)
    return need


def _lds_limit(t: torch.Tensor) -> int:
    dev = t.device.index if t.device.index is not None else torch.cuda.current_device()
    lim = _LDS_LIMIT.get(dev)
    if lim is None:
        lim = _LDS_LIMIT[dev] = _native.device_lds_limit(dev)
    return lim


def _bhnd(q: torch.Tensor):
    b, h, n, d = q.shape
    return b * h, n, d


_FNS: dict = {}
# Current device index without torch.cuda.current_device()'s lazy-init wrapper (the launch path
# runs after a CUDA tensor exists, so the runtime is initialised).
_get_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def _call(fn_name: str, err_name: str, device: torch.device, *args) -> None:
    """Launch on `device` (switching the current device only when it differs)."""
    fn = _FNS.get(fn_name)
    if fn is None:
        fn = _FNS[fn_name] = getattr(_native.lib(), fn_name)
    if device.index is None or device.index == _get_device():
        rc = fn(*args)
    else:
        with torch.cuda.device(device):
            rc = fn(*args)
    _native.check(rc, err_name)


def _unfused(fn_name: str, err_name: str, q, k, v, causal: bool) -> torch.Tensor:
    _checks.check_inputs(q, k, v)
    _checks.check_float_half(err_name, q)
    bh, n, d = _bhnd(q)
    s = torch.empty((q.shape[0], q.shape[1], n, n), dtype=torch.float32, device=q.device)
    o = torch.empty_like(q)
    _call(fn_name, err_name, q.device, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), s.data_ptr(),
          _DTYPE_CODE[q.dtype], bh, n, d, int(bool(causal)), _stream_ptr(q))
    return o


def naive(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False) -> torch.Tensor:
    """v1: three kernels, one thread per output, N x N scores in HBM."""
    return _unfused("pa_naive_fwd", "naive_forward", q, k, v, causal)


def tiled(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False) -> torch.Tensor:
    """v2: LDS-tiled matmuls and a wave-per-row softmax, N x N scores still in HBM."""
    return _unfused("pa_tiled_fwd", "tiled_forward", q, k, v, causal)


def fused(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False, *,
          out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """v3: one fused kernel with online softmax in fp32 arithmetic. Requires d == 64."""
    _checks.check_inputs(q, k, v)
    _checks.check_head_dim("fused_forward", q, (64,))
    _checks.check_float_half("fused_forward", q)
    od = _checks.resolve_out_dtype("fused_forward", q, out_dtype)
    bh, n, d = _bhnd(q)
    o = (torch.empty_like(q) if od == q.dtype else torch.empty_like(q, dtype=od))
    _call("pa_fused_fwd", "fused_forward", q.device, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
          _DTYPE_CODE[q.dtype], _DTYPE_CODE[od], bh, n, d, int(bool(causal)), _stream_ptr(q))
    return o


def fused_tuned(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                double_buffer: bool = True, br: int = 64, bc: int = 32, *,
                out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """The fp16 MFMA fused kernel at query tile br and key tile bc.
    double_buffer=True: two LDS stages, tile t+1 loaded while tile t is computed (v3.2);
    double_buffer=False: one stage (v3.1). (br, bc) in {(64, 32), (64, 64), (128, 32), (128, 64)}.
    FP16, d == 64."""
    _checks.check_inputs(q, k, v)
    _checks.check_fp16_d64_aligned("fused_tuned", q, k, v)
    _checks.check_tuned_config(br, bc)
    od = _checks.resolve_out_dtype("fused_tuned", q, out_dtype)
    key = ("tuned", int(br), int(bc), bool(double_buffer))
    need = _lds_need(key, _native.lib().pa_fused_tuned_lds_bytes, int(br), int(bc), int(bool(double_buffer)), 64,
                     _native.DTYPE_F16)
    _checks.check_lds("fused_tuned", need, _lds_limit(q), f"BR={br} BC={bc}")
    bh, n, d = _bhnd(q)
    o = (torch.empty_like(q) if od == q.dtype else torch.empty_like(q, dtype=od))
    _call("pa_fused_tuned_fwd", "fused_tuned", q.device, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
          _native.DTYPE_F16, _DTYPE_CODE[od], bh, n, d, int(bool(causal)), int(bool(double_buffer)), int(br), int(bc),
          _stream_ptr(q))
    return o


def fused_vec(q, k, v, causal=False):
    """v3.1 with default tiles (one LDS stage)."""
    return fused_tuned(q, k, v, causal, double_buffer=False)


def fused_db(q, k, v, causal=False):
    """v3.2 with default tiles (two LDS stages)."""
    return fused_tuned(q, k, v, causal, double_buffer=True)


def fused_tc(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False, *,
             out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """v4: both matmuls on MFMA (fp16/bf16 in, fp32 accumulate), online softmax in between.
    FP16 or BF16, d in {64, 128}. The library picks the launch from the shape: persistent (as many
    workgroups as fit at once, walking the query blocks) for every causal call and for non-causal
    calls with an even number of 64-key tiles or an odd number, above one, of full ones; at d = 64 a
    key split instead where the grid is small (rows of 2-4 key tiles, or 128-query blocks that fill
    at most half the CUs), and at d = 128 where the 256-query blocks would fill at most half the
    CUs (causal: at most all of them) or, non-causal, leave the last round of one block per CU at
    most 85 % full or hold mostly padding rows (N <= 128, or past one round at least 14 % of the
    rows), 128-query workgroups (same bits); otherwise one workgroup per query block.
    cuda_attn._native.fused_tc_kernel names the launch a call takes. PA_PERSISTENT=0 in the
    environment when the library loads, or cuda_attn._native.set_persistent(False), selects one
    workgroup per query block instead of the persistent launch (same bits, except for fp16 at d = 64
    on non-causal rows: the persistent kernel starts a rescale on the packed maximum of the rounded
    probabilities, the per-block one on the row maximum; both within the fp16 bar)."""
    _checks.check_inputs(q, k, v)
    _checks.check_tc(q, k, v)
    od = _checks.resolve_out_dtype("fused_tc", q, out_dtype)
    d, code = q.shape[3], _DTYPE_CODE[q.dtype]
    need = _lds_need(("tc", d, code), _native.lib().pa_fused_tc_lds_bytes, d, code)
    _checks.check_lds("fused_tc", need, _lds_limit(q))
    bh, n, d = _bhnd(q)
    o = (torch.empty_like(q) if od == q.dtype else torch.empty_like(q, dtype=od))
    _call("pa_fused_tc_fwd", "fused_tc", q.device, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
          _DTYPE_CODE[q.dtype], _DTYPE_CODE[od], bh, n, d, int(bool(causal)), _stream_ptr(q))
    return o


def reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False) -> torch.Tensor:
    """FP32 math-backend SDPA (/root/reference/cuda_attn/__init__.py:78-84)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    with sdpa_kernel(SDPBackend.MATH):
        return torch.nn.functional.scaled_dot_product_attention(
            q.float(), k.float(), v.float(), is_causal=causal)


# Every version, in the order the project builds them.
KERNELS = {"naive": naive, "tiled": tiled, "fused": fused,
           "fused_vec": fused_vec, "fused_db": fused_db, "fused_tc": fused_tc}
# Versions that do not take float32 inputs (fused_tc also takes bfloat16).
FP16_ONLY = {"fused_vec", "fused_db", "fused_tc"}

__all__ = ["naive", "tiled", "fused", "fused_tuned", "fused_vec", "fused_db", "fused_tc",
           "reference", "KERNELS", "FP16_ONLY"]
