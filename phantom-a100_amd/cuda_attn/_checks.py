"""Argument checks of the attention entry points, run in Python before the native call.

Same checks, order and message substrings as the reference's C++ glue, so callers (and the
reference's tests, which match on "contiguous", "dtype", "head dimension", "float16",
"not compiled" and "shared memory") see the same errors:
  check_inputs        /root/reference/csrc/bindings.cpp:12-22
  float/half dispatch /root/reference/csrc/common.cuh:14-19
  fp16 / d=64 / align /root/reference/csrc/common.cuh:27-33
  tile set and LDS    /root/reference/csrc/attn_fused_tuned.cu:8-14, attn_fused_tc.cu:11-13
Deliberate extensions: fused_tc also takes bfloat16 and d = 128; every fused entry takes an
optional fp32 output dtype.
"""
from __future__ import annotations

import torch

TUNED_CONFIGS = ((64, 32), (64, 64), (128, 32), (128, 64))  # /root/reference/csrc/kernels/fused_tuned.cuh:207
TC_HEAD_DIMS = (64, 128)
TC_DTYPES = (torch.float16, torch.bfloat16)


def _fail(msg: str):
    raise RuntimeError(msg)


def check_inputs(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, require_cuda: bool = True) -> None:
    """Checks shared by every entry point (csrc/bindings.cpp:12-22)."""
    for t in (q, k, v):
        if require_cuda and not t.is_cuda:
            _fail("inputs must be CUDA tensors")
        if not t.is_contiguous():
            _fail("inputs must be contiguous")
        if t.dim() != 4:
            _fail("inputs must be shaped (B, H, N, d)")
        if t.dtype != q.dtype:
            _fail("q, k, v must share a dtype")
    if q.shape != k.shape or q.shape != v.shape:
        _fail("q, k, v must have the same shape")
    if q.device != k.device or q.device != v.device:
        _fail("q, k, v must be on the same device")
    if q.numel() == 0:
        _fail("inputs must be non-empty")


def check_float_half(name: str, q: torch.Tensor) -> None:
    if q.dtype not in (torch.float32, torch.float16):
        _fail(f"{name}: only float32 and float16 are supported")


def check_head_dim(name: str, q: torch.Tensor, allowed=(64,)) -> None:
    d = q.shape[3]
    if d not in allowed:
        if len(allowed) == 1:
            _fail(f"{name}: only head dimension {allowed[0]} is compiled (got {d})")
        dims = " and ".join(str(a) for a in allowed)
        _fail(f"{name}: only head dimensions {dims} are compiled (got {d})")


def check_aligned(name: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.data_ptr() % 16 != 0:
            _fail(f"{name}: inputs must be 16-byte aligned")


def check_fp16_d64_aligned(name: str, q, k, v) -> None:
    """The reference's fp16-only / d=64 / 16-byte check (csrc/common.cuh:27-33)."""
    if q.dtype != torch.float16:
        _fail(f"{name}: float16 only")
    check_head_dim(name, q, (64,))
    check_aligned(name, q, k, v)


def check_tc(q, k, v) -> None:
    """fused_tc: fp16 or bf16, d in {64, 128}, 16-byte aligned (extends csrc/common.cuh:27-33)."""
    if q.dtype not in TC_DTYPES:
        _fail("fused_tc: float16 or bfloat16 only")
    check_head_dim("fused_tc", q, TC_HEAD_DIMS)
    check_aligned("fused_tc", q, k, v)


def check_tuned_config(br: int, bc: int) -> None:
    if (int(br), int(bc)) not in TUNED_CONFIGS:
        _fail(f"fused_tuned: (br, bc) = ({br}, {bc}) not compiled; available: (64,32) (64,64) (128,32) (128,64)")


def resolve_out_dtype(name: str, q: torch.Tensor, out_dtype) -> torch.dtype:
    """Output dtype: the input dtype by default (as in the reference) or float32 on request."""
    if out_dtype is None or out_dtype == q.dtype:
        return q.dtype
    if out_dtype == torch.float32:
        return torch.float32
    _fail(f"{name}: out_dtype must be the input dtype or torch.float32 (got {out_dtype})")


def check_lds(name: str, need: int, limit: int, detail: str = "") -> None:
    """Per-workgroup LDS against the device limit (reference wording: 'shared memory')."""
    if need < 0:
        _fail(f"{name}: configuration not compiled")
    if need > limit:
        if detail:
            _fail(f"{name}: {detail} needs {need} bytes of shared memory; this GPU allows {limit}")
        _fail(f"{name}: needs {need} bytes of shared memory, GPU allows {limit}")
