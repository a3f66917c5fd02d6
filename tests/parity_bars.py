"""Error bars of the GPU parity tests, decided by the reference algorithm itself.

The north-star bars are 1e-5 (fp32 inputs) and 2e-3 (fp16/bf16 inputs, fp32 accumulation) against
both the reference's online softmax (/root/reference/cuda_attn/online_softmax_ref.py:27-63,
restated as oracle.attention_online) and a float64 softmax(QK^T/sqrt(d))V. For bf16 inputs the
reference algorithm itself can miss float64 by more than 2e-3: P is rounded to bf16 (8 significant
bits) before P @ V, so a row whose weight sits on a few keys (short causal rows, peaked scores)
carries a rounding of up to 2^-8 max|V| per dominant key. `reference_bar` therefore runs the
reference algorithm on the same inputs, at each of the reference's own tile configurations, and
widens the bar to the bf16 P-rounding bound only when one of those runs misses float64 by more than
2e-3; everywhere else the bar stays 2e-3. fp16 inputs get
the same rule with fp16's rounding (peaked rows only).
"""
from __future__ import annotations

import numpy as np

import oracle

BAR = 2e-3
BAR_F32 = 1e-5


def p_dtype_of(dtype) -> str | None:
    """The P rounding of the reference algorithm for an input dtype (torch dtype or name)."""
    name = str(dtype).replace("torch.", "")
    return {"float16": "float16", "bfloat16": "bfloat16"}.get(name)


def reference_online(q: np.ndarray, k: np.ndarray, v: np.ndarray, causal: bool, dtype,
                     q_rows: tuple[int, int] | None = None) -> np.ndarray:
    """The reference's online softmax (br=64, bc=32, its defaults) with P rounded to the input dtype."""
    return oracle.attention_online(q, k, v, causal, br=64, bc=32, p_dtype=p_dtype_of(dtype), q_rows=q_rows)


# The relative rounding of one P value that the widened bar allows for. fp16: half an ulp of 1.0,
# 2^-11, the worst case. bf16: 2^-9, half the worst case (half an ulp of 1.0 is 2^-8); every bf16
# case passes at 2^-9, so the tighter figure is kept.
HALF_ULP = {"float16": 2.0 ** -11, "bfloat16": 2.0 ** -9}
# The reference's own tile configurations of this algorithm (fused_tuned's (br, bc) set,
# /root/reference/csrc/kernels/fused_tuned.cuh:207); (64, 32) are attention_online's defaults.
REFERENCE_TILES = ((64, 32), (64, 64), (128, 32), (128, 64))


def half_bar(dtype, e_ref: float, vmax: float) -> float:
    """2e-3, or the P-rounding bound max(2e-3, 1.25 * (half ulp of P's dtype) * max|V|) when the
    reference algorithm's own error e_ref on the same inputs exceeds 2e-3."""
    if e_ref <= BAR:
        return BAR
    return max(BAR, 1.25 * HALF_ULP[p_dtype_of(dtype)] * vmax)


def reference_bar(q: np.ndarray, k: np.ndarray, v: np.ndarray, causal: bool, dtype, ref64: np.ndarray,
                  q_rows: tuple[int, int] | None = None):
    """(bar, e_ref, online) for fp16 / bf16 inputs: `online` is the reference algorithm at its
    default tiles (br=64, bc=32) on rows q_rows, `e_ref` the largest float64 error of the
    reference algorithm over its own tile configurations (which rows' P round badly depends on
    the tile walk), and `bar` = half_bar(dtype, e_ref, max|V|). `ref64` holds the float64 truth of
    the same rows."""
    ref64 = np.asarray(ref64, np.float64)
    online, e_ref = None, 0.0
    for br, bc in REFERENCE_TILES:
        out = oracle.attention_online(q, k, v, causal, br=br, bc=bc, p_dtype=p_dtype_of(dtype), q_rows=q_rows)
        if online is None:
            online = out
        e_ref = max(e_ref, float(np.abs(out.astype(np.float64) - ref64).max(initial=0.0)))
        if e_ref > BAR:
            break
    return half_bar(dtype, e_ref, float(np.abs(v).max(initial=0.0))), e_ref, online
