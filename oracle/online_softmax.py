"""CPU oracle for the attention forward path: TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this module, and only as the checker or the timed CPU baseline. The product
(``cuda_attn`` and its HIP library) never imports or calls it.

It restates, in my own NumPy code, the reference's CPU model of the fused kernels:

* ``attention_naive``  - textbook float64 softmax(QK^T/sqrt(d))V
  (follows /root/reference/cuda_attn/online_softmax_ref.py:14-24).
* ``attention_online`` - the tile-by-tile online softmax in the log2 domain, float32
  (follows /root/reference/cuda_attn/online_softmax_ref.py:27-63): Q pre-scaled by
  log2(e)/sqrt(d), running max m and sum l per row, alpha = 2^(m - m_new) with the
  -inf guards, optional rounding of P before the P@V product while l is summed from the
  unrounded P (v4's rule, /root/reference/csrc/kernels/fused_tc.cuh:150-165).
  ``p_dtype`` extends the reference's ``p_fp16`` flag to bfloat16.
* ``attention_f64_rows`` - float64 truth computed in row blocks, for shapes whose full
  N x N score matrix would not fit in host memory (same math as attention_naive).
* ``attention_kernel_model`` - not the reference's algorithm: the arithmetic of this build's
  MFMA kernel (lazy rescale per 32-row wave, l summed from the rounded P), so the GPU test can
  compare against the same P roundings. Pinned by reducing to ``attention_online`` when the
  lazy threshold is 0 and P is not rounded, and by the exactness of O / l (below).

How each function is pinned (tests/test_oracle.py): attention_naive against the
independent C brute force in oracle/attn_ref64.c and closed forms (N=1 -> V, constant
K -> mean of V, one-hot V -> P, a hand-computed 2x2 case); attention_online against
attention_naive for the reference's own test matrix (tests/test_algorithm.py:12-46 of
the reference), tile-size invariance, and an exact-representability check that pins where
P is rounded; round_bf16 against torch's bfloat16 cast; attention_kernel_model bitwise against
attention_online at threshold 0 without rounding, against attention_naive at threshold 8
(O / l is exact for any reference max), by the P <= 2^threshold bound it keeps, and by
returning V[j] exactly on rows where one key j dominates (l sums the rounded P).
"""
from __future__ import annotations

import numpy as np

LOG2E = 1.4426950408889634


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned as float32.

    NumPy has no bfloat16; this keeps the top 16 bits of the float32 pattern after adding
    the round-to-nearest-even bias. inf stays inf; finite values past the bf16 range become inf.
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = np.isnan(x)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    r = ((u + np.uint32(0x7FFF) + lsb) & np.uint32(0xFFFF0000)).view(np.float32)
    if nan.any():
        r = np.where(nan, np.float32(np.nan), r)
    return r


def round_to(x: np.ndarray, dtype: str | None) -> np.ndarray:
    """Round float32 values to ``dtype`` ("float16", "bfloat16" or None) and back to float32."""
    if dtype is None or dtype == "float32":
        return x
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return round_bf16(x)
    raise ValueError(f"unknown rounding dtype {dtype!r}")


def attention_naive(q: np.ndarray, k: np.ndarray, v: np.ndarray, causal: bool = False) -> np.ndarray:
    """Textbook softmax(QK^T / sqrt(d)) V on (..., N, d) arrays, in float64.

    Follows /root/reference/cuda_attn/online_softmax_ref.py:14-24.
    """
    q64, k64, v64 = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    n, d = q64.shape[-2], q64.shape[-1]
    s = np.matmul(q64, np.swapaxes(k64, -1, -2)) / np.sqrt(d)
    if causal:
        s = np.where(np.tril(np.ones((n, n), dtype=bool)), s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.matmul(p, v64)


def attention_f64_rows(q: np.ndarray, k: np.ndarray, v: np.ndarray, causal: bool = False,
                       rows: int = 512) -> np.ndarray:
    """attention_naive computed in blocks of ``rows`` query rows (float64, bounded memory).

    The score block per call is (..., rows, N) float64 instead of (..., N, N).
    """
    q64, k64, v64 = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    n, d = q64.shape[-2], q64.shape[-1]
    out = np.empty(q64.shape, dtype=np.float64)
    kt = np.swapaxes(k64, -1, -2)
    inv = 1.0 / np.sqrt(d)
    for i0 in range(0, n, rows):
        i1 = min(n, i0 + rows)
        s = np.matmul(q64[..., i0:i1, :], kt) * inv
        if causal:
            keep = np.arange(n)[None, :] <= np.arange(i0, i1)[:, None]
            s = np.where(keep, s, -np.inf)
        s -= s.max(axis=-1, keepdims=True)
        np.exp(s, out=s)
        s /= s.sum(axis=-1, keepdims=True)
        out[..., i0:i1, :] = np.matmul(s, v64)
    return out


def attention_online(q: np.ndarray, k: np.ndarray, v: np.ndarray, causal: bool = False,
                     br: int = 64, bc: int = 32, p_fp16: bool = False,
                     p_dtype: str | None = None, q_rows: tuple[int, int] | None = None) -> np.ndarray:
    """Tile-by-tile online softmax in float32, the way the fused kernels compute it.

    Follows /root/reference/cuda_attn/online_softmax_ref.py:27-63. ``p_fp16=True`` (or
    ``p_dtype="float16"``) rounds P to float16 before P @ V while l sums the unrounded
    float32 P; ``p_dtype="bfloat16"`` does the same with bfloat16 (extension for the
    bf16 MFMA path, which the reference does not have).

    ``q_rows=(start, stop)`` computes only the query rows [start, stop) and returns them
    (shape (..., stop - start, d)); ``start`` must be a multiple of ``br``, so every computed
    row block is one of the full computation's (row blocks are independent: the result equals
    those rows of the full output bit for bit). For sampling long sequences.
    """
    if p_fp16:
        if p_dtype not in (None, "float16"):
            raise ValueError("p_fp16=True conflicts with p_dtype=%r" % (p_dtype,))
        p_dtype = "float16"
    q32, k32, v32 = (np.asarray(x, dtype=np.float32) for x in (q, k, v))
    *batch, n, d = q32.shape
    r_start, r_stop = (0, n) if q_rows is None else (int(q_rows[0]), min(int(q_rows[1]), n))
    if r_start % br != 0 or not 0 <= r_start < r_stop:
        raise ValueError(f"q_rows {q_rows!r}: start must be a multiple of br={br} below stop")
    out = np.empty((*batch, r_stop - r_start, d), dtype=np.float32)
    scale_log2 = np.float32(LOG2E / np.sqrt(d))
    kt = np.swapaxes(k32, -1, -2)

    for i0 in range(r_start, r_stop, br):                    # one workgroup's query rows
        i1 = min(i0 + br, n)
        qi = q32[..., i0:i1, :] * scale_log2                 # log2 domain
        r = i1 - i0
        rows = np.arange(i0, i1)
        m = np.full((*batch, r), -np.inf, np.float32)
        l = np.zeros((*batch, r), np.float32)
        o = np.zeros((*batch, r, d), np.float32)
        kv_end = min(n, i1) if causal else n
        for j0 in range(0, kv_end, bc):                      # stream K/V tiles
            j1 = min(j0 + bc, n)
            s = np.matmul(qi, kt[..., :, j0:j1])
            if causal:
                cols = np.arange(j0, j1)
                s = np.where(cols[None, :] > rows[:, None], np.float32(-np.inf), s)
            m_new = np.maximum(m, s.max(axis=-1))
            dead = np.isneginf(m_new)                        # every key so far masked
            with np.errstate(invalid="ignore"):
                alpha = np.where(dead, np.float32(0), np.exp2(m - m_new)).astype(np.float32)
                p = np.where(dead[..., None], np.float32(0),
                             np.exp2(s - m_new[..., None])).astype(np.float32)
            l = l * alpha + p.sum(axis=-1, dtype=np.float32)
            p_mm = round_to(p, p_dtype)
            o = o * alpha[..., None] + np.matmul(p_mm, v32[..., j0:j1, :])
            m = m_new
        res = o / l[..., None]
        out[..., i0 - r_start:min(i1, r_stop) - r_start, :] = res[..., :min(i1, r_stop) - i0, :]
    return out


def attention_kernel_model(q: np.ndarray, k: np.ndarray, v: np.ndarray, causal: bool = False,
                           p_dtype: str | None = None, bc: int = 64, group: int = 32,
                           lazy_log2: float = 8.0, stats: dict | None = None,
                           check: str = "max", two_term: bool = True, shift: float | None = None,
                           fire: float = 2.0) -> np.ndarray:
    """The fused MFMA kernel's arithmetic, in float32 (a model of this build, not the reference).

    Same log2-domain online softmax as ``attention_online``, with the two changes the kernel
    makes (both exact in real arithmetic):
      * lazy rescale: rows are taken ``group`` at a time (one wave). After each key tile of
        ``bc`` keys, if some row's max exceeds its reference max m by more than
        ``lazy_log2``, every row whose max grew takes it as its new m and O, l are multiplied
        by alpha = 2^(m_old - m_new); otherwise m is kept and P = 2^(s - m) may reach
        2^lazy_log2;
      * l sums the rounded P (the values multiplied into O).
    ``check`` selects how the lazy rescale is triggered:
      * ``"max"`` (the fp16 kernels): the row max of each tile is compared with m before the
        exponentials, as above;
      * ``"rounded"`` (the bf16 kernel): the exponentials are taken against the reference
        m_ref = m + shift (default lazy_log2 - 1), i.e. P' = P 2^-shift, rounded, and the rescale
        fires when some rounded P' of the group reaches ``fire`` (default 2); then every row whose
        max grew takes m_ref = max + shift, O and l are multiplied by 2^(m_ref_old - m_ref_new) and
        P' is recomputed. The fp16 kernels' non-causal persistent forms (and d = 128 per block) use
        the same rule with shift = 4 and fire = 2^14 (a packed fp16 max instead of the bf16
        exponent bit). A group's first tile always takes the exact max. m_ref starts at the
        finite -3e38, so masked scores give P' = 0. With ``two_term`` (the kernel's rule), a
        group whose rows see at most ``bc`` keys (a single tile) takes P' as two rounded terms,
        hi = round(P') and lo = round(P' - hi), both multiplied into O and summed into l.
    ``stats``, if given, receives the largest P used (P' scaled back by 2^(lazy_log2 - 1) for
    ``"rounded"``) and the number of rescales.
    """
    if check == "rounded":
        shift = lazy_log2 - 1.0 if shift is None else shift
        return _kernel_model_rounded(q, k, v, causal, p_dtype, bc, group, shift, fire, stats, two_term)
    if check != "max":
        raise ValueError(f"unknown check {check!r}")
    q32, k32, v32 = (np.asarray(x, dtype=np.float32) for x in (q, k, v))
    *batch, n, d = q32.shape
    out = np.empty_like(q32)
    scale_log2 = np.float32(LOG2E / np.sqrt(d))
    kt = np.swapaxes(k32, -1, -2)
    thr = np.float32(lazy_log2)
    p_max, rescales = 0.0, 0
    for i0 in range(0, n, group):
        i1 = min(i0 + group, n)
        qi = q32[..., i0:i1, :] * scale_log2
        r = i1 - i0
        rows = np.arange(i0, i1)
        m = np.full((*batch, r), -np.inf, np.float32)
        l = np.zeros((*batch, r), np.float32)
        o = np.zeros((*batch, r, d), np.float32)
        kv_end = min(n, i1) if causal else n
        for j0 in range(0, kv_end, bc):
            j1 = min(j0 + bc, n)
            s = np.matmul(qi, kt[..., :, j0:j1])
            if causal:
                cols = np.arange(j0, j1)
                s = np.where(cols[None, :] > rows[:, None], np.float32(-np.inf), s)
            m_cand = np.maximum(m, s.max(axis=-1))
            with np.errstate(invalid="ignore"):
                rescale = np.any(m_cand > m + thr, axis=-1, keepdims=True)
            upd = rescale & (m_cand > m)
            rescales += int(rescale.sum())
            with np.errstate(invalid="ignore"):
                alpha = np.where(upd, np.exp2(m - m_cand), np.float32(1)).astype(np.float32)
            m = np.where(upd, m_cand, m)
            dead = np.isneginf(m)
            with np.errstate(invalid="ignore"):
                p = np.where(dead[..., None], np.float32(0),
                             np.exp2(s - m[..., None])).astype(np.float32)
            p_mm = round_to(p, p_dtype)
            if p_mm.size:
                p_max = max(p_max, float(p_mm.max()))
            l = l * alpha + p_mm.sum(axis=-1, dtype=np.float32)
            o = o * alpha[..., None] + np.matmul(p_mm, v32[..., j0:j1, :])
        out[..., i0:i1, :] = o / l[..., None]
    if stats is not None:
        stats["p_max"] = p_max
        stats["rescales"] = rescales
    return out


def _kernel_model_rounded(q, k, v, causal, p_dtype, bc, group, shift, fire, stats, two_term=True):
    """``attention_kernel_model(check="rounded")``: the kernels' check on the rounded P' (bf16: the
    top exponent bit, P' >= 2 with shift 7; fp16: the packed max, P' >= 2^14 with shift 4)."""
    q32, k32, v32 = (np.asarray(x, dtype=np.float32) for x in (q, k, v))
    *batch, n, d = q32.shape
    out = np.empty_like(q32)
    scale_log2 = np.float32(LOG2E / np.sqrt(d))
    kt = np.swapaxes(k32, -1, -2)
    shift = np.float32(shift)
    fire_at = np.float32(fire)
    p_max, rescales = 0.0, 0
    for i0 in range(0, n, group):
        i1 = min(i0 + group, n)
        qi = q32[..., i0:i1, :] * scale_log2
        r = i1 - i0
        rows = np.arange(i0, i1)
        m_ref = np.full((*batch, r), -3.0e38, np.float32)
        l = np.zeros((*batch, r), np.float32)
        o = np.zeros((*batch, r, d), np.float32)
        kv_end = min(n, i1) if causal else n
        for t, j0 in enumerate(range(0, kv_end, bc)):
            j1 = min(j0 + bc, n)
            s = np.matmul(qi, kt[..., :, j0:j1])
            if causal:
                cols = np.arange(j0, j1)
                s = np.where(cols[None, :] > rows[:, None], np.float32(-np.inf), s)

            def exp_round(ref):
                with np.errstate(over="ignore"):
                    return round_to(np.exp2(s - ref[..., None]).astype(np.float32), p_dtype)

            p = exp_round(m_ref)
            fire = np.any(p >= fire_at, axis=(-1, -2), keepdims=False) if t else np.ones(batch, bool)
            alpha = np.ones_like(m_ref)
            if np.any(fire):
                mrow = s.max(axis=-1) + shift
                upd = fire[..., None] & (mrow > m_ref)
                with np.errstate(invalid="ignore", over="ignore"):
                    alpha = np.where(upd, np.exp2(m_ref - mrow), np.float32(1)).astype(np.float32)
                m_ref = np.where(upd, mrow, m_ref).astype(np.float32)
                rescales += int(np.sum(fire)) if t else 0
                p = exp_round(m_ref)
            if p.size:
                p_max = max(p_max, float(p.max()) * 2.0 ** float(shift))
            terms = [p]
            if two_term and kv_end <= bc:
                # rows of at most bc keys (one tile): P' as hi = round(P') plus
                # lo = round(P' - hi), both multiplied into O and summed into l (lo first)
                with np.errstate(over="ignore"):
                    x = np.exp2(s - m_ref[..., None]).astype(np.float32)
                terms = [round_to((x - p).astype(np.float32), p_dtype), p]
            l = l * alpha
            o = o * alpha[..., None]
            for pt in terms:
                l = l + pt.sum(axis=-1, dtype=np.float32)
                o = o + np.matmul(pt, v32[..., j0:j1, :])
        out[..., i0:i1, :] = o / l[..., None]
    if stats is not None:
        stats["p_max"] = p_max
        stats["rescales"] = rescales
    return out
