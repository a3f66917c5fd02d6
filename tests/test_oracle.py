"""CPU checks that pin the oracle before it is trusted as the parity reference.

1. The reference's own algorithm tests (/root/reference/tests/test_algorithm.py:12-46), run on
   oracle.attention_online / attention_naive.
2. Golden fixtures (tests/golden/*.npz): seeded inputs + float64 outputs of the C brute force.
3. attention_naive against the independent C brute force (oracle/attn_ref64.c) and scipy's softmax.
4. Closed forms and invariants: N=1 gives V, constant keys give the mean of V, a hand-derived
   2x2 case, causal row 0 gives V[0], key/value permutation, per-row score shifts, linearity in V.
5. Where P is rounded (p_fp16 / p_dtype): P rounded before P@V, l summed from unrounded P.
6. round_bf16 against torch's bfloat16 cast.
"""
import glob
import os

import numpy as np
import pytest
import scipy.special
import torch

import oracle
from oracle import attention_f64_rows, attention_naive, attention_online, attention_ref64, round_bf16

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def load_golden(path):
    z = np.load(path, allow_pickle=False)
    dt = str(z["dtype"])

    def f32(a):
        if dt == "bfloat16":
            return (a.astype(np.uint32) << 16).view(np.float32)
        return a.astype(np.float32)

    return f32(z["q"]), f32(z["k"]), f32(z["v"]), z["o"], bool(z["causal"]), dt, z


# ---------------------------------------------------------------- 1. reference's algorithm tests
@pytest.mark.parametrize("n", [1, 31, 32, 63, 64, 65, 100, 257])
@pytest.mark.parametrize("causal", [False, True])
def test_online_matches_naive(n, causal):
    rng = np.random.default_rng(n)
    q, k, v = (rng.standard_normal((2, 3, n, 64)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(attention_online(q, k, v, causal), attention_naive(q, k, v, causal),
                               atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("scale", [10.0, 100.0])
def test_online_is_stable_for_large_scores(scale):
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((1, 1, 200, 64)).astype(np.float32) for _ in range(3))
    out = attention_online(q * scale, k * scale, v)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, attention_naive(q * scale, k * scale, v), atol=1e-4, rtol=1e-3)


@pytest.mark.parametrize("rows", [(0, 64), (64, 300), (128, 200), (256, 300)])
@pytest.mark.parametrize("causal", [False, True])
def test_online_row_sample_equals_full_rows(rows, causal):
    """q_rows computes whole row blocks of the full computation, so its rows are bit-identical."""
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((2, 300, 64)).astype(np.float32) for _ in range(3))
    full = attention_online(q, k, v, causal, p_dtype="bfloat16")
    part = attention_online(q, k, v, causal, p_dtype="bfloat16", q_rows=rows)
    assert np.array_equal(part, full[:, rows[0]:rows[1]])


def test_online_row_sample_rejects_unaligned_start():
    q = np.zeros((1, 128, 64), np.float32)
    with pytest.raises(ValueError, match="multiple of br"):
        attention_online(q, q, q, q_rows=(10, 100))


@pytest.mark.parametrize("br,bc", [(16, 16), (64, 32), (128, 64)])
def test_tile_size_does_not_change_result(br, bc):
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal((1, 2, 300, 64)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(attention_online(q, k, v, True, br, bc), attention_naive(q, k, v, True),
                               atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("n", [1, 64, 65, 1000, 4096])
@pytest.mark.parametrize("causal", [False, True])
def test_fp16_p_stays_within_test_tolerance(n, causal):
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((1, 2, n, 64)).astype(np.float16).astype(np.float32) for _ in range(3))
    out = attention_online(q, k, v, causal, br=64, bc=64, p_fp16=True)
    out = out.astype(np.float16).astype(np.float32)
    assert np.abs(out - attention_naive(q, k, v, causal)).max() <= 2e-3


@pytest.mark.parametrize("n", [1, 65, 1000])
def test_bf16_p_stays_within_test_tolerance(n):
    """bf16 analogue (extension): P rounded to bf16, fp32 output."""
    rng = np.random.default_rng(8)
    q, k, v = (round_bf16(rng.standard_normal((1, 2, n, 128)).astype(np.float32)) for _ in range(3))
    out = attention_online(q, k, v, False, br=64, bc=64, p_dtype="bfloat16")
    assert np.abs(out - attention_naive(q, k, v, False)).max() <= 2e-3


# ---------------------------------------------------------------- 2. golden fixtures
@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_golden_inputs_regenerate_bit_exactly(path):
    """The seeded generator (cuda_attn.workloads.make_qkv) reproduces the stored inputs."""
    from cuda_attn.workloads import make_qkv
    q, k, v, o, causal, dt, z = load_golden(path)
    b, h, n, d = q.shape
    tq, tk, tv = make_qkv(b, h, n, d, getattr(torch, dt), seed=int(z["seed"]), qk_scale=float(z["qk_scale"]))
    for ref, t in ((q, tq), (k, tk), (v, tv)):
        assert np.array_equal(ref, t.float().numpy())


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_oracle_matches_golden(path):
    q, k, v, o, causal, dt, z = load_golden(path)
    np.testing.assert_allclose(attention_naive(q, k, v, causal), o, atol=2e-7, rtol=1e-6)
    np.testing.assert_allclose(attention_ref64(q, k, v, causal), o, atol=2e-7, rtol=1e-6)
    np.testing.assert_allclose(attention_f64_rows(q, k, v, causal, rows=37), o, atol=2e-7, rtol=1e-6)
    # fp32 online model within the fp32 gate (1e-5 for unit-scale scores; with Q, K x3 the
    # log2-domain scores reach ~60 and fp32 rounding of them alone is ~1e-5 of O, so use the
    # reference's large-score tolerance 1e-4, /root/reference/tests/test_algorithm.py:21-27);
    # with P rounded, within the fp16/bf16 gate.
    fp32_tol = 1e-5 if float(z["qk_scale"]) == 1.0 else 1e-4
    assert np.abs(attention_online(q, k, v, causal) - o).max() <= fp32_tol
    p_dtype = {"float16": "float16", "bfloat16": "bfloat16"}.get(dt)
    if p_dtype:
        assert np.abs(attention_online(q, k, v, causal, 64, 64, p_dtype=p_dtype) - o).max() <= p_round_tol(dt, causal, v)


def p_round_tol(dt, causal, v):
    """Bound on the error that rounding P to `dt` adds. fp16 (11-bit significand) stays within
    the 2e-3 gate. bf16 (8-bit) rounding errors average out over long non-causal rows (the bf16
    BASELINE config) but not over the first rows of a causal mask, where one rounded weight can
    carry half a bf16 ulp (2^-9) of max|V|."""
    if dt == "bfloat16" and causal:
        return max(2e-3, 2.0 ** -9 * float(np.abs(v).max()) * 1.25)
    return 2e-3


# ---------------------------------------------------------------- 3. independent implementations
@pytest.mark.parametrize("n,d,causal", [(1, 64, False), (7, 16, True), (130, 64, True), (97, 128, False)])
def test_naive_matches_c_brute_force(n, d, causal):
    rng = np.random.default_rng(100 + n)
    q, k, v = (rng.standard_normal((2, 2, n, d)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(attention_naive(q, k, v, causal), attention_ref64(q, k, v, causal),
                               atol=1e-12, rtol=1e-10)


def test_naive_matches_scipy_softmax():
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((1, 1, 50, 32)) for _ in range(3))
    p = scipy.special.softmax(q[0, 0] @ k[0, 0].T / np.sqrt(32), axis=-1)
    np.testing.assert_allclose(attention_naive(q, k, v)[0, 0], p @ v[0, 0], atol=1e-13)


# ---------------------------------------------------------------- 4. closed forms and invariants
@pytest.mark.parametrize("fn", [attention_naive, attention_online, attention_ref64])
def test_single_key_returns_v(fn):
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((2, 3, 1, 64)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(fn(q, k, v), v, atol=1e-6)


@pytest.mark.parametrize("fn", [attention_naive, attention_online, attention_ref64])
def test_constant_keys_average_v(fn):
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 2, 77, 64)).astype(np.float32)
    k = np.broadcast_to(rng.standard_normal((1, 2, 1, 64)).astype(np.float32), q.shape).copy()
    v = rng.standard_normal((1, 2, 77, 64)).astype(np.float32)
    np.testing.assert_allclose(fn(q, k, v), np.broadcast_to(v.mean(axis=-2, keepdims=True), v.shape), atol=2e-6)


@pytest.mark.parametrize("fn", [attention_naive, attention_online, attention_ref64])
def test_hand_derived_two_by_two(fn):
    # d = 2, scores = I / sqrt(2): row 0 weights (p, 1-p) with p = 1 / (1 + e^{-1/sqrt 2}) = 0.669761549...
    q = np.array([[[[1.0, 0.0], [0.0, 1.0]]]], np.float32)
    v = np.array([[[[1.0, 2.0], [3.0, 4.0]]]], np.float32)
    want = np.array([[1.660476902, 2.660476902], [2.339523098, 3.339523098]])
    np.testing.assert_allclose(fn(q, q, v)[0, 0], want, atol=1e-6)


@pytest.mark.parametrize("fn", [attention_naive, attention_online, attention_ref64])
def test_causal_first_row_is_v0(fn):
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal((1, 2, 40, 64)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(fn(q, k, v, True)[..., 0, :], v[..., 0, :], atol=1e-6)


def test_key_value_permutation_invariance():
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((1, 1, 90, 64)).astype(np.float32) for _ in range(3))
    perm = rng.permutation(90)
    np.testing.assert_allclose(attention_online(q, k[..., perm, :], v[..., perm, :]), attention_online(q, k, v),
                               atol=2e-6)


def test_row_shift_invariance():
    """k -> k + u shifts every score of row i by q_i.u; softmax is unchanged."""
    rng = np.random.default_rng(10)
    q, k, v = (rng.standard_normal((1, 1, 64, 16)).astype(np.float64) for _ in range(3))
    u = rng.standard_normal(16)
    np.testing.assert_allclose(attention_naive(q, k + u, v), attention_naive(q, k, v), atol=1e-12)


def test_linearity_in_v():
    rng = np.random.default_rng(11)
    q, k, v1, v2 = (rng.standard_normal((1, 1, 70, 32)).astype(np.float32) for _ in range(4))
    lhs = attention_online(q, k, 2 * v1 - 3 * v2)
    rhs = 2 * attention_online(q, k, v1) - 3 * attention_online(q, k, v2)
    np.testing.assert_allclose(lhs, rhs, atol=1e-5)


# ---------------------------------------------------------------- 5. where P is rounded
@pytest.mark.parametrize("p_dtype", ["float16", "bfloat16"])
def test_p_rounded_before_pv_and_l_from_unrounded_p(p_dtype):
    """One tile, V = identity: O[i, j] = round(p_ij) / l_i with p_i,argmax = 1 exactly.
    So O / O[:, argmax] recovers round(p) (fp16/bf16-representable), and the rows of O do not
    sum to 1 because l sums the unrounded p."""
    n = 32
    rng = np.random.default_rng(12)
    q, k = (rng.standard_normal((1, 1, n, n)).astype(np.float32) for _ in range(2))
    v = np.eye(n, dtype=np.float32)[None, None]
    exact = attention_online(q, k, v, bc=32)[0, 0]
    rnd = attention_online(q, k, v, bc=32, p_dtype=p_dtype)[0, 0]
    jmax = exact.argmax(axis=-1)
    rows = np.arange(n)
    ratio = rnd / rnd[rows, jmax][:, None]
    back = oracle.round_to(ratio.astype(np.float32), p_dtype)
    np.testing.assert_allclose(ratio, back, rtol=3e-7)         # representable in p_dtype
    p_exact = exact / exact[rows, jmax][:, None]
    assert not np.allclose(ratio, p_exact, rtol=1e-6)          # rounding did happen
    ulp = 2.0 ** -10 if p_dtype == "float16" else 2.0 ** -7
    assert np.abs(ratio - p_exact).max() <= ulp * 0.5 * 1.0001  # ... to nearest
    sums = rnd.sum(axis=-1)
    assert np.abs(sums - 1).max() > 1e-5                       # l not taken from rounded P
    np.testing.assert_allclose(sums * exact.sum(axis=-1), sums, rtol=1e-5)  # unrounded rows sum to 1


# ---------------------------------------------------------------- 6. bf16 rounding
def test_round_bf16_matches_torch():
    rng = np.random.default_rng(13)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10,
        (rng.integers(0, 2**16, 5000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),  # exact ties
        np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38, 1e-40], np.float32),
    ])
    x = x[np.isfinite(x) | np.isinf(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = round_bf16(x)
    assert np.array_equal(np.nan_to_num(want), np.nan_to_num(got))


# ---------------------------------------------------------------- 7. model of the MFMA kernel's arithmetic
@pytest.mark.parametrize("causal", [False, True])
def test_kernel_model_reduces_to_online_softmax(causal):
    """Threshold 0 (rescale whenever a max grows) and unrounded P: the same float32 operations
    as attention_online with 32-row blocks, so the results agree bit for bit."""
    rng = np.random.default_rng(21)
    q, k, v = (rng.standard_normal((2, 3, 150, 32)).astype(np.float32) for _ in range(3))
    got = oracle.attention_kernel_model(q, k, v, causal, p_dtype=None, bc=64, group=32, lazy_log2=0.0)
    want = attention_online(q, k, v, causal, br=32, bc=64)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [1.0, 4.0])
def test_kernel_model_lazy_rescale_is_exact(causal, scale):
    """O / l does not depend on which reference max is used: at threshold 8 (P up to 256) the
    result still matches float64 softmax to float32 accuracy, and rescales became rare."""
    rng = np.random.default_rng(22)
    q, k, v = (rng.standard_normal((1, 2, 300, 64)).astype(np.float32) for _ in range(3))
    q *= scale
    st_lazy, st_eager = {}, {}
    got = oracle.attention_kernel_model(q, k, v, causal, lazy_log2=8.0, stats=st_lazy)
    oracle.attention_kernel_model(q, k, v, causal, lazy_log2=0.0, stats=st_eager)
    want = attention_naive(q, k, v, causal)
    assert np.abs(got - want).max() < 2e-5
    assert 1.0 <= st_lazy["p_max"] <= 2.0 ** 8
    assert st_lazy["rescales"] < st_eager["rescales"]


def test_kernel_model_keeps_p_below_the_threshold():
    """Scores that keep growing along the row force rescales; P never exceeds 2^threshold."""
    n, d = 512, 16
    q = np.ones((1, 1, n, d), np.float32)
    k = (np.linspace(0, 12, n, dtype=np.float32)[:, None] * np.ones((1, d), np.float32))[None, None]
    v = np.random.default_rng(23).standard_normal((1, 1, n, d)).astype(np.float32)
    for thr in (2.0, 8.0):
        st = {}
        got = oracle.attention_kernel_model(q, k, v, lazy_log2=thr, stats=st)
        assert st["p_max"] <= 2.0 ** thr
        assert st["rescales"] > 1
        assert np.abs(got - attention_naive(q, k, v)).max() < 2e-5


@pytest.mark.parametrize("p_dtype,check", [("float16", "max"), ("bfloat16", "max"), ("bfloat16", "rounded")])
def test_kernel_model_dominant_key_returns_its_value(p_dtype, check):
    """One key dominates each row (every other P underflows to 0) and the stale max leaves its
    P = 2^x with fractional x, not representable in p_dtype. Summing l from the rounded P
    returns that key's V exactly; summing the unrounded P (the reference's rule) would scale it
    by round(p) / p."""
    n, d = 64, 64
    rng = np.random.default_rng(24)
    v = rng.standard_normal((1, 1, n, d)).astype(np.float32)
    # tile 0: every row's max is 0 (key 0); tile 1 (keys 32..63, bc=32): key 40 scores
    # 7.3 (log2 domain) above, inside the lazy threshold, and dominates everything else.
    s_log2 = np.full((n, n), -200.0, np.float32)
    s_log2[:, 0] = 0.0
    s_log2[:, 40] = 7.3
    d_q = d
    scale_log2 = np.float32(oracle.LOG2E / np.sqrt(d_q))
    # realise the scores with q = e_i-style rows: q k^T * scale_log2 = s_log2
    q = np.eye(n, d_q, dtype=np.float32)[None, None]
    k = np.zeros((1, 1, n, d_q), np.float32)
    k[0, 0, :, :n] = (s_log2 / scale_log2).T
    got = oracle.attention_kernel_model(q, k, v, p_dtype=p_dtype, bc=32, lazy_log2=8.0, check=check)
    p40 = np.float32(2.0) ** np.float32(7.3)
    w40 = oracle.round_to(np.array([p40], np.float32), p_dtype)[0]
    want = (w40 * v[0, 0, 40] + v[0, 0, 0]) / (w40 + 1)       # keys 0 and 40 carry all mass
    np.testing.assert_allclose(got[0, 0], np.broadcast_to(want, (n, d)), rtol=2e-6, atol=2e-6)
    unrounded_l = (w40 * v[0, 0, 40] + v[0, 0, 0]) / (p40 + 1)
    assert np.abs(unrounded_l - want).max() > 1e-4


# ---------------------------------------------------------------- 8. the bf16 kernel's overflow check
def test_bf16_top_exponent_bit_marks_values_from_two():
    """Every non-negative bf16 pattern up to +inf: bit 14 (the exponent's top bit) is set exactly
    when the value is >= 2, so an OR over packed P' patterns tests "some P' >= 2"."""
    pats = np.arange(0, 0x7F81, dtype=np.uint32)             # +0 .. +inf
    vals = (pats << 16).view(np.float32)
    assert np.array_equal((pats & 0x4000) != 0, vals >= 2.0)
    # the packed form: two patterns per 32-bit word, either half
    lo, hi = pats[:-1:2], pats[1::2]
    word = lo | (hi << 16)
    assert np.array_equal((word & 0x40004000) != 0, (vals[:-1:2] >= 2) | (vals[1::2] >= 2))


def test_bf16_rounding_commutes_with_power_of_two_scale():
    """round_bf16(x 2^-7) = round_bf16(x) 2^-7 for normal x: computing P' = P 2^-7 instead of P
    changes no rounding, only the common scale of O and l."""
    rng = np.random.default_rng(25)
    x = np.concatenate([np.exp2(rng.uniform(-100, 120, 200000)),
                        np.array([1.0, 2.0, 1.00390625, 1.005859375, 255.5, 256.0])]).astype(np.float32)
    a = oracle.round_bf16(x * np.float32(2.0 ** -7))
    b = oracle.round_bf16(x) * np.float32(2.0 ** -7)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [1.0, 4.0])
def test_kernel_model_rounded_check_is_exact(causal, scale):
    """check="rounded" with unrounded P: O / l still equals float64 softmax to float32 accuracy,
    P stays below 2^8, and it rescales no more often than the row-max rule."""
    rng = np.random.default_rng(26)
    q, k, v = (rng.standard_normal((1, 2, 300, 64)).astype(np.float32) for _ in range(3))
    q *= scale
    st_r, st_m = {}, {}
    got = oracle.attention_kernel_model(q, k, v, causal, lazy_log2=8.0, stats=st_r, check="rounded")
    oracle.attention_kernel_model(q, k, v, causal, lazy_log2=8.0, stats=st_m, check="max")
    assert np.abs(got - attention_naive(q, k, v, causal)).max() < 2e-5
    assert st_r["p_max"] < 2.0 ** 8
    assert st_r["rescales"] <= st_m["rescales"]


def test_kernel_model_rounded_check_rescales_growing_rows():
    """Scores that keep growing along the row: the rounded-P' check fires, P stays below 2^8 and
    the result matches the reference."""
    n, d = 512, 16
    q = np.ones((1, 1, n, d), np.float32)
    k = (np.linspace(0, 12, n, dtype=np.float32)[:, None] * np.ones((1, d), np.float32))[None, None]
    v = np.random.default_rng(27).standard_normal((1, 1, n, d)).astype(np.float32)
    st = {}
    got = oracle.attention_kernel_model(q, k, v, lazy_log2=8.0, stats=st, check="rounded", p_dtype="bfloat16")
    assert st["p_max"] < 2.0 ** 8 and st["rescales"] > 1
    assert np.abs(got - attention_naive(q, k, v)).max() < 2e-3


@pytest.mark.parametrize("n, causal", [(15, False), (64, False), (64, True), (65, True), (200, True)])
def test_kernel_model_two_term_p_on_single_tile_rows(n, causal):
    """Rows of at most 64 keys take P' as two bf16 terms (hi + lo carry ~16 significant bits):
    they then match float64 to ~2^-16 max|V| instead of half a bf16 ulp; rows of longer groups are
    bit for bit the one-term model."""
    rng = np.random.default_rng(n)
    q, k, v = (oracle.round_bf16(rng.standard_normal((2, n, 64)).astype(np.float32)) for _ in range(3))
    ref = attention_naive(q, k, v, causal)
    two = oracle.attention_kernel_model(q, k, v, causal, p_dtype="bfloat16", check="rounded")
    one = oracle.attention_kernel_model(q, k, v, causal, p_dtype="bfloat16", check="rounded", two_term=False)
    single = slice(0, 64 if causal else (n if n <= 64 else 0))   # groups whose rows see <= 64 keys
    vmax = float(np.abs(v).max())
    assert np.abs(two[:, single] - ref[:, single]).max(initial=0) <= 2.0 ** -16 * vmax
    rest = slice(single.stop, n)
    assert np.array_equal(two[:, rest], one[:, rest])
    if single.stop:
        assert np.abs(one[:, single] - ref[:, single]).max() > 4 * np.abs(two[:, single] - ref[:, single]).max()


# ---------------------------------------------------------------- 9. the fp16 kernels' packed-max check
F16_CHECK = dict(check="rounded", shift=4.0, fire=2.0 ** 14)   # fp16 non-causal persistent forms


def test_f16_packed_max_order_is_the_value_order():
    """Every non-negative fp16 value up to +inf: the packed max (v_pk_maximum3_f16) of the P'
    registers reaches 2^14 exactly when some P' does, and a P' that overflowed to inf reads as
    >= 2^14 too (it fires and is recomputed)."""
    pats = np.arange(0, 0x7C01, dtype=np.uint16)              # +0 .. +inf
    vals = pats.view(np.float16).astype(np.float32)
    rng = np.random.default_rng(28)
    for _ in range(200):
        pick = rng.choice(vals, 8)
        assert (np.maximum.reduce(pick) >= 2.0 ** 14) == np.any(pick >= 2.0 ** 14)
    assert np.float32(np.float16(np.inf)) >= 2.0 ** 14
    with np.errstate(over="ignore"):
        assert np.float16(np.float32(65520.0)) == np.inf      # the first fp32 value fp16 rounds to inf


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [1.0, 4.0])
def test_kernel_model_f16_check_is_exact(causal, scale):
    """The fp16 rule (m_ref = m + 4, fire when some P' >= 2^14) with unrounded P: O / l equals
    float64 softmax to float32 accuracy, P = P' 2^4 stays below 2^18, and it rescales no more
    often than the row-max rule with its 2^8 window."""
    rng = np.random.default_rng(29)
    q, k, v = (rng.standard_normal((1, 2, 300, 64)).astype(np.float32) for _ in range(3))
    q *= scale
    st_r, st_m = {}, {}
    got = oracle.attention_kernel_model(q, k, v, causal, stats=st_r, **F16_CHECK)
    oracle.attention_kernel_model(q, k, v, causal, lazy_log2=8.0, stats=st_m, check="max")
    assert np.abs(got - attention_naive(q, k, v, causal)).max() < 2e-5
    assert st_r["p_max"] < 2.0 ** 18
    assert st_r["rescales"] <= st_m["rescales"]


def test_kernel_model_f16_check_on_growing_and_peaked_rows():
    """Rows whose max keeps growing (18 octaves over the row) rescale under the fp16 rule and still
    match float64; peaked rows (scores spread ~13 octaves, as in C5) rescale less often than with
    the row-max rule, within the fp16 bar."""
    n, d = 512, 16
    q = np.ones((1, 1, n, d), np.float32)
    k = (np.linspace(0, 50, n, dtype=np.float32)[:, None] * np.ones((1, d), np.float32))[None, None]
    v = np.random.default_rng(30).standard_normal((1, 1, n, d)).astype(np.float32)
    st = {}
    got = oracle.attention_kernel_model(q, k, v, stats=st, p_dtype="float16", **F16_CHECK)
    assert st["rescales"] >= 1 and st["p_max"] < 2.0 ** 18
    assert np.abs(got - attention_naive(q, k, v)).max() < 2e-3
    rng = np.random.default_rng(31)
    qp, kp, vp = (rng.standard_normal((1, 4, 1024, 64)).astype(np.float32) for _ in range(3))
    qp, kp = (oracle.round_to(3 * x, "float16") for x in (qp, kp))
    vp = oracle.round_to(vp, "float16")
    st_r, st_m = {}, {}
    got = oracle.attention_kernel_model(qp, kp, vp, stats=st_r, p_dtype="float16", **F16_CHECK)
    oracle.attention_kernel_model(qp, kp, vp, lazy_log2=8.0, stats=st_m, p_dtype="float16", check="max")
    assert st_r["rescales"] < st_m["rescales"]
    assert np.abs(got - attention_naive(qp, kp, vp)).max() < 2e-3


def test_kernel_model_f16_check_dominant_key_returns_its_value():
    """A dominant key whose P' = 2^(x - m_ref) is not an fp16 value: l sums the rounded P', so the
    key's V comes back exactly, as under the other rules."""
    n, d = 64, 64
    rng = np.random.default_rng(32)
    v = rng.standard_normal((1, 1, n, d)).astype(np.float32)
    s_log2 = np.full((n, n), -200.0, np.float32)
    s_log2[:, 0] = 0.0
    s_log2[:, 40] = 11.3                      # past the row-max rule's 2^8 window, inside 2^(14+4)
    scale_log2 = np.float32(oracle.LOG2E / np.sqrt(d))
    q = np.eye(n, d, dtype=np.float32)[None, None]
    k = np.zeros((1, 1, n, d), np.float32)
    k[0, 0, :, :n] = (s_log2 / scale_log2).T
    st = {}
    got = oracle.attention_kernel_model(q, k, v, p_dtype="float16", bc=32, stats=st, **F16_CHECK)
    assert st["rescales"] == 0                # 11.3 - 4 octaves above m_ref: P' < 2^14, no rescale
    p40 = np.float32(2.0) ** np.float32(11.3 - 4.0)
    w40 = oracle.round_to(np.array([p40], np.float32), "float16")[0]
    w0 = np.float32(2.0 ** -4)
    want = (w40 * v[0, 0, 40] + w0 * v[0, 0, 0]) / (w40 + w0)
    np.testing.assert_allclose(got[0, 0], np.broadcast_to(want, (n, d)), rtol=2e-6, atol=2e-6)


def test_kernel_model_rejects_unknown_check():
    with pytest.raises(ValueError):
        oracle.attention_kernel_model(np.zeros((1, 4, 8), np.float32), np.zeros((1, 4, 8), np.float32),
                                      np.zeros((1, 4, 8), np.float32), check="sum")
