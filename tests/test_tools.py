"""CPU tests of the benchmark harness (phantom-a100_amd/bench) and the counter-driven tile choice
(phantom-a100_amd/autotune): status rules, the CSV schema, counter-pass limits, parsing of
rocprofv3 and compiler output recorded on gfx950 (tests/golden/rocprof), the occupancy model and
the bottleneck rules. The GPU runs of the same tools are in test_gpu_tools.py."""
from __future__ import annotations

import importlib.util
import os
import re
import sys

import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "phantom-a100_amd")
FIX = os.path.join(HERE, "golden", "rocprof")
sys.path.insert(0, PKG)

from autotune import diagnose as dg  # noqa: E402
from autotune import hw_counters as hc  # noqa: E402
from autotune import select_tiles as st  # noqa: E402
from cuda_attn import _native  # noqa: E402


def load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


benchmark = load("pa_benchmark", os.path.join(PKG, "bench", "benchmark.py"))
build_native = load("pa_build_native", os.path.join(PKG, "build_native.py"))
rw = load("pa_reference_workload", os.path.join(PKG, "bench", "reference_workload.py"))


# ---------------------------------------------------------------- benchmark harness
def test_csv_schema_is_the_references():
    # /root/reference/bench/benchmark.py:132-133
    assert benchmark.FIELDS == ["gpu", "cc", "torch", "cuda", "timestamp", "impl", "dtype", "causal", "B", "H", "N",
                                "d", "median_ms", "p10_ms", "p90_ms", "tflops", "peak_mem_mb", "max_abs_err", "status"]


@pytest.mark.parametrize("name,dtype,d,want", [
    ("flash2", torch.float16, 64, "unavailable"),
    ("fused_vec", torch.float32, 64, "fp16_only"),
    ("fused_db", torch.bfloat16, 64, "fp16_only"),
    ("fused_tc", torch.float32, 64, "fp16_only"),
    ("fused_tc", torch.bfloat16, 128, None),
    ("fused_tc", torch.float16, 80, "unsupported_d"),
    ("fused", torch.float32, 128, "unsupported_d"),
    ("fused", torch.float32, 64, None),
    ("naive", torch.bfloat16, 64, "unsupported_dtype"),
    ("naive", torch.float16, 80, None),
    ("sdpa_math", torch.bfloat16, 80, None),
])
def test_status_rows(name, dtype, d, want):
    assert benchmark.status_before_run(name, dtype, d) == want


def test_workspace_accounting():
    b, h, n, d = 4, 16, 8192, 64
    s = b * h * n * n * 4
    o = b * h * n * d * 2
    assert benchmark.workspace_bytes("naive", b, h, n, d, 2) == s + o
    assert benchmark.workspace_bytes("sdpa_math", b, h, n, d, 2) == 2 * s + o
    assert benchmark.workspace_bytes("fused_tc", b, h, n, d, 2) == o
    assert not benchmark.fits_in_memory("naive", b, h, n, d, 2, free_bytes=16 << 30)
    assert benchmark.fits_in_memory("naive", b, h, n, d, 2, free_bytes=288 << 30)
    assert benchmark.fits_in_memory("fused_tc", b, h, n, d, 2, free_bytes=1 << 30)


def test_summary_statistics():
    med, p10, p90 = benchmark.summarize([float(x) for x in range(1, 101)])
    assert med == 50.5 and p10 < 12 and p90 > 89
    assert benchmark.summarize([2.0]) == (2.0, 2.0, 2.0)


def test_bf16_half_ulp_is_the_largest_rounding_move():
    """Over every finite positive bf16 pattern's midpoints to its neighbours: rounding to bf16 moves a
    value by at most half_ulp_bf16, and a value just past the midpoint moves by almost exactly that."""
    pats = torch.arange(0x0080, 0x7F7F, dtype=torch.int32).to(torch.int16)   # normal bf16, +0x80 .. max-1
    lo = pats.view(torch.bfloat16).float()
    hi = (pats + 1).view(torch.bfloat16).float()
    mid = (lo.double() + hi.double()) / 2
    x = torch.nextafter(mid, torch.zeros_like(mid)).float()                    # just below the midpoint
    moved = (x.to(torch.bfloat16).float().double() - x.double()).abs()
    bound = benchmark.half_ulp_bf16(x).double()
    assert (moved <= bound).all()
    assert ((bound - moved) <= bound * 2.0 ** -14).all()
    assert benchmark.half_ulp_bf16(torch.tensor([1.0, 1.99, 2.0, 0.75])).tolist() == [2.0 ** -8, 2.0 ** -8,
                                                                                       2.0 ** -7, 2.0 ** -9]


def test_gate_bars_for_fp32_and_fp16_are_the_references():
    ref = torch.tensor([3.0, -2.5, 0.1])
    assert (benchmark.gate_bar(torch.float32, ref) == 1e-4).all()
    assert (benchmark.gate_bar(torch.float16, ref, out_dtype=torch.float16) == 2e-3).all()
    out16 = ref.to(torch.float16)
    err, ok = benchmark.gate(out16, ref, benchmark.gate_bar(torch.float16, ref, out_dtype=torch.float16))
    assert ok and err == (out16.float() - ref).abs().max().item()
    err, ok = benchmark.gate(ref + 3e-3, ref, benchmark.gate_bar(torch.float16, ref))
    assert not ok and err == pytest.approx(3e-3, rel=1e-4)


def _bf16_weights_attention(s, v):
    """O with every weight rounded to bf16 and l the sum of the rounded weights (float64)."""
    p = torch.softmax(s.double(), dim=-1)
    pr = p.float().to(torch.bfloat16).double()
    return (pr @ v.double()) / pr.sum(-1, keepdim=True), p @ v.double(), p @ v.double().abs()


def test_bf16_gate_admits_the_weights_rounding_and_no_more():
    """Two keys with weights near 0.4 / 0.6 and V = +4 / -4: rounding the weights to bf16 moves O
    past 2e-3, inside the bound u / (1 - u) (sum p|V| + |O|); a planted error of twice the bound
    fails, and so does one of 3e-3 on a row whose bound stays under 2e-3."""
    s = torch.tensor([[0.0, 0.41]])                   # p = 0.398.. / 0.601..
    v = torch.tensor([[4.0], [-4.0]])
    got, ref, ref_absv = _bf16_weights_attention(s, v)
    ref, ref_absv, got = ref.float(), ref_absv.float(), got.float()
    moved = (got - ref).abs().item()
    assert moved > 2e-3
    bar = benchmark.gate_bar(torch.bfloat16, ref, ref_absv, out_dtype=torch.float32)
    assert moved <= bar.item()
    assert benchmark.gate(got, ref, bar)[1]
    assert not benchmark.gate(ref + 2 * bar, ref, bar)[1]
    # many keys of similar weight and small |V|: the bound is below 2e-3, the bar stays there
    g = torch.Generator().manual_seed(5)
    s = torch.randn(4, 512, generator=g) * 0.1
    v = torch.randn(512, 8, generator=g) * 0.2
    got, ref, ref_absv = (t.float() for t in _bf16_weights_attention(s, v))
    bar = benchmark.gate_bar(torch.bfloat16, ref, ref_absv, out_dtype=torch.float32)
    assert (bar == 2e-3).all() and benchmark.gate(got, ref, bar)[1]
    assert not benchmark.gate(ref + 3e-3, ref, bar)[1]


def test_bf16_gate_bound_holds_on_random_rows():
    """The bound is a worst case: over random rows of 1-64 keys (the short causal rows where it
    matters), rounding every weight to bf16 never moves O past it."""
    g = torch.Generator().manual_seed(6)
    for keys in (1, 2, 3, 5, 8, 17, 64):
        s = torch.randn(256, keys, generator=g) * 3
        v = torch.randn(keys, 16, generator=g) * 2
        got, ref, ref_absv = _bf16_weights_attention(s, v)
        bound = benchmark.BF16_U / (1 - benchmark.BF16_U) * (ref_absv + ref.abs())
        assert ((got - ref).abs() <= bound * (1 + 1e-9)).all(), keys


def test_gate_against_reference_pair_on_attention():
    """The harness's own path: reference_pair() of bf16 inputs (fp32 SDPA, on the CPU here) and
    gate_against() of an output whose weights were rounded to bf16 pass, causal rows included;
    the same output shifted by 0.05 on one row fails. fp16 inputs need no |V| reference."""
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(1, 2, 96, 32, generator=g).to(torch.bfloat16) for _ in range(3))
    for causal in (False, True):
        pair = benchmark.reference_pair(q, k, v, causal)
        assert pair[1] is not None and pair[1].shape == pair[0].shape
        s = (q.double() @ k.double().transpose(-1, -2)) / 32 ** 0.5
        if causal:
            s = s.masked_fill(torch.ones(96, 96, dtype=torch.bool).triu(1), float("-inf"))
        p = torch.softmax(s, -1).float().to(torch.bfloat16).double()
        out = ((p @ v.double()) / p.sum(-1, keepdim=True)).to(torch.bfloat16)
        err, ok = benchmark.gate_against(out, pair, torch.bfloat16)
        assert ok, err
        bad = out.clone()
        bad[0, 1, 40] += 0.05
        assert not benchmark.gate_against(bad, pair, torch.bfloat16)[1]
    assert benchmark.reference_pair(q.half(), k.half(), v.half(), False)[1] is None


def test_bf16_gate_allows_the_outputs_rounding():
    ref = torch.tensor([3.0, -2.5, 0.1, 1.0 + 2.0 ** -8 + 2.0 ** -12])
    absv = ref.abs()
    out = ref.to(torch.bfloat16)                      # pure output rounding: passes
    bar = benchmark.gate_bar(torch.bfloat16, ref, absv, out_dtype=torch.bfloat16)
    assert benchmark.gate(out, ref, bar)[1]
    assert not benchmark.gate((ref + torch.tensor([0.0, 0.0, 0.01, 0.0])).to(torch.bfloat16), ref, bar)[1]


def test_tile_sweep_points_and_rows():
    """The tile sweep loads by path (as the GPU test does) and covers every compiled tile."""
    sw = load("pa_sweep_tiles", os.path.join(PKG, "bench", "sweep_tiles.py"))
    assert sorted(sw.tile_points()) == sorted((br, bc, db) for br, bc in ((64, 32), (64, 64), (128, 32), (128, 64))
                                              for db in (False, True))
    assert sw.TileRun(256, 64, 32, True).csv_row("gpu") == ["gpu", 256, 64, 32, True, "", "", "ok"]
    assert sw.TileRun(256, 64, 32, False, "ok", 1.5, 2.25).csv_row("gpu")[5:] == ["1.5000", "2.250", "ok"]
    assert sw.FIELDS == ["gpu", "N", "br", "bc", "double_buffer", "median_ms", "tflops", "status"]


def test_flush_buffer_exceeds_infinity_cache():
    assert benchmark.FLUSH_BYTES_MIN > 256 * 2**20


# ---------------------------------------------------------------- the reference's measured workload
def test_reference_workload_points_map_to_entry_points():
    assert rw.parse_point("fused_tc") == ("fused_tc", {})
    assert rw.parse_point("fused/br64/bc32") == ("fused", {})
    assert rw.parse_point("fused_vec/br128/bc32/db") == ("fused_tuned", {"br": 128, "bc": 32, "double_buffer": True})
    assert rw.parse_point("fused_vec/br64/bc64") == ("fused_tuned", {"br": 64, "bc": 64, "double_buffer": False})
    with pytest.raises(ValueError):
        rw.parse_point("fused/br128/bc32")            # harness-only launcher argument
    for point in rw.A100_MS:
        name, kw = rw.parse_point(point)
        if name == "fused_tuned":
            assert (kw["br"], kw["bc"]) in {(64, 32), (64, 64), (128, 32), (128, 64)}


def test_reference_workload_flops_match_the_published_derivation():
    """4 * 324 * 128^2 * 64 FLOP over the A100's 0.06918 ms is the 19.64 TFLOP/s derived for the
    reference's fused_tc."""
    assert rw.FLOPS == 1_358_954_496
    assert round(rw.FLOPS / (rw.A100_MS["fused_tc"] * 1e-3) / 1e12, 2) == 19.64


def test_reference_workload_report_lists_every_row():
    rows = [{"point": "fused_tc", "entry": "fused_tc", "kwargs": {}, "max_abs_err": 1e-4, "a100_ms": 0.06918,
             "status": "ok", "median_ms": 0.01, "min_ms": 0.009, "tflops": 135.9, "speedup_vs_a100": 6.92},
            {"point": "naive", "entry": "naive", "kwargs": {}, "max_abs_err": 1.0, "a100_ms": 1.75677,
             "status": "wrong_result"}]
    text = rw.report(rows, "cmd")
    assert "| fused_tc | fused_tc | 0.06918 | 0.01000 | 135.9 | 6.92x |" in text
    assert "| naive | naive | 1.75677 | wrong_result |" in text


# ---------------------------------------------------------------- counter passes and parsing
def test_passes_fit_the_hardware_limits():
    for p in hc.PASSES:
        hc.check_pass(p)
    with pytest.raises(ValueError):
        hc.check_pass(["FETCH_SIZE", "WRITE_SIZE"])           # 5 TCC counters
    with pytest.raises(ValueError):
        hc.check_pass([f"SQ_X{i}" for i in range(9)])           # 9 SQ counters
    with pytest.raises(ValueError):
        hc.check_pass(["GRBM_GUI_ACTIVE", "GRBM_COUNT", "GRBM_X"])


def test_every_mapped_counter_is_collected_by_some_pass():
    collected = {c for p in hc.PASSES for c in p}
    for key, m in hc.MAPPING.items():
        for c in m["counters"]:
            assert c in collected, (key, c)


def fixture_passes():
    return [hc.parse_counter_csv(os.path.join(FIX, f"c4_pass{i}_counter_collection.csv")) for i in range(4)]


def test_fixture_passes_are_the_tools_passes():
    for p, rows in zip(hc.PASSES, fixture_passes()):
        names = {k for d in rows.values() for k in d if k.isupper()}
        assert names == set(p)


def test_parse_counter_csv_and_aggregate():
    """C4 (bf16, B=4 H=32 N=4096 d=128) profiled on MI355X by select_tiles.py: one copy of 1 GiB
    (the FETCH_SIZE calibration) and the steady-state fused_tc dispatch."""
    passes = fixture_passes()
    d, calib = hc.merge_passes(passes, "fa_mfma_fwd")
    assert 1.9 < calib < 2.1                              # FETCH_SIZE reads half of a copy's bytes
    for c in {c for p in hc.PASSES for c in p} - {"SQ_LDS_BANK_CONFLICT"}:
        assert d[c] is not None and d[c] > 0, c
    assert d["SQ_LDS_BANK_CONFLICT"] == 0                 # the XOR-swizzled K/V rows never conflict
    assert d["grid"] == 1048576 and d["workgroup"] == 512 and d["lds"] == 65536
    trace = hc.parse_kernel_trace(os.path.join(FIX, "c4_kernel_trace.csv"))
    d["duration_ns"] = trace[-1]["duration_ns"]
    agg = hc.aggregate([d], {"vgprs": 238, "agprs": 0, "lds_bytes": 65536}, fetch_calibration=calib)
    compulsory = (3 * 2 + 2) * 128 * 4096 * 128
    assert abs(agg["hbm_bytes"] / compulsory - 1) < 0.01  # C4 streams Q, K, V, O once
    assert 30 < agg["mfma_util"] < 80                     # about 52 % in the committed C4 profile
    assert agg["waves_per_simd_limit"] == 2 and agg["occupancy_limiter"] == "vgpr"
    assert 10 < agg["occupancy"] <= 25                    # 2 of 8 waves per SIMD resident at most
    assert 0 < agg["wait_frac"] < 1
    assert agg["workgroups"] == 2048
    flops = 4 * 128 * 4096 ** 2 * 128
    assert 500 < flops / (agg["cycles"] * 1e-9) / 1e12 < 2000   # the trace's kernel time is the C4 rate


def test_aggregate_formulas_on_known_numbers():
    grbm_per_xcd = 1_000_000
    d = {"kernel": "k", "duration_ns": 1000, "grid": 256 * 64, "workgroup": 64,
         "GRBM_GUI_ACTIVE": grbm_per_xcd * hc.XCDS,
         "SQ_VALU_MFMA_BUSY_CYCLES": 0.25 * grbm_per_xcd * hc.CUS * hc.SIMDS_PER_CU,
         "SQ_WAVE_CYCLES": 0.5 * grbm_per_xcd * hc.CUS * 32 / 4,
         "SQ_ACTIVE_INST_VALU": 0.4 * grbm_per_xcd * hc.CUS,
         "SQ_WAIT_INST_ANY": 0.2 * 0.5 * grbm_per_xcd * hc.CUS * 32 / 4,   # 20 % of the wave cycles
         "FETCH_SIZE": 100.0, "WRITE_SIZE": 50.0}
    a = hc.aggregate([d], None, fetch_calibration=2.0)
    assert a["mfma_util"] == pytest.approx(25.0)
    assert a["occupancy"] == pytest.approx(50.0)
    assert a["valu_busy"] == pytest.approx(40.0)
    assert a["wait_frac"] == pytest.approx(0.2)
    assert a["hbm_bytes"] == pytest.approx(100 * 1024 * 2 + 50 * 1024)
    missing = hc.aggregate([{"kernel": "k", "duration_ns": 5}], None)
    assert missing["mfma_util"] is None and missing["hbm_bytes"] is None   # unobservable, not zero


def test_parse_kernel_trace():
    rows = hc.parse_kernel_trace(os.path.join(FIX, "c4_kernel_trace.csv"))
    assert len(rows) == 4 and "fa_mfma_fwd" in rows[-1]["kernel"]
    assert all(r["duration_ns"] > 0 for r in rows)
    assert rows[-1]["grid"] == 1048576 and rows[-1]["workgroup"] == 512


# ---------------------------------------------------------------- compiler resources and occupancy
def resources_fixture():
    with open(os.path.join(FIX, "resource_remarks.txt")) as fh:
        return build_native.parse_resource_remarks(fh.read())


def test_parse_resource_remarks():
    res = resources_fixture()
    assert len(res) == 5
    c4 = [v for k, v in res.items() if "fa_mfma_fwdIDF16bLi128ELi256ELi64ELi2EDF16bLi1ELb1ELb0ELb0E" in k][0]   # persistent
    # 64 KB of K/V stages and 64 KB of O staging rows
    assert c4["vgprs"] == 224 and c4["agprs"] == 0 and c4["lds_bytes"] == 131072
    assert c4["occupancy_waves_per_simd"] == 2 and c4["vgpr_spill"] == 0 and c4["scratch_bytes"] == 0


def test_vgpr_occupancy_model_agrees_with_the_compiler():
    """Our VGPR limit (512 registers per lane, granule 8, at most 8 waves) gives the compiler's
    reported occupancy for every kernel of the fixture (none of them is LDS-limited at its launch
    size)."""
    for name, r in resources_fixture().items():
        waves, _ = hc.theoretical_waves_per_simd(r["vgprs"], r["agprs"], 0, 64)
        assert waves == r["occupancy_waves_per_simd"], name


@pytest.mark.parametrize("vgprs,lds,threads,want", [
    (238, 65536, 512, (2, "vgpr")),
    (96, 8192, 256, (5, "vgpr")),
    (128, 16384, 256, (4, "vgpr")),
    (64, 65536, 256, (2, "lds")),        # 2 workgroups of 4 waves fit in 160 KB
    (16, 0, 64, (8, "waves")),
])
def test_theoretical_waves(vgprs, lds, threads, want):
    assert hc.theoretical_waves_per_simd(vgprs, 0, lds, threads) == want


def test_candidates_name_compiled_kernels():
    res = resources_fixture()
    # the fixture holds one fused_tuned instantiation and the persistent d=128 fused_tc one
    assert st.find_resources(res, st.kernel_key(torch.float16, 64, 128, 32, 1, torch.float16))
    assert st.find_resources(res, st.kernel_key(torch.bfloat16, 128, 256, 64, 2, torch.bfloat16, persistent=True))
    assert not st.find_resources(res, st.kernel_key(torch.bfloat16, 128, 256, 64, 2, torch.bfloat16))
    assert len(st.candidates("fused_tuned", 64)) == 8
    assert st.candidates("fused_tc", 128, with_alternatives=False) == [
        ("br256_bc64_2stage", 256, 64, 2, st.SHIPPED), ("br256_bc64_2stage_per_block", 256, 64, 2, st.PER_BLOCK)]


def test_tile_alternatives_library_without_gpu():
    """libphantom_attn_tiles.so loads, exports what its header declares, lists at least three
    alternatives per fused_tc head dim (none of them the shipped tile) with distinct labels, and
    rejects calls it does not compile before any HIP call."""
    import ctypes
    from autotune import tile_candidates as tc
    header = os.path.join(os.path.dirname(HERE), "include", "phantom_attn_tiles.h")
    text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(pa_[a-z0-9_]+)\s*\(", text)))
    assert declared == sorted(tc.PROTOTYPES)
    for name in declared:
        assert ctypes.cast(getattr(tc.lib(), name), ctypes.c_void_p).value, name
    cands = tc.candidates()
    assert len({c["label"] for c in cands}) == len(cands)
    for d, dtype in ((128, torch.bfloat16), (64, torch.float16)):
        alts = [c for c in cands if c["d"] == d and c["dtype"] == dtype]
        assert len(alts) >= 3, d
        shipped = st.TC_TILE[d]
        # an alternative with the shipped tile differs in its launch (per block, or fewer workgroups
        # per CU), except d = 128's persistent 256-query tile: the alternative on the grids where
        # fused_tc launches the 128-query tile (select_tiles skips it where it is the shipped launch)
        assert all((c["br"], c["bc"], c["stages"]) != shipped or not c["persistent"] or c["wgs_per_cu"] > 0
                   or c["label"] == "br256_bc64_2stage_persistent_d128" for c in alts)
        rows = st.candidates("fused_tc", d, dtype)
        assert rows[0][4] == st.SHIPPED and len(rows) == 2 + len(alts)
        assert [r[0] for r in rows[2:]] == [c["label"] for c in alts]
    c0 = cands[0]
    desc = tc.kernel(c0["index"], 128, 4096)
    assert desc.startswith(f"fa_mfma_fwd<bf16, D={c0['d']}, BM={c0['br']}, BN={c0['bc']}") and "grid" in desc
    lib, p = tc.lib(), ctypes.c_void_p(256)   # never dereferenced: validation fails first
    rc = lib.pa_tiles_fwd(c0["index"], p, p, p, p, _native.DTYPE_BF16, 1, 4096, c0["d"], 1, None)
    assert rc == _native.ERR_UNSUPPORTED and b"non-causal" in lib.pa_tiles_last_error()
    rc = lib.pa_tiles_fwd(c0["index"], p, p, p, p, _native.DTYPE_F16, 1, 4096, c0["d"], 0, None)
    assert rc == _native.ERR_UNSUPPORTED and b"compiled for" in lib.pa_tiles_last_error()
    rc = lib.pa_tiles_fwd(len(cands), p, p, p, p, _native.DTYPE_BF16, 1, 4096, 128, 0, None)
    assert rc == _native.ERR_INVALID
    assert lib.pa_tiles_label(-1) == b""


# ---------------------------------------------------------------- bottleneck rules
def test_rules_fire_on_their_evidence():
    comp = 1e6
    cases = {
        "materialized_intermediate": dict(kernel_launches=3, hbm_bytes=5e6),
        "redundant_hbm_traffic": dict(hbm_bytes=3.5e6),
        "vgpr_limited_occupancy": dict(waves_per_simd_limit=1, occupancy_limiter="vgpr", regs=300),
        "lds_limited_occupancy": dict(waves_per_simd_limit=1, occupancy_limiter="lds"),
        "scalar_math_bound": dict(mfma_insn=0, valu_busy=80.0),
        "valu_bound_softmax": dict(mfma_insn=100, mfma_util=40.0, valu_busy=55.0),
        "lds_bank_conflicts": dict(lds_bank_conflict_cycles=10.0, lds_active_cycles=100.0),
        "latency_bound": dict(wait_frac=0.7, occupancy=20.0),
        "low_parallelism": dict(workgroups=42, resident_wgs_per_cu=2),
        "register_spills": dict(spill=16),
    }
    assert set(cases) == set(dg.THRESHOLDS)
    for rule, counters in cases.items():
        got = [f.rule for f in dg.diagnose(counters, comp)]
        assert rule in got, (rule, got)
        assert all(f.score >= 1 for f in dg.diagnose(counters, comp))


def test_clean_point_triggers_nothing():
    c4_like = dict(kernel_launches=1, hbm_bytes=1.0004e6, waves_per_simd_limit=2, occupancy_limiter="vgpr",
                   mfma_insn=1000, mfma_util=65.0, valu_busy=43.0, lds_bank_conflict_cycles=0.0,
                   lds_active_cycles=100.0, wait_frac=0.3, occupancy=25.0, workgroups=2048,
                   resident_wgs_per_cu=1, spill=0)
    assert dg.diagnose(c4_like, 1e6) == []


def test_unobservable_inputs_disable_rules():
    assert dg.diagnose({}, None) == []
    assert dg.resident_wgs_per_cu(2, 512) == 1 and dg.resident_wgs_per_cu(4, 256) == 4
