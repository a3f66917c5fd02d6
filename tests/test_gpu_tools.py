"""GPU runs of the benchmark harness, the tile sweep and the counter-driven tile choice, at small
sizes: the CSV rows they write, their status rows, and a rocprofv3-profiled candidate whose
counters come back observable."""
from __future__ import annotations

import csv
import importlib.util
import os
import shutil
import sys

import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "phantom-a100_amd")
sys.path.insert(0, PKG)
sys.path.insert(0, os.path.join(PKG, "bench"))

pytestmark = pytest.mark.gpu


def load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def read_rows(path):
    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))


def test_benchmark_writes_status_and_timing_rows(tmp_path):
    bm = load("pa_benchmark_gpu", os.path.join(PKG, "bench", "benchmark.py"))
    out = str(tmp_path / "bench.csv")
    bm.main(["--ns", "64", "200", "--batch", "1", "--heads", "2", "--iters", "3", "--warmup", "1",
             "--causal", "both", "--impls", "naive", "tiled", "fused", "fused_vec", "fused_db", "fused_tc",
             "sdpa_math", "flash2", "--out", out])
    rows = read_rows(out)
    assert len(rows) == 2 * 2 * 8
    assert list(rows[0].keys()) == bm.FIELDS
    by = {(r["impl"], r["N"], r["causal"]): r for r in rows}
    for impl in ("naive", "tiled", "fused", "fused_vec", "fused_db", "fused_tc", "sdpa_math"):
        r = by[(impl, "200", "True")]
        assert r["status"] == "ok", r
        assert float(r["median_ms"]) > 0 and float(r["tflops"]) > 0 and float(r["max_abs_err"]) <= 2e-3
    assert by[("flash2", "64", "False")]["status"] == "unavailable"
    assert rows[0]["cc"].startswith("gfx9")


def test_benchmark_bf16_and_unsupported_rows(tmp_path):
    bm = load("pa_benchmark_gpu2", os.path.join(PKG, "bench", "benchmark.py"))
    out = str(tmp_path / "bench_bf16.csv")
    bm.main(["--ns", "128", "--batch", "1", "--heads", "2", "--dim", "128", "--dtype", "bf16", "--iters", "3",
             "--warmup", "1", "--causal", "off", "--impls", "fused_tc", "fused", "fused_vec", "--out", out])
    st = {r["impl"]: r["status"] for r in read_rows(out)}
    assert st == {"fused_tc": "ok", "fused": "unsupported_dtype", "fused_vec": "fp16_only"}


def test_sweep_tiles_covers_every_compiled_tile(tmp_path):
    sw = load("pa_sweep_gpu", os.path.join(PKG, "bench", "sweep_tiles.py"))
    out = str(tmp_path / "tiles.csv")
    sw.main(["--ns", "256", "--batch", "1", "--heads", "2", "--iters", "3", "--out", out])
    rows = read_rows(out)
    assert len(rows) == 8 and all(r["status"] == "ok" for r in rows)
    assert {(int(r["br"]), int(r["bc"]), r["double_buffer"]) for r in rows} == \
        {(br, bc, db) for br, bc in ((64, 32), (64, 64), (128, 32), (128, 64)) for db in ("False", "True")}


def test_select_tiles_picks_the_fastest_passing_candidate():
    from autotune import select_tiles as st
    best = st.main(["--entry", "fused_tuned", "--n", "512", "--batch", "1", "--heads", "4", "--iters", "3"])
    assert best is not None and best["status"] == "ok"
    assert best["regs"] > 0 and 1 <= best["waves_per_simd_limit"] <= 8


@pytest.mark.skipif(shutil.which("rocprofv3") is None, reason="rocprofv3 not installed")
@pytest.mark.parametrize("label, shown", [("br256_bc64_2stage", "br128_bc64_2stage (as launched)"),
                                          ("br128_bc64_2stage_persistent", "br128_bc64_2stage_persistent")])
def test_select_tiles_profiles_a_candidate(tmp_path, label, shown):
    """fused_tc at a small bf16 d=128 shape under rocprofv3, the shipped tile and one alternative of
    libphantom_attn_tiles.so (run by bench/run_one.py --candidate): the counters the rules use come
    back. On this 8-head grid fused_tc launches its 128-query tile, and the shipped row names it."""
    from autotune import select_tiles as st
    out = str(tmp_path / "report.md")
    print(f"[select_tiles profile] {label}", flush=True)
    best = st.main(["--entry", "fused_tc", "--dtype", "bf16", "--dim", "128", "--n", "1024", "--batch", "1",
                    "--heads", "8", "--iters", "3", "--profile", "--profile-dir", str(tmp_path / "prof"),
                    "--pass-timeout", "90", "--only", label, "--out", out])
    assert best is not None and best["candidate"] == shown
    assert best.get("profile_status") == "ok", best
    for key in ("mfma_util", "valu_busy", "hbm_bytes", "occupancy", "lds_active_cycles", "wait_frac"):
        assert best.get(key) is not None, key
    assert 0 < best["mfma_util"] <= 100
    assert os.path.exists(out) and "Chosen" in open(out).read()


def test_reference_workload_runs_the_harness_protocol():
    """The reference's measured shape through fused_tc and one fused_tuned point: gated, timed."""
    rw = load("pa_reference_workload", os.path.join(PKG, "bench", "reference_workload.py"))
    rows = rw.measure(["fused_tc", "fused_vec/br128/bc32"], iters=5)
    assert [r["status"] for r in rows] == ["ok", "ok"]
    for r in rows:
        assert r["median_ms"] > 0 and r["max_abs_err"] <= 2e-3 and r["speedup_vs_a100"] > 0


def test_tile_alternatives_compute_attention():
    """Every candidate of libphantom_attn_tiles.so on a small shape of its dtype and head dim: within
    the benchmark's gate of float64 attention (fp16 2e-3; bf16 the weights' rounding bound), and the
    shipped tile held to fewer workgroups per CU bitwise equal to fused_tc's own launch."""
    from autotune import tile_candidates as tc
    bm = load("pa_benchmark_gpu3", os.path.join(PKG, "bench", "benchmark.py"))
    import cuda_attn
    from autotune import select_tiles as st
    for c in tc.candidates():
        b, h, n, d = 2, 64, 512, c["d"]   # enough heads that fused_tc takes its persistent launch
        g = torch.Generator().manual_seed(c["index"])
        q, k, v = (torch.randn(b, h, n, d, generator=g).to(c["dtype"]).cuda() for _ in range(3))
        print(f"[tiles] {c['label']} {c['dtype']} d={d}: {tc.kernel(c['index'], b * h, n)}", flush=True)
        out = tc.forward(c["index"], q, k, v)
        torch.cuda.synchronize()
        ref32, ref_absv = bm.reference_pair(q, k, v, False)
        err, ok = bm.gate_against(out, (ref32, ref_absv), q.dtype)
        assert ok, (c["label"], err)
        if (c["br"], c["bc"], c["stages"]) == st.TC_TILE[d] and c["persistent"]:
            assert torch.equal(out, cuda_attn.fused_tc(q, k, v)), c["label"]
