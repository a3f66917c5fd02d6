"""The reference's own measured workload, timed the reference's way on one MI355X.

    python phantom-a100_amd/bench/reference_workload.py              # every entry point -> table
    python phantom-a100_amd/bench/reference_workload.py --out report.md

The reference published one set of hardware numbers for this path: an A100-SXM4-80GB at
BH = 324, N = 128, d = 64, fp16 inputs for every kernel, non-causal
(/root/reference/results/autotune/measured/hw_measurements.json:2-12). Its harness
(/root/reference/sim/harness.cu:77-86,146-163) draws Q, K, V ~ N(0, 1) rounded to fp16, checks the
output against a float reference at 2e-3, then runs 10 warm-up launches and times 200 launches one
by one (event, launch, event, synchronise; no cache flush) and reports the median. This module
repeats that protocol through the `cuda_attn` entry points that reach the same kernels:

    naive, tiled, fused (br64/bc32)       -> cuda_attn.naive / tiled / fused
    fused_vec/brX/bcY[/db]                -> cuda_attn.fused_tuned(br=X, bc=Y, double_buffer=db)
    fused_vec/br64/bc32, .../db           -> also cuda_attn.fused_vec / fused_db (their defaults)
    fused_tc                              -> cuda_attn.fused_tc

The harness-only points (the `/r128` register caps and `fused/br128`) have no Python entry point
and are not repeated.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys

import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))
import cuda_attn  # noqa: E402

SHAPE = (1, 324, 128, 64)          # (B, H, N, d): BH = 324 flattened as H
FLOPS = 4 * 324 * 128 * 128 * 64   # 4 * BH * N^2 * d
A100_SOURCE = "/root/reference/results/autotune/measured/hw_measurements.json"
# A100-SXM4-80GB medians (ms) of the points this API reaches, from A100_SOURCE ("points").
A100_MS = {
    "naive": 1.75677,
    "tiled": 0.4209,
    "fused/br64/bc32": 0.33792,
    "fused_vec/br64/bc32": 0.2393,
    "fused_vec/br64/bc32/db": 0.23677,
    "fused_vec/br64/bc64": 0.22288,
    "fused_vec/br64/bc64/db": 0.21728,
    "fused_vec/br128/bc32": 0.16432,
    "fused_vec/br128/bc32/db": 0.16307,
    "fused_vec/br128/bc64": 0.16378,
    "fused_vec/br128/bc64/db": 0.21901,
    "fused_tc": 0.06918,
}


def parse_point(point: str):
    """Reference point name -> (entry point, keyword arguments)."""
    if point in ("naive", "tiled", "fused_tc"):
        return point, {}
    if point == "fused/br64/bc32":
        return "fused", {}
    parts = point.split("/")
    if parts[0] != "fused_vec" or len(parts) not in (3, 4):
        raise ValueError(f"no entry point reaches {point!r}")
    br, bc = int(parts[1][2:]), int(parts[2][2:])
    db = len(parts) == 4 and parts[3] == "db"
    return "fused_tuned", {"br": br, "bc": bc, "double_buffer": db}


def harness_time(fn, warmup: int = 10, iters: int = 200) -> tuple[float, float]:
    """/root/reference/sim/harness.cu:146-163: warm-ups, then each launch alone between two events
    followed by a synchronise; median and minimum in ms."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    return statistics.median(times), min(times)


def inputs(seed: int = 1):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(SHAPE, generator=g).to(torch.float16).cuda() for _ in range(3))


def measure(points=None, iters: int = 200) -> list[dict]:
    q, k, v = inputs()
    ref = cuda_attn.reference(q, k, v, False)
    rows = []
    for point in points or list(A100_MS):
        name, kw = parse_point(point)
        fn_raw = getattr(cuda_attn, name)
        fn = lambda: fn_raw(q, k, v, False, **kw)  # noqa: E731
        err = (fn().float() - ref).abs().max().item()
        row = {"point": point, "entry": name, "kwargs": kw, "max_abs_err": float(f"{err:.3e}"),
               "a100_ms": A100_MS.get(point)}
        if not err <= 2e-3:
            row["status"] = "wrong_result"
        else:
            med, mn = harness_time(fn, iters=iters)
            row.update(status="ok", median_ms=round(med, 5), min_ms=round(mn, 5),
                       tflops=round(FLOPS / (med * 1e-3) / 1e12, 2))
            if row["a100_ms"]:
                row["speedup_vs_a100"] = round(row["a100_ms"] / med, 2)
        rows.append(row)
    return rows


def report(rows: list[dict], command: str) -> str:
    lines = ["# The reference's measured workload on MI355X: BH=324, N=128, d=64, fp16, non-causal", "",
             "Command (repo root):", "", f"    {command}", "",
             f"A100 column: the reference's medians ({A100_SOURCE}). Both columns use the reference",
             "harness protocol (sim/harness.cu:146-163): 10 warm-ups, then 200 launches each timed alone",
             "between two events, no cache flush, median. Gate: fp32 SDPA reference, 2e-3.", "",
             "| reference point | entry point here | A100 ms | MI355X ms | MI355X TFLOP/s | speed-up | max abs err |",
             "|---|---|---|---|---|---|---|"]
    for r in rows:
        kw = ", ".join(f"{k}={v}" for k, v in r["kwargs"].items())
        entry = f"{r['entry']}({kw})" if kw else r["entry"]
        if r["status"] == "ok":
            lines.append(f"| {r['point']} | {entry} | {r['a100_ms']} | {r['median_ms']:.5f} | {r['tflops']:.1f} | "
                         f"{r.get('speedup_vs_a100', '')}x | {r['max_abs_err']:.1e} |")
        else:
            lines.append(f"| {r['point']} | {entry} | {r['a100_ms']} | {r['status']} | | | {r['max_abs_err']:.1e} |")
    return "\n".join(lines) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--points", nargs="+", default=None, choices=list(A100_MS))
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--out", default=None, help="markdown report path")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("reference_workload.py needs a GPU")
    rows = measure(args.points, args.iters)
    for r in rows:
        print(json.dumps(r), flush=True)
    if args.out:
        cmd = f"python3 phantom-a100_amd/bench/reference_workload.py --out {args.out}"
        with open(args.out, "w") as fh:
            fh.write(report(rows, cmd))
    return rows


if __name__ == "__main__":
    main()
