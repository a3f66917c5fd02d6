"""Tile sweep of the tuned fused kernel: every compiled (br, bc) x {one, two} LDS stages -> CSV.

    python phantom-a100_amd/bench/sweep_tiles.py                # N = 1024, 4096, 8192
    python phantom-a100_amd/bench/sweep_tiles.py --causal --ns 2048

Reference behaviour (/root/reference/bench/sweep_tiles.py:25-63): fp16, d = 64, every compiled
(BR, BC) with and without double buffering; each configuration is gated against ``fused`` first
(``wrong_result`` rows are not timed); configurations the device cannot run become
``skipped: <reason>`` rows; the fastest configuration per N is printed. The CSV columns are the
reference's. Timing uses the flushing protocol of benchmark.py.
"""
from __future__ import annotations

import argparse
import csv
import os
import sys

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(_HERE, ".."))
sys.path.insert(0, _HERE)
import cuda_attn  # noqa: E402
from cuda_attn import _checks  # noqa: E402
from cuda_attn.workloads import attention_flops  # noqa: E402

from benchmark import FLUSH_BYTES_MIN, time_calls  # noqa: E402

FIELDS = ["gpu", "N", "br", "bc", "double_buffer", "median_ms", "tflops", "status"]
CONFIGS = list(_checks.TUNED_CONFIGS)


def sweep(ns, batch, heads, causal, iters, warmup=5, writer=None, gpu=""):
    """Time every tile configuration at each N; returns {N: (median_ms, br, bc, double_buffer)}."""
    flush = torch.empty(FLUSH_BYTES_MIN, dtype=torch.uint8, device="cuda")
    gen = torch.Generator().manual_seed(0)
    best_by_n = {}
    for n in ns:
        q, k, v = (torch.randn(batch, heads, n, 64, generator=gen).half().cuda() for _ in range(3))
        ref = cuda_attn.fused(q, k, v, causal).float()
        best = None
        for br, bc in CONFIGS:
            for db in (False, True):
                fn = lambda: cuda_attn.fused_tuned(q, k, v, causal, db, br, bc)  # noqa: E731
                try:
                    err = (fn().float() - ref).abs().max().item()
                    if err > 2e-3:
                        if writer:
                            writer.writerow([gpu, n, br, bc, db, "", "", "wrong_result"])
                        continue
                    med, _, _ = time_calls(fn, warmup, iters, flush)
                except RuntimeError as e:
                    if writer:
                        writer.writerow([gpu, n, br, bc, db, "", "", "skipped: " + str(e).splitlines()[0][:80]])
                    continue
                tf = attention_flops(batch, heads, n, 64, causal) / (med * 1e-3) / 1e12
                if writer:
                    writer.writerow([gpu, n, br, bc, db, f"{med:.4f}", f"{tf:.3f}", "ok"])
                print(f"N={n:5} BR={br:3} BC={bc:3} double_buffer={db!s:5} {med:8.3f} ms {tf:7.2f} TFLOP/s")
                if best is None or med < best[0]:
                    best = (med, br, bc, db)
        if best:
            best_by_n[n] = best
            print(f"--> best at N={n}: BR={best[1]} BC={best[2]} double_buffer={best[3]} ({best[0]:.3f} ms)\n")
        del q, k, v, ref
    return best_by_n


def main(argv=None) -> str:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--ns", nargs="+", type=int, default=[1024, 4096, 8192])
    p.add_argument("--batch", type=int, default=4)
    p.add_argument("--heads", type=int, default=16)
    p.add_argument("--causal", action="store_true")
    p.add_argument("--iters", type=int, default=50)
    p.add_argument("--out", default=None)
    args = p.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("sweep_tiles.py needs a GPU")
    gpu = torch.cuda.get_device_name()
    out = args.out or os.path.join("results", "measured",
                                   f"tiles_{gpu.replace(' ', '_')}{'_causal' if args.causal else ''}.csv")
    os.makedirs(os.path.dirname(out) or ".", exist_ok=True)
    with open(out, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(FIELDS)
        sweep(args.ns, args.batch, args.heads, args.causal, args.iters, writer=w, gpu=gpu)
    print(f"wrote {out}")
    return out


if __name__ == "__main__":
    main()
