"""Tile sweep of the tuned fused kernel: every compiled (br, bc) x {one, two} LDS stages -> CSV.

    python phantom-a100_amd/bench/sweep_tiles.py                # N = 1024, 4096, 8192
    python phantom-a100_amd/bench/sweep_tiles.py --causal --ns 2048

Behaviour of the reference's sweep (/root/reference/bench/sweep_tiles.py:25-63), kept so its CSVs
compare: fp16, d = 64, every compiled (BR, BC) with and without double buffering; a configuration
is first gated against ``fused`` (a ``wrong_result`` row is not timed); one the device cannot run
becomes a ``skipped: <reason>`` row; the fastest configuration per N is reported. The CSV columns
are the reference's. Timing uses benchmark.py's flushing protocol.
"""
import argparse
import csv
import os
import sys
from dataclasses import dataclass
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(_HERE, ".."))
sys.path.insert(0, _HERE)
import cuda_attn  # noqa: E402
from cuda_attn import _checks  # noqa: E402
from cuda_attn.workloads import attention_flops  # noqa: E402

from benchmark import FLUSH_BYTES_MIN, time_calls  # noqa: E402

FIELDS = ["gpu", "N", "br", "bc", "double_buffer", "median_ms", "tflops", "status"]
GATE = 2e-3   # the reference's bar for fp16 inputs against `fused`


@dataclass
class TileRun:
    """One (N, br, bc, stages) point of the sweep."""
    n: int
    br: int
    bc: int
    double_buffer: bool
    status: str = "ok"
    median_ms: Optional[float] = None
    tflops: Optional[float] = None

    def csv_row(self, gpu: str) -> list:
        timed = self.median_ms is not None
        return [gpu, self.n, self.br, self.bc, self.double_buffer, f"{self.median_ms:.4f}" if timed else "",
                f"{self.tflops:.3f}" if timed else "", self.status]


def tile_points():
    """Every compiled tuned configuration: (br, bc, double_buffer)."""
    return [(br, bc, db) for br, bc in _checks.TUNED_CONFIGS for db in (False, True)]


def run_tile(q, k, v, causal: bool, ref: torch.Tensor, point, iters: int, warmup: int, flush) -> TileRun:
    b, h, n, d = q.shape
    br, bc, db = point
    run = TileRun(n, br, bc, db)

    def call():
        return cuda_attn.fused_tuned(q, k, v, causal, db, br, bc)

    try:
        if (call().float() - ref).abs().max().item() > GATE:
            run.status = "wrong_result"
            return run
        run.median_ms = time_calls(call, warmup, iters, flush)[0]
    except RuntimeError as e:   # a tile the device cannot run: record why, keep sweeping
        reason = " ".join(str(e).split())
        run.status = f"skipped: {reason[:100]}"
        return run
    run.tflops = attention_flops(b, h, n, d, causal) / (run.median_ms * 1e-3) / 1e12
    return run


def sweep(ns, batch, heads, causal, iters, warmup=5, writer=None, gpu=""):
    """Run every tile point at each N; returns {N: (median_ms, br, bc, double_buffer)} of the
    fastest passing point."""
    flush = torch.empty(FLUSH_BYTES_MIN, dtype=torch.uint8, device="cuda")
    gen = torch.Generator().manual_seed(0)
    fastest = {}
    for n in ns:
        q, k, v = (torch.randn(batch, heads, n, 64, generator=gen).half().cuda() for _ in range(3))
        ref = cuda_attn.fused(q, k, v, causal).float()
        runs = [run_tile(q, k, v, causal, ref, pt, iters, warmup, flush) for pt in tile_points()]
        for r in runs:
            if writer:
                writer.writerow(r.csv_row(gpu))
            shown = f"{r.median_ms:8.3f} ms {r.tflops:7.2f} TFLOP/s" if r.status == "ok" else r.status
            print(f"N={n:<5} br={r.br:<3} bc={r.bc:<3} stages={2 if r.double_buffer else 1}  {shown}")
        ok = [r for r in runs if r.status == "ok"]
        if ok:
            top = min(ok, key=lambda r: r.median_ms)
            fastest[n] = (top.median_ms, top.br, top.bc, top.double_buffer)
            print(f"N={n}: fastest br={top.br} bc={top.bc} double_buffer={top.double_buffer} "
                  f"({top.median_ms:.3f} ms, {top.tflops:.1f} TFLOP/s)\n")
        del q, k, v, ref
    return fastest


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
    suffix = "_causal" if args.causal else ""
    out = args.out or os.path.join("results", "measured", f"tiles_{gpu.replace(' ', '_')}{suffix}.csv")
    os.makedirs(os.path.dirname(out) or ".", exist_ok=True)
    with open(out, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(FIELDS)
        sweep(args.ns, args.batch, args.heads, args.causal, args.iters, writer=w, gpu=gpu)
    print(f"wrote {out}")
    return out


if __name__ == "__main__":
    main()
