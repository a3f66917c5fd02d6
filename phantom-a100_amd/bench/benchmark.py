"""Benchmark sweep of the cuda_attn entry points (and torch SDPA) on one MI355X -> CSV.

    python phantom-a100_amd/bench/benchmark.py                         # full sweep
    python phantom-a100_amd/bench/benchmark.py --ns 1024 4096 --impls fused_tc sdpa_default

Same harness behaviour and CSV schema as the reference's bench/benchmark.py:106-190:
  * every run is first checked against the fp32 SDPA reference (``cuda_attn.reference``); a
    result outside the gate (1e-4 fp32, 2e-3 fp16; bf16: ``gate_bar``) is written as
    ``wrong_result`` and never timed;
  * timing: warm-up calls, then per timed call a zeroing of a flush buffer followed by one call
    between two HIP events; median and 10th / 90th percentiles;
  * peak device memory of one call above what was live before it (caching-allocator statistics);
  * configurations that cannot run are status rows, not crashes: ``unavailable`` (flash-attn is
    not installed on ROCm here), ``fp16_only``, ``unsupported_d``, ``skipped_oom`` (the N x N
    score workspace of naive / tiled / sdpa_math would not fit), ``oom``, ``error``.
MI355X-specific: the flush buffer must exceed the 256 MB Infinity Cache as well as L2, so it is
max(1 GiB, 2 x L2); ``cc`` records the gfx target and ``cuda`` the HIP version; fused_tc also
takes bf16 (the reference only fp16), so ``--dtype bf16`` exists.
"""
from __future__ import annotations

import argparse
import csv
import os
import sys
from datetime import datetime, timezone

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))
import cuda_attn  # noqa: E402
from cuda_attn.workloads import attention_flops  # noqa: E402

FIELDS = ["gpu", "cc", "torch", "cuda", "timestamp", "impl", "dtype", "causal", "B", "H", "N", "d",
          "median_ms", "p10_ms", "p90_ms", "tflops", "peak_mem_mb", "max_abs_err", "status"]
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
FLUSH_BYTES_MIN = 1 << 30   # > 256 MB Infinity Cache + L2 on MI355X


def sdpa_math(q, k, v, causal):
    with sdpa_kernel(SDPBackend.MATH):
        return F.scaled_dot_product_attention(q, k, v, is_causal=causal)


def sdpa_default(q, k, v, causal):
    return F.scaled_dot_product_attention(q, k, v, is_causal=causal)


IMPLS = {
    "naive": cuda_attn.naive,
    "tiled": cuda_attn.tiled,
    "fused": cuda_attn.fused,
    "fused_vec": cuda_attn.fused_vec,
    "fused_db": cuda_attn.fused_db,
    "fused_tc": cuda_attn.fused_tc,
    "sdpa_math": sdpa_math,
    "sdpa_default": sdpa_default,
    "flash2": None,  # flash-attn's CUDA package; not installable here
}
MATERIALIZES_S = {"naive", "tiled", "sdpa_math"}
FUSED_HEAD_DIMS = {"fused": (64,), "fused_vec": (64,), "fused_db": (64,), "fused_tc": (64, 128)}
ACCEPTS = {"fused_vec": (torch.float16,), "fused_db": (torch.float16,),
           "fused_tc": (torch.float16, torch.bfloat16),
           "naive": (torch.float16, torch.float32), "tiled": (torch.float16, torch.float32),
           "fused": (torch.float16, torch.float32)}


BF16_U = 2.0 ** -8   # bf16 unit roundoff: rounding to nearest moves x by at most 2^-8 |x|


def half_ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    """Half the spacing of bf16 values at |x| (8 significant bits): for |x| in [2^(e-1), 2^e) the
    spacing is 2^(e-8), so rounding x to bf16 moves it by at most 2^(e-9)."""
    _, e = torch.frexp(x.float())
    return torch.ldexp(torch.ones_like(x, dtype=torch.float32), e - 9)


def gate_bar(dtype: torch.dtype, ref: torch.Tensor, ref_absv: torch.Tensor | None = None,
             out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Element-wise pass bar of an output against the fp32 reference `ref`.

    fp32 inputs: 1e-4; fp16 inputs: 2e-3, the reference's bars (/root/reference/bench/benchmark.py:170).
    bf16 inputs (an extension): the attention weights P are rounded to bf16 before P.V, and one
    rounding can move an output further than 2e-3 on rows of few keys. With every weight rounded,
    p~ = p (1 + e), |e| <= u = 2^-8, and l the sum of the weights (rounded or not), the output moves by
    at most u / (1 - u) * (sum_j p_j |V_j| / sum_j p_j + |O|) (O~ - O = sum_j (p~_j - p_j) (V_j - O) / l~,
    since sum_j p_j (V_j - O) = 0). `ref_absv` is the first term, the reference attention of |V|.
    The bar is the larger of 2e-3 and that bound, element by element: it widens only where the
    weights' rounding can reach past 2e-3. A bf16 output also carries its own rounding: half a bf16
    ulp of the output is added."""
    if dtype == torch.float32:
        return torch.full_like(ref, 1e-4)
    bar = torch.full_like(ref, 2e-3)
    if dtype == torch.bfloat16:
        if ref_absv is None:
            raise ValueError("bf16 gate: the reference attention of |V| is needed")
        bar = torch.maximum(bar, BF16_U / (1 - BF16_U) * (ref_absv + ref.abs()))
    if out_dtype == torch.bfloat16:
        bar = bar + half_ulp_bf16(ref)
    return bar


def gate(out: torch.Tensor, ref: torch.Tensor, bar: torch.Tensor) -> tuple[float, bool]:
    """(max abs error against the fp32 reference, every element within its bar)."""
    err = (out.float() - ref).abs()
    return err.max().item(), bool((err <= bar).all().item())


def reference_pair(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool):
    """What the gate compares with: the fp32 SDPA reference and, for bf16 inputs, the fp32
    reference attention of |V| (gate_bar's bound), else None."""
    return (cuda_attn.reference(q, k, v, causal),
            cuda_attn.reference(q, k, v.abs(), causal) if q.dtype == torch.bfloat16 else None)


def gate_against(out: torch.Tensor, ref_pair, in_dtype: torch.dtype) -> tuple[float, bool]:
    """gate() of one output against reference_pair() of its inputs."""
    ref32, ref_absv = ref_pair
    return gate(out, ref32, gate_bar(in_dtype, ref32, ref_absv, out.dtype))


def workspace_bytes(name: str, b: int, h: int, n: int, d: int, elem: int) -> int:
    """Device bytes one call allocates: the fp32 N x N scores of the materialising paths (sdpa_math
    keeps scores and probabilities) plus the output."""
    out = b * h * n * d * elem
    if name not in MATERIALIZES_S:
        return out
    return b * h * n * n * 4 * (2 if name == "sdpa_math" else 1) + out


def fits_in_memory(name: str, b: int, h: int, n: int, d: int, elem: int, free_bytes: int) -> bool:
    """Skip a materialising kernel whose workspace cannot fit, instead of failing the sweep."""
    return workspace_bytes(name, b, h, n, d, elem) + 3 * b * h * n * d * elem < 0.85 * free_bytes


def status_before_run(name: str, dtype: torch.dtype, d: int) -> str | None:
    """Status row for a configuration the implementation does not take (None: runnable)."""
    if IMPLS.get(name) is None:
        return "unavailable"
    accepts = ACCEPTS.get(name)
    if accepts is not None and dtype not in accepts:
        return "fp16_only" if name in cuda_attn.FP16_ONLY else "unsupported_dtype"
    if name in FUSED_HEAD_DIMS and d not in FUSED_HEAD_DIMS[name]:
        return "unsupported_d"
    return None


def time_calls(fn, warmup: int, iters: int, flush_buf: torch.Tensor):
    """(median, p10, p90) in ms of `iters` calls under the reference's timing protocol
    (/root/reference/bench/benchmark.py:78-93, whose steps are kept so the numbers compare):
    untimed warm-up calls, then for every timed call a rewrite of `flush_buf` (so every cache level
    starts cold), the call between two HIP events on the current stream, and a host wait for it."""
    stream = torch.cuda.current_stream()
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    samples = []
    while len(samples) < iters:
        flush_buf.zero_()
        begin.record(stream)
        fn()
        end.record(stream)
        end.synchronize()
        samples.append(begin.elapsed_time(end))
    return summarize(samples)


def summarize(times) -> tuple[float, float, float]:
    """Median, 10th and 90th percentile (linear interpolation between order statistics)."""
    med, p10, p90 = np.percentile(np.asarray(times, dtype=np.float64), [50, 10, 90])
    return float(med), float(p10), float(p90)


def allocated_peak_mb(fn) -> float:
    """MiB the caching allocator held at its peak during one call above what was live before it
    (outputs and workspaces; the reference's peak_mem_mb column)."""
    torch.cuda.synchronize()
    live = torch.cuda.memory_stats().get("allocated_bytes.all.current", 0)
    torch.cuda.reset_peak_memory_stats()
    result = fn()
    torch.cuda.synchronize()
    peak = torch.cuda.memory_stats().get("allocated_bytes.all.peak", live)
    del result
    return (peak - live) / 2**20


def device_meta() -> dict:
    props = torch.cuda.get_device_properties(0)
    return dict(gpu=torch.cuda.get_device_name(), cc=getattr(props, "gcnArchName", "").split(":")[0],
                torch=torch.__version__, cuda=torch.version.hip or "",
                timestamp=datetime.now(timezone.utc).isoformat(timespec="seconds"))


class Sweep:
    """One benchmark run: the (causal, N) grid of input shapes, every implementation at each, one
    CSV row per (shape, implementation) written as soon as it is measured."""

    def __init__(self, args):
        self.args = args
        self.dtype = DTYPES[args.dtype]
        self.meta = device_meta()
        l2 = torch.cuda.get_device_properties(0).L2_cache_size
        self.flush = torch.empty(max(2 * l2, FLUSH_BYTES_MIN), dtype=torch.uint8, device="cuda")
        self.gen = torch.Generator().manual_seed(0)

    def shapes(self):
        modes = {"off": (False,), "on": (True,), "both": (False, True)}[self.args.causal]
        return [(causal, n) for causal in modes for n in self.args.ns]

    def inputs(self, n: int):
        a = self.args
        return [torch.randn(a.batch, a.heads, n, a.dim, generator=self.gen).to(self.dtype).cuda() for _ in range(3)]

    def measure(self, name: str, q, k, v, causal: bool, ref) -> dict:
        """The CSV row of one implementation at one shape: a status row if it cannot run here, else
        gated against `ref` (reference_pair() of the inputs, None above --ref-max-n), then timed
        and its allocation peak taken."""
        b, h, n, d = q.shape
        row = dict(self.meta, impl=name, dtype=self.args.dtype, causal=causal, B=b, H=h, N=n, d=d)
        status = status_before_run(name, q.dtype, d)
        if status is None and not fits_in_memory(name, b, h, n, d, q.element_size(), torch.cuda.mem_get_info()[0]):
            status = "skipped_oom"
        if status is not None:
            row["status"] = status
            return row
        impl = IMPLS[name]

        def call():
            return impl(q, k, v, causal)

        try:
            err = float("nan")
            if ref is not None:
                err, ok = gate_against(call(), ref, q.dtype)
                if not ok:
                    row.update(max_abs_err=f"{err:.2e}", status="wrong_result")
                    return row
            # naive re-reads S from HBM three times per call: fewer timed calls past N = 2048
            iters = self.args.iters if name != "naive" or n <= 2048 else max(10, self.args.iters // 10)
            med, p10, p90 = time_calls(call, self.args.warmup, iters, self.flush)
            mem = allocated_peak_mb(call)
        except torch.cuda.OutOfMemoryError:
            torch.cuda.empty_cache()
            row["status"] = "oom"
            return row
        except RuntimeError as e:
            print(f"{name} N={n}: {e}", file=sys.stderr)
            row["status"] = "error"
            return row
        tflops = attention_flops(b, h, n, d, causal) / (med * 1e-3) / 1e12
        row.update(median_ms=f"{med:.4f}", p10_ms=f"{p10:.4f}", p90_ms=f"{p90:.4f}", tflops=f"{tflops:.3f}",
                   peak_mem_mb=f"{mem:.1f}", max_abs_err=f"{err:.2e}", status="ok")
        return row

    def run(self, out: str) -> None:
        print(f"# {self.meta}")
        with open(out, "w", newline="") as fh:
            writer = csv.DictWriter(fh, fieldnames=FIELDS)
            writer.writeheader()
            for causal, n in self.shapes():
                q, k, v = self.inputs(n)
                ref = reference_pair(q, k, v, causal) if n <= self.args.ref_max_n else None
                for name in self.args.impls:
                    row = self.measure(name, q, k, v, causal, ref)
                    writer.writerow(row)
                    fh.flush()
                    print(report_line(row))
                del q, k, v, ref
                torch.cuda.empty_cache()


def report_line(row: dict) -> str:
    head = f"{row['impl']:12} N={row['N']:<5} causal={int(bool(row['causal']))}"
    if row.get("status") != "ok":
        return f"{head}  {row.get('status')}"
    return (f"{head}  {float(row['median_ms']):9.3f} ms  {float(row['tflops']):8.2f} TFLOP/s  "
            f"peak {float(row['peak_mem_mb']):8.1f} MiB  err {row['max_abs_err']}")


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--impls", nargs="+", default=list(IMPLS), choices=list(IMPLS))
    p.add_argument("--ns", nargs="+", type=int, default=[512, 1024, 2048, 4096, 8192])
    p.add_argument("--batch", type=int, default=4)
    p.add_argument("--heads", type=int, default=16)
    p.add_argument("--dim", type=int, default=64)
    p.add_argument("--dtype", choices=list(DTYPES), default="fp16")
    p.add_argument("--causal", choices=["off", "on", "both"], default="both")
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--iters", type=int, default=100)
    p.add_argument("--ref-max-n", type=int, default=4096, help="largest N checked against the fp32 reference")
    p.add_argument("--out", default=None)
    return p.parse_args(argv)


def main(argv=None) -> str:
    args = parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("benchmark.py needs a GPU")
    sweep = Sweep(args)
    out = args.out or os.path.join("results", "measured", f"bench_{sweep.meta['gpu'].replace(' ', '_')}.csv")
    os.makedirs(os.path.dirname(out) or ".", exist_ok=True)
    sweep.run(out)
    print(f"wrote {out}")
    return out


if __name__ == "__main__":
    main()
