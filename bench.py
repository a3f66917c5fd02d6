"""Benchmark of the attention forward path on one MI355X; prints ONE JSON line.

    python bench.py                         # N=1: headline C4 + per-config table + CPU baselines
    python bench.py --steps 100 --warmup 25
    python bench.py --mode pmc              # short fixed workload for rocprofv3 --pmc runs

A step is one cuda_attn.fused_tc call on the headline workload, C4: non-causal SDPA forward,
B=4 H=32 N=4096 d=128, bf16 inputs from a seeded generator (synthetic data), already resident in
HBM. `value` = 4*B*H*N^2*d FLOPs per step x steps / the time of the K steps between two
synchronisations (HIP events on the launch stream). MI355X raises its clock over the first ~30
launches of this kernel, so before the warm-up a fixed-duration settle phase (--settle seconds of
back-to-back calls, reported as `settle`) brings the clock to its steady state; the warm-up and
the timed steps are exactly --warmup and --steps calls. A host thread samples amdsmi's per-XCD
shader clocks and the socket power during the settle's last second and during the warm-up and timed
steps (`clock`; null where amdsmi does not import), so the line can be read against the clock the
box held under its power cap. Every config of the measurement plan is
also timed with the reference's protocol (/root/reference/bench/benchmark.py:78-93: warm-ups,
then per call a flush of a buffer larger than the 256 MB Infinity Cache, event timing,
median/p10/p90), each after its own settle phase, and reported under "per_config" beside the
measured device copy bandwidth. Before timing, outputs are gated against a float64 GPU reference
on sampled heads. The CPU baseline is the oracle's NumPy restatement of the reference's online
softmax (oracle/online_softmax.py, br=64 bc=32, P rounded to the config's input dtype), and
beside it the row-chunked float64 reference, timed for every config on whole-head samples of
the same inputs (median of 3 runs) on the host's cores. "reference_workload" times fused_tc on
the one shape the reference measured on hardware (A100, BH=324 N=128 d=64 fp16) with the
reference harness's protocol and reports the ratio to its median.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "phantom-a100_amd"))

import cuda_attn  # noqa: E402
from cuda_attn import _native  # noqa: E402
from cuda_attn.workloads import CONFIGS, config_inputs  # noqa: E402

METRIC = "attention fwd TFLOP/s + % of MFMA/HBM roofline per config, 1 MI355X"
HEADLINE = "C4"
# MI355X published dense peaks (TFLOP/s) and HBM3E bandwidth (GB/s).
PEAK_TFLOPS = {torch.bfloat16: 2500.0, torch.float16: 2500.0, torch.float32: 157.3}
PEAK_HBM_GBS = 8000.0
DTYPE_NAME = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic_fa_mfma_C4.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def entry_call(cfg, q, k, v, out_dtype=None):
    od = cfg.out_dtype if out_dtype is None else out_dtype
    if cfg.entry == "fused":
        return lambda: cuda_attn.fused(q, k, v, out_dtype=od)
    return lambda: cuda_attn.fused_tc(q, k, v, out_dtype=od)


def gate(cfg, q, k, v, fn) -> float:
    """Max abs error of the config's output (fp32 output) on sampled heads vs float64 on the GPU."""
    out = entry_call(cfg, q, k, v, torch.float32)()
    heads = sorted({0, cfg.BH // 2, cfg.BH - 1})
    qh, kh, vh, oh = (t.reshape(cfg.BH, cfg.N, cfg.d)[heads] for t in (q, k, v, out))
    s = torch.matmul(qh.double(), kh.double().transpose(1, 2).contiguous()) / (cfg.d ** 0.5)
    ref = torch.matmul(torch.softmax(s, dim=-1), vh.double())
    return (oh.double() - ref).abs().max().item()


def time_steps(fn, steps: int, warmup: int):
    """Warm-up, then EXACTLY `steps` back-to-back calls bracketed by synchronisations; events on
    the stream the kernel is launched on (torch's current stream)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_time(e1), wall * 1e3


def settle(fn, seconds: float) -> dict:
    """Back-to-back calls for a fixed wall-clock duration (outside any timed region), so that the
    clock has reached its steady state under this load before warm-up and timing."""
    calls, t0 = 0, time.perf_counter()
    while True:
        for _ in range(8):
            fn()
        calls += 8
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            break
    return {"seconds": round(time.perf_counter() - t0, 3), "calls": calls}


def copy_bandwidth(nbytes: int = 1 << 30, reps: int = 20) -> float:
    """Device copy bandwidth in GB/s (read + write bytes / time) of a torch copy of `nbytes`:
    the practical HBM ceiling beside the 8 TB/s specification."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    gbs = 2 * nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9
    del src, dst
    return gbs


def time_reference_protocol(fn, flush, warmup=10, iters=100):
    """/root/reference/bench/benchmark.py:78-93 with a flush buffer larger than the Infinity Cache."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        flush.zero_()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b))
    times.sort()
    qs = statistics.quantiles(times, n=10)
    return statistics.median(times), qs[0], qs[-1]


def kernel_description(cfg) -> str:
    """The kernel instantiation and launch the library uses for cfg (its own dispatch rule)."""
    if cfg.entry == "fused":
        return f"fa_f32_fwd<{DTYPE_NAME[cfg.dtype]}, D=64, 4 key groups> grid {-(-cfg.N // 32) * cfg.BH} x 256 threads"
    code = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16}
    out = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16, torch.float32: _native.DTYPE_F32}
    return _native.fused_tc_kernel(code[cfg.dtype], out[cfg.out_dtype], cfg.BH, cfg.N, cfg.d, False)


def per_config(flush, iters: int, settle_s: float, copy_gbs: float):
    rows = {}
    for name, cfg in CONFIGS.items():
        q, k, v = config_inputs(cfg, device="cuda")
        fn = entry_call(cfg, q, k, v)
        err = gate(cfg, q, k, v, fn)
        st = settle(fn, settle_s)
        med, p10, p90 = time_reference_protocol(fn, flush, iters=iters)
        tf = cfg.flops() / (med * 1e-3) / 1e12
        gbs = cfg.hbm_bytes() / (med * 1e-3) / 1e9
        rows[name] = {
            "shape": [cfg.B, cfg.H, cfg.N, cfg.d], "dtype": DTYPE_NAME[cfg.dtype], "out_dtype": DTYPE_NAME[cfg.out_dtype],
            "entry": cfg.entry, "kernel": kernel_description(cfg), "settle": st,
            "median_ms": round(med, 5), "p10_ms": round(p10, 5), "p90_ms": round(p90, 5),
            "tflops": round(tf, 3), "pct_mfma_peak": round(100 * tf / PEAK_TFLOPS[cfg.dtype], 3),
            "achieved_GBps": round(gbs, 1), "pct_hbm_bw": round(100 * gbs / PEAK_HBM_GBS, 3),
            "pct_copy_bw": round(100 * gbs / copy_gbs, 3) if copy_gbs else None,
            "max_abs_err_vs_f64": float(f"{err:.3e}"),
        }
        log(f"[per-config] {name}: {med:.4f} ms  {tf:.1f} TFLOP/s  err={err:.2e}")
        del q, k, v
    return rows


def reference_workload():
    """fused_tc at the reference's own measured workload (BH=324, N=128, d=64, fp16) with its
    harness protocol (/root/reference/sim/harness.cu:146-163), beside the A100 median the reference
    published (/root/reference/results/autotune/measured/hw_measurements.json:42-47)."""
    sys.path.insert(0, os.path.join(REPO, "phantom-a100_amd", "bench"))
    import reference_workload as rw
    row = rw.measure(["fused_tc"])[0]
    log(f"[reference workload] fused_tc BH=324 N=128: {row.get('median_ms')} ms vs A100 {row['a100_ms']} ms")
    return {"shape": list(rw.SHAPE), "dtype": "fp16", "entry": "fused_tc", "protocol": "reference harness "
            "(10 warm-ups, 200 launches each between two events, no flush, median)",
            "median_ms": row.get("median_ms"), "tflops": row.get("tflops"), "max_abs_err": row["max_abs_err"],
            "status": row["status"], "a100_median_ms": row["a100_ms"], "speedup_vs_a100": row.get("speedup_vs_a100")}


def host_info() -> dict:
    """Host CPU model, cores visible to this process and the BLAS thread count NumPy uses."""
    model = ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"cpu_model": model, "nproc": cores, "blas_threads": int(threads)}


def _median_time(fn, runs: int):
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), times


def cpu_baseline_config(cfg, target_s: float, runs: int = 3) -> dict:
    """The reference's CPU path on whole heads of cfg: oracle.attention_online (br=64, bc=32,
    P rounded to the config's input dtype; fp32 P for fp32 inputs) over as many heads as fit in
    about `target_s` seconds per run (all heads when they fit), median of `runs` runs, scaled to
    the whole config by heads; beside it the row-chunked float64 reference on the same heads."""
    import numpy as np  # noqa: F401
    import oracle
    q, k, v = (t.reshape(cfg.BH, cfg.N, cfg.d) for t in config_inputs(cfg, device="cpu"))
    p_dtype = {torch.bfloat16: "bfloat16", torch.float16: "float16"}.get(cfg.dtype)

    def sample(h):
        return tuple(t[:h].float().numpy() for t in (q, k, v))

    # size the sample from one head (one untimed call also warms the BLAS threads)
    one = sample(1)
    t0 = time.perf_counter()
    oracle.attention_online(*one, False, br=64, bc=32, p_dtype=p_dtype)
    t1 = time.perf_counter() - t0
    heads = int(max(1, min(cfg.BH, target_s // max(t1, 1e-6))))
    qs, ks, vs = sample(heads)
    med, times = _median_time(lambda: oracle.attention_online(qs, ks, vs, False, br=64, bc=32, p_dtype=p_dtype), runs)
    med64, times64 = _median_time(lambda: oracle.attention_f64_rows(qs, ks, vs, rows=512), runs)
    scale = cfg.BH / heads
    flops = cfg.flops()
    return {
        "heads": heads, "of_heads": cfg.BH, "runs": runs, "p_dtype": p_dtype or "float32",
        "online_s_median": round(med, 4), "online_s_runs": [round(x, 4) for x in times],
        "online_full_config_s": round(med * scale, 3), "online_tflops": round(flops / (med * scale) / 1e12, 6),
        "f64_s_median": round(med64, 4), "f64_full_config_s": round(med64 * scale, 3),
        "f64_tflops": round(flops / (med64 * scale) / 1e12, 6),
    }


def cpu_baseline(headline: str, target_s: float) -> dict:
    """The CPU baseline of every config, reported under the bench contract's `cpu_baseline` key
    with the headline config's attention_online rate as `value`."""
    info = host_info()
    rows = {}
    for name, cfg in CONFIGS.items():
        rows[name] = cpu_baseline_config(cfg, target_s)
        r = rows[name]
        log(f"[cpu] {name}: {r['heads']}/{r['of_heads']} heads, attention_online median {r['online_s_median']} s "
            f"-> {r['online_tflops']} TFLOP/s; float64 rows {r['f64_s_median']} s")
    h = rows[headline]
    return {
        "value": h["online_tflops"], "unit": "TFLOP/s", "cores": info["blas_threads"], "kind": "port",
        "sample": (f"{h['heads']} of {h['of_heads']} heads of {headline} through oracle.attention_online(br=64, "
                   f"bc=32, p_dtype={h['p_dtype']}), median of {h['runs']} runs, scaled to the config by heads; "
                   f"every config under per_config; host {info['cpu_model']}, {info['nproc']} cores, "
                   f"NumPy BLAS threads {info['blas_threads']}"),
        **info, "per_config": rows,
    }


class ClockSampler:
    """Samples the GPU's shader clock (per XCD) and socket power with amdsmi on a background thread
    while the steps run, so that the line's `frac` can be read against the clock the box ran at
    (MI355X runs this load at its power cap; the clock differs from box to box). Inactive (the
    line reports null) where amdsmi does not import or cannot read the device."""

    def __init__(self, period_s: float = 0.005):
        self.period, self.samples, self.error = period_s, [], None
        self._stop, self._thread, self._smi, self._handle = False, None, None, None
        try:
            import amdsmi
            amdsmi.amdsmi_init()
            self._smi, self._handle = amdsmi, amdsmi.amdsmi_get_processor_handles()[0]
            self._smi.amdsmi_get_gpu_metrics_info(self._handle)
        except Exception as e:   # noqa: BLE001 - any failure means no clock in the line
            self._smi, self.error = None, f"{type(e).__name__}: {e}"[:200]

    def _run(self):
        while not self._stop:
            t = time.perf_counter()
            try:
                m = self._smi.amdsmi_get_gpu_metrics_info(self._handle)
                xcd = [int(c) for c in (m.get("current_gfxclks") or []) if isinstance(c, int) and 0 < c < 65535]
                power = m.get("current_socket_power")
                self.samples.append((t, xcd, power if isinstance(power, (int, float)) else None))
            except Exception as e:   # noqa: BLE001
                self.error = f"{type(e).__name__}: {e}"[:200]
            time.sleep(self.period)

    def start(self):
        if self._smi is not None:
            import threading
            self._thread = threading.Thread(target=self._run, daemon=True)
            self._thread.start()
        return self

    def stop(self):
        self._stop = True
        if self._thread is not None:
            self._thread.join()

    def summary(self, t0: float, t1: float):
        """Median per-XCD clock (MHz), their mean and min, and median socket power (W) of the samples
        taken in [t0, t1]; None without samples."""
        win = [s for s in self.samples if t0 <= s[0] <= t1 and s[1]]
        if not win:
            return None
        nx = min(len(s[1]) for s in win)
        per_xcd = [statistics.median(s[1][i] for s in win) for i in range(nx)]
        powers = [s[2] for s in win if s[2] is not None]
        return {"samples": len(win), "per_xcd_mhz": per_xcd, "mean_mhz": round(statistics.mean(per_xcd), 1),
                "min_mhz": min(per_xcd), "socket_power_w": statistics.median(powers) if powers else None}


def traffic_from_profile():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3 PMC summary."""
    try:
        with open(TRAFFIC_FILE) as fh:
            return json.load(fh).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=25)
    ap.add_argument("--settle", type=float, default=2.0,
                    help="seconds of back-to-back calls before warm-up (clock settle; reported, not timed)")
    ap.add_argument("--config", default=HEADLINE, choices=list(CONFIGS))
    ap.add_argument("--iters", type=int, default=100, help="timed calls per config (reference protocol)")
    ap.add_argument("--config-settle", type=float, default=1.0, help="settle seconds before each config's timing")
    ap.add_argument("--cpu-target", type=float, default=3.0, help="seconds per CPU baseline run (heads sampled to fit)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-per-config", action="store_true")
    ap.add_argument("--mode", choices=["bench", "pmc"], default="bench")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        log("bench.py: this build measures one GPU; the attention forward path has no multi-GPU "
            "code (every GPU box here has one GPU). Run with --gpus 1.")
        sys.exit(2)
    if not torch.cuda.is_available():
        log("bench.py: no GPU visible")
        sys.exit(1)
    _native.lib()  # fail loudly if the HIP library is missing

    cfg = CONFIGS[args.config]
    q, k, v = config_inputs(cfg, device="cuda")
    fn = entry_call(cfg, q, k, v)

    if args.mode == "pmc":
        # Known-size copy (calibrates FETCH_SIZE / WRITE_SIZE), then a few launches of the kernel.
        src = torch.ones(256 * 2**20, dtype=torch.float32, device="cuda")   # 1 GiB
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        log(f"pmc workload done: copy {src.numel() * 4} bytes, 3 x {cfg.name}")
        return

    err = gate(cfg, q, k, v, fn)
    tol = 1e-5 if cfg.dtype == torch.float32 else 2e-3
    log(f"[gate] {cfg.name} max abs error vs float64 (sampled heads) = {err:.3e} (tol {tol:.0e})")
    if not err <= tol:
        log("bench.py: correctness gate failed; not timing a wrong result")
        sys.exit(3)

    clock = ClockSampler().start()
    t_settle = time.perf_counter()
    st = settle(fn, args.settle)
    log(f"[settle] {st['calls']} calls in {st['seconds']} s before warm-up")
    t_timed = time.perf_counter()
    ms_total, wall_ms = time_steps(fn, args.steps, args.warmup)
    t_end = time.perf_counter()
    clock.stop()
    clk_timed = clock.summary(t_timed, t_end)
    clk_settle = clock.summary(max(t_settle, t_timed - 1.0), t_timed)
    log(f"[clock] warm-up + timed steps: {clk_timed}; last second of settle: {clk_settle}")
    ms_step = ms_total / args.steps
    flops = cfg.flops()
    value = flops * args.steps / (ms_total * 1e-3) / 1e12
    log(f"[timed] {args.steps} steps: {ms_total:.3f} ms (wall {wall_ms:.3f} ms) -> {value:.1f} TFLOP/s")

    out = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": DTYPE_NAME[cfg.dtype], "data": "synthetic",
        "config": {"workload": f"{cfg.name}: non-causal SDPA forward B={cfg.B} H={cfg.H} N={cfg.N} d={cfg.d} "
                               f"{DTYPE_NAME[cfg.dtype]}, Q/K/V ~ N(0,1) (Q,K x{cfg.qk_scale:g}), seed {cfg.seed}, "
                               f"cuda_attn.{cfg.entry}",
                   "B": cfg.B, "H": cfg.H, "N": cfg.N, "d": cfg.d, "causal": False, "entry": cfg.entry,
                   "out_dtype": DTYPE_NAME[cfg.out_dtype]},
        "settle": dict(st, note="back-to-back calls before the warm-up, outside the timed region"),
        "roofline": {"bound": "mfma", "achieved": round(flops / (ms_step * 1e-3) / 1e12, 3),
                     "peak": PEAK_TFLOPS[cfg.dtype], "unit": "TFLOP/s",
                     "frac": round(flops / (ms_step * 1e-3) / 1e12 / PEAK_TFLOPS[cfg.dtype], 5),
                     "traffic": traffic_from_profile() if cfg.name == HEADLINE else None,
                     "kernel": kernel_description(cfg), "flops_per_launch": flops},
        "gate_max_abs_err": float(f"{err:.3e}"),
        "clock": None if clk_timed is None and clk_settle is None else {
            "source": "amdsmi gpu_metrics current_gfxclks (shader clock per XCD) and current_socket_power, "
                      "sampled every 5 ms on a host thread",
            "warmup_and_timed_steps": clk_timed, "last_second_of_settle": clk_settle},
        "library": _native.version(),
        "device": torch.cuda.get_device_name(0),
    }
    del q, k, v
    torch.cuda.empty_cache()
    if not args.no_per_config:
        copy_gbs = copy_bandwidth()
        out["copy_GBps"] = round(copy_gbs, 1)
        log(f"[copy] device copy {copy_gbs:.0f} GB/s (read + write)")
        flush = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")  # > 256 MB Infinity Cache
        out["per_config"] = per_config(flush, args.iters, args.config_settle, copy_gbs)
        del flush
        out["reference_workload"] = reference_workload()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg.name, args.cpu_target)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
