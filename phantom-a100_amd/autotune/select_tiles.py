"""Tile-shape and occupancy choice for the fused kernels, justified by measured counters.

    python phantom-a100_amd/autotune/select_tiles.py --entry fused_tuned --n 4096
    python phantom-a100_amd/autotune/select_tiles.py --entry fused_tuned --n 4096 --profile --out report.md
    python phantom-a100_amd/autotune/select_tiles.py --entry fused_tc --dtype bf16 --dim 128 --n 4096 --profile

Replaces the reference's simulator-driven loop (/root/reference/autotune/hw_counters.py,
diagnose.py) with measurements on the device. For every compiled candidate of the entry point
(fused_tuned: (br, bc) x {one, two} LDS stages; fused_tc: its shipped tile in both launch forms,
persistent and one workgroup per query block, plus the alternatives of libphantom_attn_tiles.so at
the same dtype and head dim: other query rows per workgroup, keys per tile, LDS stages and
workgroups per CU) the tool
  1. gates the output against a float64 reference (failing candidates are reported, not timed),
  2. times it with the flushing protocol of bench/benchmark.py,
  3. with --profile, runs bench/run_one.py under rocprofv3 (one kernel trace, then one run per
     counter pass of hw_counters.PASSES) and joins the counters with the compiler's resource
     report (kernel_resources.json): MFMA busy, VALU busy, HBM bytes vs compulsory, LDS
     bank-conflict rate, VGPRs, resident waves per SIMD and what limits them, achieved
     occupancy, wait fraction,
  4. applies the rules of diagnose.py to each candidate,
  5. picks the fastest passing candidate and prints a markdown table with every candidate's
     numbers and triggered rules, so the choice and the reasons the others lose can be read.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import tempfile

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG = os.path.dirname(_HERE)
sys.path.insert(0, _PKG)

import torch  # noqa: E402

import cuda_attn  # noqa: E402
from cuda_attn import _checks, _native  # noqa: E402
from cuda_attn.workloads import attention_flops, compulsory_bytes  # noqa: E402

from autotune import diagnose as dg  # noqa: E402
from autotune import hw_counters as hc  # noqa: E402
from autotune import tile_candidates as tc  # noqa: E402

RUN_ONE = os.path.join(_PKG, "bench", "run_one.py")
RESOURCES = os.path.join(_PKG, "cuda_attn", "kernel_resources.json")
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}
MANGLED_T = {torch.float16: "DF16_", torch.bfloat16: "DF16b", torch.float32: "f"}
# fused_tc's general tile per head dim (the launch table in csrc/pa_attn.hip). On small grids the
# library takes another launch (d = 64: a key split; d = 128: 128-query workgroups); the report's
# launch column names it, and its resources are looked up for the tile that launch uses.
TC_TILE = {64: (128, 64, 2), 128: (256, 64, 2)}


SHIPPED, PER_BLOCK = "shipped", "per_block"


def candidates(entry: str, d: int, dtype: torch.dtype | None = None, with_alternatives: bool = True):
    """(label, br, bc, stages, source) of every compiled configuration of `entry` at head dim d.
    source: "tuned" (fused_tuned), SHIPPED (fused_tc as launched), PER_BLOCK (fused_tc's tile with
    the persistent launch switched off), or the index of an alternative in libphantom_attn_tiles.so
    (those of the dtype, when the library is built and with_alternatives is set)."""
    if entry == "fused_tuned":
        return [(f"br{br}_bc{bc}_{'db' if db else 'sb'}", br, bc, 2 if db else 1, "tuned")
                for br, bc in _checks.TUNED_CONFIGS for db in (False, True)]
    br, bc, st = TC_TILE[d]
    out = [(f"br{br}_bc{bc}_{st}stage", br, bc, st, SHIPPED),
           (f"br{br}_bc{bc}_{st}stage_per_block", br, bc, st, PER_BLOCK)]
    if with_alternatives and tc.available():
        out += [(c["label"], c["br"], c["bc"], c["stages"], c["index"]) for c in tc.candidates()
                if c["d"] == d and (dtype is None or c["dtype"] == dtype)]
    return out


def kernel_key(dtype: torch.dtype, d: int, br: int, bc: int, stages: int, out_dtype: torch.dtype,
               ksplit: int = 1, persistent: bool = False, ragged: bool = False, causal: bool = False,
               check: bool = False) -> str:
    """Fragment of the mangled name of
    pa::fa_mfma_fwd<T, D, BM, BN, STAGES, OutT, KSPLIT, PERSIST, RAGGED, CAUSAL, CHECK>."""
    return (f"fa_mfma_fwdI{MANGLED_T[dtype]}Li{d}ELi{br}ELi{bc}ELi{stages}E{MANGLED_T[out_dtype]}"
            f"Li{ksplit}ELb{int(persistent)}ELb{int(ragged)}ELb{int(causal)}ELb{int(check)}EE")


def launch_form(entry: str, dtype: torch.dtype, d: int, n: int, bh: int, causal: bool, br: int,
                source="shipped") -> dict:
    """How the library launches this call: the key split, persistent and ragged flags and the
    number of workgroups, read from the launcher's own description (pa_fused_tc_kernel, or
    pa_tiles_kernel for an alternative), so the report names the kernel that actually runs."""
    if entry != "fused_tc":
        return {"ksplit": 1, "persistent": False, "ragged": False, "causal": False, "check": False,
                "workgroups": -(-n // br) * bh, "description": "", "tile": None}
    if isinstance(source, int):
        desc = tc.kernel(source, bh, n)
    else:
        code = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16}[dtype]
        prev = _native.set_persistent(source != PER_BLOCK)
        try:
            desc = _native.fused_tc_kernel(code, code, bh, n, d, causal)
        finally:
            _native.set_persistent(prev)
    grid = re.search(r"grid (\d+) x", desc)
    # fp16 two-stage tiles on non-causal rows use the packed-max check in fused_tc's persistent
    # forms, at d = 128 per block, and in every alternative; both launchers name it
    check = ", packed-max check" in desc
    tile = re.search(r"BM=(\d+), BN=(\d+), (\d) stages", desc)
    return {"ksplit": 2 if "key split 2" in desc else 1, "persistent": ", persistent" in desc,
            "ragged": ", ragged" in desc, "causal": ", persistent, causal" in desc, "check": check,
            "workgroups": int(grid.group(1)) if grid else -(-n // br) * bh, "description": desc,
            # the tile the launch uses (fused_tc takes a smaller one on small grids)
            "tile": tuple(int(x) for x in tile.groups()) if tile else None}


def load_resources(path: str = RESOURCES) -> dict:
    if not os.path.exists(path):
        return {}
    with open(path) as fh:
        return json.load(fh)


def find_resources(res: dict, key: str) -> dict | None:
    for name, v in res.items():
        if key in name:
            return dict(v, kernel=name)
    return None


def make_call(entry, q, k, v, causal, br, bc, stages, out_dtype=None, source=SHIPPED):
    if entry == "fused_tuned":
        return lambda: cuda_attn.fused_tuned(q, k, v, causal, stages == 2, br, bc, out_dtype=out_dtype)
    if isinstance(source, int):   # an alternative: output in the input dtype only
        return lambda: tc.forward(source, q, k, v, causal)
    if source == PER_BLOCK:
        def per_block():
            prev = _native.set_persistent(False)
            try:
                return cuda_attn.fused_tc(q, k, v, causal, out_dtype=out_dtype)
            finally:
                _native.set_persistent(prev)
        return per_block
    return lambda: cuda_attn.fused_tc(q, k, v, causal, out_dtype=out_dtype)


def float64_error(q, k, v, out, causal) -> tuple[float, float]:
    """Max abs error against float64 on the first and last head, and half an ulp of the output
    dtype at the largest reference value (the output's own rounding, 0 for fp32 outputs)."""
    b, h, n, d = q.shape
    heads = sorted({0, b * h - 1})
    qh, kh, vh, oh = (t.reshape(b * h, n, d)[heads].double() for t in (q, k, v, out.float()))
    s = torch.matmul(qh, kh.transpose(1, 2).contiguous()) / d ** 0.5
    if causal:
        s = s.masked_fill(torch.ones(n, n, dtype=torch.bool, device=s.device).triu(1), float("-inf"))
    ref = torch.matmul(torch.softmax(s, -1), vh)
    rounding = 0.0 if out.dtype == torch.float32 else 0.5 * torch.finfo(out.dtype).eps * ref.abs().max().item()
    return (oh - ref).abs().max().item(), rounding


def profile_candidate(args, br, bc, stages, out_dir, source="tuned", label="") -> dict:
    """Kernel trace + counter passes of one candidate; returns the aggregated quantities."""
    cmd = [sys.executable, RUN_ONE, "--impl", args.entry, "--n", str(args.n), "--batch", str(args.batch),
           "--heads", str(args.heads), "--dim", str(args.dim), "--dtype", args.dtype, "--reps", "3",
           "--br", str(br), "--bc", str(bc), "--db", str(1 if stages == 2 else 0), "--calibrate"]
    if isinstance(source, int):
        cmd += ["--candidate", label]
    elif source == PER_BLOCK:
        cmd.append("--per-block")
    if args.causal:
        cmd.append("--causal")
    tr = hc.run_pass(cmd, None, out_dir, "trace", timeout=args.pass_timeout)
    if tr["status"] != "ok":
        return {"profile_status": tr["status"]}
    trace = [r for r in hc.parse_kernel_trace(tr["files"][0]) if "fa_mfma_fwd" in r["kernel"]]
    parsed = []
    for i, counters in enumerate(hc.PASSES):
        p = hc.run_pass(cmd, counters, out_dir, f"pmc{i}", timeout=args.pass_timeout)
        if p["status"] != "ok":
            return {"profile_status": f"pass {i}: {p['status']}"}
        parsed.append(hc.parse_counter_csv(p["files"][0]))
    dispatches, calib = hc.merge_passes(parsed, "fa_mfma_fwd")
    if not trace or not dispatches:
        return {"profile_status": "kernel not found in the profile"}
    dispatches["duration_ns"] = trace[-1]["duration_ns"]
    for kk in ("grid", "workgroup", "lds"):
        dispatches[kk] = trace[-1][kk]
    res = find_resources(load_resources(), dispatches["kernel"].split("(")[0])
    agg = hc.aggregate([dispatches], res, fetch_calibration=calib)
    agg["fetch_calibration"] = calib
    agg["profile_status"] = "ok"
    return agg


def evaluate(args) -> list[dict]:
    dt = DTYPES[args.dtype]
    gen = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(args.batch, args.heads, args.n, args.dim, generator=gen).to(dt).cuda() for _ in range(3))
    flush = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    sys.path.insert(0, os.path.join(_PKG, "bench"))
    from benchmark import time_calls  # noqa: E402
    res_all = load_resources()
    flops = attention_flops(args.batch, args.heads, args.n, args.dim, args.causal)
    comp = compulsory_bytes(args.batch * args.heads, args.n, args.dim, dt, dt)
    rows = []
    only = set(args.only.split(",")) if args.only else None
    bh = args.batch * args.heads
    # An alternative whose launch is the shipped one is skipped where the shipped row is evaluated too.
    shipped = ""
    if args.entry == "fused_tc":
        sbr, sbc, sst = TC_TILE[args.dim]
        if only is None or f"br{sbr}_bc{sbc}_{sst}stage" in only:
            shipped = launch_form(args.entry, dt, args.dim, args.n, bh, args.causal, sbr, SHIPPED)["description"]
    for label, br, bc, st, source in candidates(args.entry, args.dim, dt, with_alternatives=not args.shipped_only):
        if only is not None and label not in only:
            continue
        form = launch_form(args.entry, dt, args.dim, args.n, bh, args.causal, br, source)
        if source in (SHIPPED, PER_BLOCK) and form.get("tile") and form["tile"] != (br, bc, st):
            # fused_tc launches another tile on this grid: the row names the tile that runs
            tb, tn, ts = form["tile"]
            label = f"br{tb}_bc{tn}_{ts}stage{'_per_block' if source == PER_BLOCK else ''} (as launched)"
        row = {"candidate": label, "br": br, "bc": bc, "stages": st}
        if isinstance(source, int) and shipped and form["description"] == shipped:
            rows.append(dict(row, status="skipped: the shipped launch"))
            continue
        fn = make_call(args.entry, q, k, v, args.causal, br, bc, st, source=source)
        try:   # gate on fp32 output where the candidate has one, so the 2e-3 bar does not include
            # the output's own rounding; the alternatives (input-dtype output) get that rounding on top
            out = make_call(args.entry, q, k, v, args.causal, br, bc, st,
                            None if isinstance(source, int) else torch.float32, source)()
            err, rounding = float64_error(q, k, v, out, args.causal)
        except RuntimeError as e:
            rows.append(dict(row, status="skipped: " + str(e).splitlines()[0][:80]))
            continue
        row["max_abs_err"] = err
        if not err <= 2e-3 + rounding:
            rows.append(dict(row, status="wrong_result"))
            continue
        med, p10, p90 = time_calls(fn, 5, args.iters, flush)
        row.update(status="ok", median_ms=med, p10_ms=p10, p90_ms=p90, tflops=flops / (med * 1e-3) / 1e12)
        kbr, kbc, kst = form.get("tile") or (br, bc, st)
        res = find_resources(res_all, kernel_key(dt, args.dim, kbr, kbc, kst, dt, form["ksplit"], form["persistent"],
                                                 form["ragged"], form["causal"], form["check"]))
        row["launch"] = form["description"]
        threads = kbr // 32 * 64 * form["ksplit"]   # one wave per 32 query rows per key group
        if res:
            waves, lim = hc.theoretical_waves_per_simd(res["vgprs"], res["agprs"], res["lds_bytes"], threads)
            row.update(regs=res["vgprs"] + res["agprs"], waves_per_simd_limit=waves, occupancy_limiter=lim,
                       spill=res["vgpr_spill"] + res["sgpr_spill"] + res["scratch_bytes"])
            row["resident_wgs_per_cu"] = dg.resident_wgs_per_cu(waves, threads)
        row["workgroups"] = form["workgroups"]
        if args.profile and args.profile_dir:      # keep the raw rocprofv3 output per candidate
            prof = profile_candidate(args, br, bc, st, os.path.join(args.profile_dir, label.split()[0]), source, label)
        elif args.profile:
            with tempfile.TemporaryDirectory() as tmp:
                prof = profile_candidate(args, br, bc, st, tmp, source, label)
        if args.profile:
            for kk, vv in prof.items():
                if vv is not None:
                    row[kk] = vv
        row["bottlenecks"] = [str(b) for b in dg.diagnose(row, comp)]
        rows.append(row)
    return rows


def choose(rows: list[dict]) -> dict | None:
    ok = [r for r in rows if r.get("status") == "ok"]
    return min(ok, key=lambda r: r["median_ms"]) if ok else None


def _fmt(v, spec):
    return "" if v is None else format(v, spec)


def report(args, rows, best) -> str:
    comp = compulsory_bytes(args.batch * args.heads, args.n, args.dim, DTYPES[args.dtype], DTYPES[args.dtype])
    lines = [f"# Tile choice: {args.entry}, B={args.batch} H={args.heads} N={args.n} d={args.dim} {args.dtype}"
             f"{' causal' if args.causal else ''}", "",
             "| candidate | status | ms | TFLOP/s | MFMA busy % | VALU busy % | HBM / compulsory | LDS conflict % "
             "| VGPRs | waves/SIMD (limit) | occupancy % | wait % | rules triggered |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        hbm = r.get("hbm_bytes")
        conf = (100 * r["lds_bank_conflict_cycles"] / r["lds_active_cycles"]
                if r.get("lds_bank_conflict_cycles") is not None and r.get("lds_active_cycles") else None)
        lines.append(
            f"| {r['candidate']} | {r.get('status')} | {_fmt(r.get('median_ms'), '.4f')} | {_fmt(r.get('tflops'), '.1f')} "
            f"| {_fmt(r.get('mfma_util'), '.1f')} | {_fmt(r.get('valu_busy'), '.1f')} "
            f"| {_fmt(hbm / comp if hbm is not None else None, '.2f')} | {_fmt(conf, '.2f')} | {r.get('regs', '')} "
            f"| {r.get('waves_per_simd_limit', '')} ({r.get('occupancy_limiter', '')}) | {_fmt(r.get('occupancy'), '.1f')} "
            f"| {_fmt(100 * r['wait_frac'] if r.get('wait_frac') is not None else None, '.0f')} "
            f"| {'; '.join(b.split(' (')[0] for b in r.get('bottlenecks', [])) or '-'} |")
    lines.append("")
    for r in rows:
        if r.get("launch"):
            lines.append(f"Launch of {r['candidate']}: `{r['launch']}`.")
    lines.append("")
    if best:
        lines.append(f"**Chosen: {best['candidate']}** ({best['median_ms']:.4f} ms, {best['tflops']:.1f} TFLOP/s).")
        for r in rows:
            if r is best or r.get("status") != "ok":
                continue
            why = "; ".join(r.get("bottlenecks", [])) or "no rule triggered; slower by measurement"
            lines.append(f"- {r['candidate']}: {r['median_ms'] / best['median_ms']:.2f}x the time. {why}")
    else:
        lines.append("No candidate passed.")
    return "\n".join(lines) + "\n"


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--entry", choices=["fused_tuned", "fused_tc"], default="fused_tuned")
    p.add_argument("--n", type=int, default=4096)
    p.add_argument("--batch", type=int, default=4)
    p.add_argument("--heads", type=int, default=16)
    p.add_argument("--dim", type=int, default=64)
    p.add_argument("--dtype", choices=list(DTYPES), default="fp16")
    p.add_argument("--causal", action="store_true")
    p.add_argument("--iters", type=int, default=30)
    p.add_argument("--profile", action="store_true", help="collect rocprofv3 counters for every candidate")
    p.add_argument("--profile-dir", default=None, help="keep the raw rocprofv3 output here (default: a temporary directory)")
    p.add_argument("--pass-timeout", type=int, default=120)
    p.add_argument("--shipped-only", action="store_true",
                   help="fused_tc: only the shipped tile (both launch forms), not the alternatives")
    p.add_argument("--only", default="", help="comma-separated candidate labels to evaluate (default: all)")
    p.add_argument("--out", default=None, help="write the markdown report here (and <out>.json)")
    a = p.parse_args(argv)
    if a.entry == "fused_tuned" and (a.dim != 64 or a.dtype != "fp16"):
        p.error("fused_tuned is compiled for fp16, d = 64")
    return a


def main(argv=None):
    args = parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("select_tiles.py needs a GPU")
    rows = evaluate(args)
    best = choose(rows)
    text = report(args, rows, best)
    print(text, flush=True)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text)
        with open(args.out + ".json", "w") as fh:
            json.dump({"args": vars(args), "rows": rows, "chosen": best and best["candidate"]}, fh, indent=1)
    return best


if __name__ == "__main__":
    main()
