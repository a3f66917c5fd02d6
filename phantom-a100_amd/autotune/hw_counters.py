"""Hardware counters on MI355X (gfx950) through rocprofv3, and the mapping from the counters the
reference's optimizer reasons about to the ones measured here.

The reference maps GPGPU-Sim counters to Nsight Compute metrics (/root/reference/autotune/
hw_counters.py:33-76). Here the measured side is rocprofv3 on gfx950 and the static side is the
compiler's resource report (kernel_resources.json, written by build_native.py). MAPPING states,
for every quantity the tile choice uses, where it comes from and how close it is to the
reference's notion:

  same_definition   the same quantity (registers per lane, workgroups, kernel time)
  approximate       same intent, different accounting (HBM bytes from TCC request counts)
  proxy             a related quantity (wait cycles per wave cycle for "scoreboard stalls")

A counter rocprofv3 could not collect is None (unobservable), never a zero.

rocprofv3 does not split counters over passes, and one pass may hold at most 8 SQ_, 4 TCC_
(FETCH_SIZE alone takes 3, WRITE_SIZE 2), 4 TCP_, 2 TA_, 2 TD_ and 2 GRBM_ counters; PASSES
respects that and check_pass() enforces it before anything runs.
"""
from __future__ import annotations

import csv
import glob
import os
import shutil
import subprocess
from collections import OrderedDict

# gfx950 (MI355X) machine constants used to turn counters into rates.
CUS = 256
XCDS = 8                            # GRBM_GUI_ACTIVE arrives summed over the 8 XCDs
SIMDS_PER_CU = 4
MAX_WAVES_PER_SIMD = 8
VGPRS_PER_SIMD_LANE = 512           # unified arch + accumulation VGPR file per lane
VGPR_GRANULE = 8
LDS_BYTES_PER_CU = 160 * 1024
WAVE = 64

MAPPING = OrderedDict([
    ("cycles", dict(source="kernel-trace", counters=[], equivalence="same_definition",
                    label="Kernel time", note="End - Start of the dispatch (--kernel-trace)")),
    ("regs", dict(source="static", counters=[], equivalence="same_definition", label="VGPRs + AGPRs per lane",
                  note="compiler resource report (-Rpass-analysis=kernel-resource-usage)")),
    ("occupancy", dict(source="pmc", counters=["SQ_WAVE_CYCLES", "GRBM_GUI_ACTIVE"], equivalence="same_definition",
                       label="Achieved occupancy",
                       note="rocprofv3 OccupancyPercent: 400 * SQ_WAVE_CYCLES / GRBM_GUI_ACTIVE(per XCD) / CUs / 32")),
    ("waves_per_simd_limit", dict(source="static", counters=[], equivalence="same_definition",
                                  label="Resident waves per SIMD",
                                  note="min of the VGPR, LDS and wave-slot limits (theoretical occupancy)")),
    ("workgroups", dict(source="kernel-trace", counters=[], equivalence="same_definition",
                        label="Workgroups (grid size)", note="Grid_Size / Workgroup_Size")),
    ("kernel_launches", dict(source="kernel-trace", counters=[], equivalence="same_definition",
                             label="Kernel launches", note="dispatches per forward call")),
    ("hbm_bytes", dict(source="pmc", counters=["FETCH_SIZE", "WRITE_SIZE"], equivalence="approximate",
                       label="HBM traffic",
                       note="TCC->EA request bytes; FETCH_SIZE scaled by a copy-kernel calibration")),
    ("mfma_util", dict(source="pmc", counters=["SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"],
                       equivalence="same_definition", label="MFMA busy",
                       note="rocprofv3 MfmaUtil (no reference counterpart: tensor-core busy)")),
    ("valu_busy", dict(source="pmc", counters=["SQ_ACTIVE_INST_VALU", "GRBM_GUI_ACTIVE"], equivalence="proxy",
                       label="VALU busy (issue utilisation)", note="rocprofv3 VALUBusy")),
    ("lds_insn", dict(source="pmc", counters=["SQ_INSTS_LDS"], equivalence="approximate",
                      label="LDS instructions", note="shared-memory instructions, wave level")),
    ("lds_bank_conflict_cycles", dict(source="pmc", counters=["SQ_LDS_BANK_CONFLICT"], equivalence="same_definition",
                                      label="LDS bank-conflict cycles", note="per-SE sum")),
    ("lds_active_cycles", dict(source="pmc", counters=["SQ_LDS_IDX_ACTIVE"], equivalence="same_definition",
                               label="LDS active cycles", note="denominator of the conflict rate")),
    ("valu_insn", dict(source="pmc", counters=["SQ_INSTS_VALU"], equivalence="approximate",
                       label="VALU instructions", note="wave-level, includes MFMA")),
    ("mfma_insn", dict(source="pmc", counters=["SQ_INSTS_MFMA"], equivalence="same_definition",
                       label="MFMA instructions", note="wave-level")),
    ("wait_frac", dict(source="pmc", counters=["SQ_WAIT_INST_ANY", "SQ_WAVE_CYCLES"], equivalence="proxy",
                       label="Waiting for an issue dependency",
                       note="SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES (both quad-cycles); reference: scoreboard stalls")),
])

# One rocprofv3 --pmc run per entry; every entry fits the per-block limits.
PASSES = [
    ["FETCH_SIZE"],
    ["WRITE_SIZE"],
    ["SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU",
     "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "GRBM_GUI_ACTIVE"],
    ["SQ_ACTIVE_INST_VALU", "SQ_WAIT_INST_ANY", "SQ_LDS_IDX_ACTIVE", "SQ_INSTS_SALU", "GRBM_GUI_ACTIVE"],
]
# Hardware blocks that one pass can sample, and how many counters of each (FETCH_SIZE and
# WRITE_SIZE are derived from 3 and 2 TCC counters).
BLOCK_LIMITS = {"SQ": 8, "TCC": 4, "TCP": 4, "TA": 2, "TD": 2, "GRBM": 2}
DERIVED_COST = {"FETCH_SIZE": ("TCC", 3), "WRITE_SIZE": ("TCC", 2)}


def counter_block(name: str) -> tuple[str, int]:
    if name in DERIVED_COST:
        return DERIVED_COST[name]
    return name.split("_", 1)[0], 1


def check_pass(counters: list[str]) -> None:
    """Raise ValueError if one rocprofv3 pass would ask a block for more counters than it has
    (rocprofv3 then reports error 38 and hangs instead of exiting)."""
    used: dict[str, int] = {}
    for c in dict.fromkeys(counters):
        block, n = counter_block(c)
        used[block] = used.get(block, 0) + n
    for block, n in used.items():
        if n > BLOCK_LIMITS.get(block, 0):
            raise ValueError(f"pass {counters} needs {n} {block} counters; at most {BLOCK_LIMITS.get(block, 0)}")


def rocprof_path() -> str | None:
    return shutil.which("rocprofv3")


def _num(v):
    v = (v or "").strip()
    if v in ("", "n/a", "N/A", "nan"):
        return None
    try:
        return float(v)
    except ValueError:
        return None


def parse_counter_csv(path: str) -> "OrderedDict[int, dict]":
    """rocprofv3 *_counter_collection.csv -> {dispatch id: {kernel, duration_ns, grid, workgroup,
    lds, vgpr, <counter>: value}} (one row per dispatch and counter in the file)."""
    out: "OrderedDict[int, dict]" = OrderedDict()
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            did = int(r["Dispatch_Id"])
            d = out.setdefault(did, {"kernel": r.get("Kernel_Name", "")})
            if "Start_Timestamp" in r and "End_Timestamp" in r and r["End_Timestamp"]:
                d["duration_ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            for src, key in (("Grid_Size", "grid"), ("Workgroup_Size", "workgroup"), ("LDS_Block_Size", "lds"),
                             ("VGPR_Count", "vgpr_field"), ("Accum_VGPR_Count", "agpr_field")):
                if r.get(src):
                    d[key] = int(float(r[src]))
            d[r["Counter_Name"]] = _num(r["Counter_Value"])
    return out


def merge_passes(passes: list, kernel: str, copy_bytes: int = 1 << 30) -> tuple[dict | None, float]:
    """Merge the per-pass counter files of one profiled program: the counters of the LAST dispatch
    whose name contains `kernel` (a steady-state call) from every pass, and the FETCH_SIZE
    calibration from the program's copy of `copy_bytes` (rocclr copyBuffer), 1.0 if absent.
    `passes`: parse_counter_csv() results, one per pass."""
    merged: dict = {}
    calib = 1.0
    for rows in passes:
        copies = [r for r in rows.values() if "copyBuffer" in r["kernel"]]
        if copies and copies[-1].get("FETCH_SIZE"):
            calib = copy_bytes / (copies[-1]["FETCH_SIZE"] * 1024)
        mine = [r for r in rows.values() if kernel in r["kernel"]]
        if mine:
            for k, v in mine[-1].items():
                merged.setdefault(k, v)
    return (merged or None), calib


def parse_kernel_trace(path: str) -> list[dict]:
    """rocprofv3 *_kernel_trace.csv -> [{kernel, duration_ns, grid, workgroup, lds}] in launch order."""
    rows = []
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            rows.append({"kernel": r["Kernel_Name"],
                         "duration_ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"]),
                         "grid": int(r["Grid_Size_X"]) * int(r.get("Grid_Size_Y") or 1) * int(r.get("Grid_Size_Z") or 1),
                         "workgroup": int(r["Workgroup_Size_X"]) * int(r.get("Workgroup_Size_Y") or 1)
                         * int(r.get("Workgroup_Size_Z") or 1),
                         "lds": int(r["LDS_Block_Size"])})
    return rows


def run_pass(cmd: list[str], counters: list[str] | None, out_dir: str, name: str, timeout: int = 120) -> dict:
    """One rocprofv3 run of `cmd` (a program and its arguments, run as the profiler's direct
    child): --pmc `counters`, or --kernel-trace when counters is None. Returns {'status', 'files'}."""
    prof = rocprof_path()
    if not prof:
        return {"status": "no_rocprof", "files": []}
    if counters is not None:
        check_pass(counters)
        args = [prof, "--pmc", *counters]
    else:
        args = [prof, "--kernel-trace", "--stats"]
    args += ["--output-format", "csv", "-d", os.path.join(out_dir, name), "-o", name, "--", *cmd]
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    try:
        p = subprocess.run(args, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=timeout, env=env)
    except subprocess.TimeoutExpired:
        return {"status": "timeout", "files": []}
    pattern = "*_counter_collection.csv" if counters is not None else "*_kernel_trace.csv"
    files = sorted(glob.glob(os.path.join(out_dir, name, "**", pattern), recursive=True))
    # rocprofv3 may exit with a signal after the program finished and wrote complete results.
    status = "ok" if files else ("error" if p.returncode else "empty")
    return {"status": status, "files": files, "log": p.stdout[-2000:] if status != "ok" else ""}


def theoretical_waves_per_simd(vgprs: int, agprs: int, lds_bytes: int, threads: int) -> tuple[int, str]:
    """Resident waves per SIMD for a kernel and what limits it ('vgpr', 'lds', 'waves')."""
    waves_per_wg = max(1, threads // WAVE)
    regs = -(-(vgprs + agprs) // VGPR_GRANULE) * VGPR_GRANULE
    by_vgpr = VGPRS_PER_SIMD_LANE // max(regs, VGPR_GRANULE)    # the wave-slot cap is its own limit
    wg_by_vgpr = (by_vgpr * SIMDS_PER_CU) // waves_per_wg
    wg_by_lds = LDS_BYTES_PER_CU // lds_bytes if lds_bytes else 10**9
    wg_by_waves = (MAX_WAVES_PER_SIMD * SIMDS_PER_CU) // waves_per_wg
    limits = {"vgpr": wg_by_vgpr, "lds": wg_by_lds, "waves": wg_by_waves}
    limiter = min(limits, key=limits.get)
    wgs = limits[limiter]
    return min(MAX_WAVES_PER_SIMD, (wgs * waves_per_wg) // SIMDS_PER_CU), limiter


def aggregate(dispatches: list[dict], resources: dict | None = None, fetch_calibration: float = 1.0) -> dict:
    """Combine the counters of the dispatches of one forward call into the MAPPING quantities
    (None where a counter is missing). `resources`: the compiler report entry of the dominant
    kernel."""
    def tot(key):
        vals = [d.get(key) for d in dispatches]
        return None if not vals or any(v is None for v in vals) else sum(vals)

    if not dispatches:
        return {k: None for k in MAPPING}
    dom = max(dispatches, key=lambda d: d.get("duration_ns") or 0)
    out = {"cycles": tot("duration_ns"), "kernel_launches": len(dispatches),
           "workgroups": (dom["grid"] // dom["workgroup"]) if dom.get("grid") and dom.get("workgroup") else None}
    grbm = dom.get("GRBM_GUI_ACTIVE")
    grbm = grbm / XCDS if grbm else None      # cycles of one XCD = kernel cycles
    wave_cycles = tot("SQ_WAVE_CYCLES")
    out["occupancy"] = (400.0 * wave_cycles / grbm / CUS / 32) if wave_cycles is not None and grbm else None
    busy = tot("SQ_VALU_MFMA_BUSY_CYCLES")
    out["mfma_util"] = (100.0 * busy / (grbm * CUS * SIMDS_PER_CU)) if busy is not None and grbm else None
    valu = tot("SQ_ACTIVE_INST_VALU")
    out["valu_busy"] = (100.0 * valu / CUS / grbm) if valu is not None and grbm else None
    fetch, write = tot("FETCH_SIZE"), tot("WRITE_SIZE")
    out["hbm_bytes"] = (fetch * 1024 * fetch_calibration + write * 1024) if fetch is not None and write is not None else None
    for key, ctr in (("lds_insn", "SQ_INSTS_LDS"), ("lds_bank_conflict_cycles", "SQ_LDS_BANK_CONFLICT"),
                     ("lds_active_cycles", "SQ_LDS_IDX_ACTIVE"), ("valu_insn", "SQ_INSTS_VALU"),
                     ("mfma_insn", "SQ_INSTS_MFMA")):
        out[key] = tot(ctr)
    wait = tot("SQ_WAIT_INST_ANY")
    out["wait_frac"] = (wait / wave_cycles) if wait is not None and wave_cycles else None   # both in quad-cycles
    if resources:
        out["regs"] = resources.get("vgprs", 0) + resources.get("agprs", 0)
        out["spill"] = resources.get("vgpr_spill", 0) + resources.get("sgpr_spill", 0) + resources.get("scratch_bytes", 0)
        waves, limiter = theoretical_waves_per_simd(resources.get("vgprs", 0), resources.get("agprs", 0),
                                                    dom.get("lds") or resources.get("lds_bytes", 0), dom.get("workgroup") or 256)
        out["waves_per_simd_limit"] = waves
        out["occupancy_limiter"] = limiter
    else:
        out["regs"] = out["spill"] = out["waves_per_simd_limit"] = out["occupancy_limiter"] = None
    return out
