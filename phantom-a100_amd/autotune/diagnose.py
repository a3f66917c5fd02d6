"""Counter rules for one measured kernel: what keeps it from its MFMA roofline on gfx950.

Every rule reads the measurements of one design point (the quantities of hw_counters.aggregate(),
the compiler's resource report and the launch shape, as one dict) and, when its condition holds,
returns a Finding: the rule, a score (the measured value over the rule's threshold, so at least 1
when it fires; findings are ranked by it) and the numbers that made it fire. A rule whose inputs
were not measured (None or absent) stays silent. Named, printable rules rather than a fitted model
follow the reference's classifier (/root/reference/autotune/diagnose.py:17-77); the rules are
CDNA4's: MFMA and VALU busy instead of tensor-core and CUDA-core math, LDS bank conflicts in
cycles, occupancy in waves per SIMD (8 at most, a 512-entry VGPR file per lane, 160 KB of LDS per
CU), and parallelism counted in workgroups against 256 CUs.
"""
from __future__ import annotations

from typing import Callable, NamedTuple, Optional, Tuple

from .hw_counters import CUS, MAX_WAVES_PER_SIMD


class Finding(NamedTuple):
    rule: str
    score: float    # measured / threshold; >= 1 when the rule fires
    detail: str

    def __str__(self) -> str:
        return f"{self.rule} (score {self.score:.2f}): {self.detail}"


Verdict = Optional[Tuple[float, str]]
_RULES: dict[str, Tuple[str, Callable[["_Point"], Verdict]]] = {}


def _rule(name: str, condition: str):
    """Register a rule under `name`; `condition` is its threshold in words (THRESHOLDS)."""
    def register(fn: Callable[["_Point"], Verdict]):
        _RULES[name] = (condition, fn)
        return fn
    return register


class _Point:
    """The measured quantities of one design point, with the derived ones the rules share."""

    def __init__(self, m: dict, compulsory_bytes: float | None):
        self.m = m
        hbm = m.get("hbm_bytes")
        self.traffic = hbm / compulsory_bytes if hbm is not None and compulsory_bytes else None
        self.launches = m.get("kernel_launches") or 1

    def __getattr__(self, key):   # a counter, None when it was not measured
        return self.m.get(key)


@_rule("materialized_intermediate", "more than one kernel launch AND HBM traffic > 4x compulsory")
def _materialized(p: _Point) -> Verdict:
    if p.traffic is not None and p.launches > 1 and p.traffic > 4:
        return p.traffic / 4, f"{p.launches} launches, HBM traffic {p.traffic:.1f}x compulsory"
    return None


@_rule("redundant_hbm_traffic", "HBM traffic > 3x compulsory (Q, K, V read once, O written once)")
def _redundant(p: _Point) -> Verdict:
    if p.traffic is not None and p.traffic > 3:
        return p.traffic / 3, f"HBM traffic {p.traffic:.1f}x compulsory"
    return None


def _occupancy_rule(limiter: str):
    def check(p: _Point) -> Verdict:
        w = p.waves_per_simd_limit
        if w is None or w >= 2 or (p.occupancy_limiter or "") != limiter:
            return None
        why = f"{p.regs} VGPRs per lane" if limiter == "vgpr" else "LDS"
        return 2 / max(w, 0.5), f"{w} wave(s) per SIMD, limited by {why}"
    return check


_rule("vgpr_limited_occupancy", "resident waves limited by VGPRs AND < 2 waves per SIMD")(_occupancy_rule("vgpr"))
_rule("lds_limited_occupancy", "resident waves limited by LDS AND < 2 waves per SIMD")(_occupancy_rule("lds"))


@_rule("scalar_math_bound", "no MFMA instructions AND VALU busy > 50% (matmuls run as scalar FMAs)")
def _scalar(p: _Point) -> Verdict:
    if p.mfma_insn == 0 and p.valu_busy is not None and p.valu_busy > 50:
        return p.valu_busy / 50, f"no MFMA instructions, VALU busy {p.valu_busy:.0f}%"
    return None


@_rule("valu_bound_softmax",
       "MFMA busy < 60% AND VALU busy > MFMA busy (exp/max/sum/rescale crowd the matrix cores)")
def _valu(p: _Point) -> Verdict:
    mf, va = p.mfma_util, p.valu_busy
    if mf is None or va is None or not p.mfma_insn or mf >= 60 or va <= mf:
        return None
    return 60 / max(mf, 1.0), f"MFMA busy {mf:.0f}% with VALU busy {va:.0f}%"


@_rule("lds_bank_conflicts", "> 5% of LDS active cycles stalled on bank conflicts")
def _lds(p: _Point) -> Verdict:
    if p.lds_bank_conflict_cycles is None or not p.lds_active_cycles:
        return None
    share = p.lds_bank_conflict_cycles / p.lds_active_cycles
    return (share / 0.05, f"{100 * share:.1f}% of LDS cycles in bank conflicts") if share > 0.05 else None


@_rule("latency_bound", "> 50% of wave cycles waiting for an issue dependency AND occupancy < 30%")
def _latency(p: _Point) -> Verdict:
    wf, occ = p.wait_frac, p.occupancy
    if wf is None or occ is None or wf <= 0.5 or occ >= 30:
        return None
    return wf / 0.5, f"{100 * wf:.0f}% of wave cycles waiting, occupancy {occ:.0f}%"


@_rule("low_parallelism", "< 0.75 waves of workgroups over the 256 CUs (CUs left idle)")
def _parallelism(p: _Point) -> Verdict:
    if not p.workgroups or not p.resident_wgs_per_cu:
        return None
    rounds = p.workgroups / (CUS * p.resident_wgs_per_cu)
    if rounds >= 0.75:
        return None
    return (0.75 / max(rounds, 1e-3),
            f"{p.workgroups} workgroups for {CUS} CUs x {p.resident_wgs_per_cu} resident = {rounds:.2f} waves")


@_rule("register_spills", "the compiler reports VGPR/SGPR spills or scratch for the kernel")
def _spills(p: _Point) -> Verdict:
    return (1.0 + p.spill / 64, f"{p.spill} spill/scratch units reported by the compiler") if p.spill else None


THRESHOLDS = {name: condition for name, (condition, _) in _RULES.items()}


def diagnose(measured: dict, compulsory_bytes: float | None = None) -> list[Finding]:
    """The rules that fire for one design point, highest score first. `measured` holds
    hw_counters.aggregate() quantities plus the optional launch-shape keys (workgroups,
    resident_wgs_per_cu, kernel_launches) and the compiler's (regs, spill)."""
    point = _Point(measured, compulsory_bytes)
    found = []
    for name, (_, check) in _RULES.items():
        verdict = check(point)
        if verdict is not None:
            found.append(Finding(name, *verdict))
    return sorted(found, key=lambda f: f.score, reverse=True)


def resident_wgs_per_cu(waves_per_simd: int, threads: int) -> int:
    """Workgroups resident per CU at `waves_per_simd` (a workgroup's waves spread over 4 SIMDs)."""
    waves_per_wg = max(1, threads // 64)
    return max(1, (min(waves_per_simd, MAX_WAVES_PER_SIMD) * 4) // waves_per_wg)
