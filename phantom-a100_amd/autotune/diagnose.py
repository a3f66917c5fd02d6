"""Bottleneck rules over measured gfx950 counters: explicit, printable, no fitted model.

Same idea as the reference's classifier (/root/reference/autotune/diagnose.py:17-77): each rule
returns a Bottleneck with a severity (how far past its threshold the measurement is; >= 1 means
triggered) and the evidence that triggered it. The rules are re-derived for CDNA4: MFMA busy and
VALU busy replace the "CUDA-core math" rule, LDS bank conflicts are counted in cycles, occupancy
is waves per SIMD out of 8 with a 512-entry VGPR file per lane and 160 KB of LDS per CU, and
"low parallelism" counts workgroups against 256 CUs.
"""
from __future__ import annotations

from dataclasses import dataclass

from .hw_counters import CUS, MAX_WAVES_PER_SIMD

THRESHOLDS = {
    "materialized_intermediate": "more than one kernel launch AND HBM traffic > 4x compulsory",
    "redundant_hbm_traffic": "HBM traffic > 3x compulsory (Q, K, V read once, O written once)",
    "vgpr_limited_occupancy": "resident waves limited by VGPRs AND < 2 waves per SIMD",
    "lds_limited_occupancy": "resident waves limited by LDS AND < 2 waves per SIMD",
    "scalar_math_bound": "no MFMA instructions AND VALU busy > 50% (matmuls run as scalar FMAs)",
    "valu_bound_softmax": "MFMA busy < 60% AND VALU busy > MFMA busy (exp/max/sum/rescale crowd the matrix cores)",
    "lds_bank_conflicts": "> 5% of LDS active cycles stalled on bank conflicts",
    "latency_bound": "> 50% of wave cycles waiting for an issue dependency AND occupancy < 30%",
    "low_parallelism": "< 0.75 waves of workgroups over the 256 CUs (CUs left idle)",
    "register_spills": "the compiler reports VGPR/SGPR spills or scratch for the kernel",
}


@dataclass(frozen=True)
class Bottleneck:
    name: str
    severity: float
    evidence: str

    def __str__(self):
        return f"{self.name} (severity {self.severity:.2f}): {self.evidence}"


def _get(c: dict, k: str, default=None):
    v = c.get(k)
    return default if v is None else v


def diagnose(c: dict, compulsory_bytes: float | None = None) -> list[Bottleneck]:
    """Rules over one measured design point. `c` holds hw_counters.aggregate() quantities plus
    optional 'resident_wgs_per_cu'; unobservable (None) inputs disable the rules that need them."""
    out: list[Bottleneck] = []
    launches = _get(c, "kernel_launches", 1)
    hbm = c.get("hbm_bytes")
    ratio = (hbm / compulsory_bytes) if hbm is not None and compulsory_bytes else None
    if ratio is not None and launches > 1 and ratio > 4:
        out.append(Bottleneck("materialized_intermediate", ratio / 4,
                              f"{launches} launches, HBM traffic {ratio:.1f}x compulsory"))
    if ratio is not None and ratio > 3:
        out.append(Bottleneck("redundant_hbm_traffic", ratio / 3, f"HBM traffic {ratio:.1f}x compulsory"))
    waves = c.get("waves_per_simd_limit")
    lim = c.get("occupancy_limiter") or ""
    if waves is not None and waves < 2 and lim == "vgpr":
        out.append(Bottleneck("vgpr_limited_occupancy", 2 / max(waves, 0.5),
                              f"{waves} wave(s) per SIMD, limited by {c.get('regs')} VGPRs per lane"))
    if waves is not None and waves < 2 and lim == "lds":
        out.append(Bottleneck("lds_limited_occupancy", 2 / max(waves, 0.5), f"{waves} wave(s) per SIMD, limited by LDS"))
    mfma, valu = c.get("mfma_util"), c.get("valu_busy")
    if c.get("mfma_insn") == 0 and valu is not None and valu > 50:
        out.append(Bottleneck("scalar_math_bound", valu / 50, f"no MFMA instructions, VALU busy {valu:.0f}%"))
    if mfma is not None and valu is not None and c.get("mfma_insn") and mfma < 60 and valu > mfma:
        out.append(Bottleneck("valu_bound_softmax", 60 / max(mfma, 1.0),
                              f"MFMA busy {mfma:.0f}% with VALU busy {valu:.0f}%"))
    conf, act = c.get("lds_bank_conflict_cycles"), c.get("lds_active_cycles")
    if conf is not None and act:
        rate = conf / act
        if rate > 0.05:
            out.append(Bottleneck("lds_bank_conflicts", rate / 0.05, f"{100 * rate:.1f}% of LDS cycles in bank conflicts"))
    wf, occ = c.get("wait_frac"), c.get("occupancy")
    if wf is not None and occ is not None and wf > 0.5 and occ < 30:
        out.append(Bottleneck("latency_bound", wf / 0.5, f"{100 * wf:.0f}% of wave cycles waiting, occupancy {occ:.0f}%"))
    wgs = c.get("workgroups")
    per_cu = _get(c, "resident_wgs_per_cu", None)
    if wgs and per_cu:
        waves_of_wgs = wgs / (CUS * per_cu)
        if waves_of_wgs < 0.75:
            out.append(Bottleneck("low_parallelism", 0.75 / max(waves_of_wgs, 1e-3),
                                  f"{wgs} workgroups for {CUS} CUs x {per_cu} resident = {waves_of_wgs:.2f} waves"))
    spill = c.get("spill")
    if spill:
        out.append(Bottleneck("register_spills", 1.0 + spill / 64, f"{spill} spill/scratch units reported by the compiler"))
    out.sort(key=lambda b: -b.severity)
    return out


def resident_wgs_per_cu(waves_per_simd: int, threads: int) -> int:
    """Workgroups resident per CU at `waves_per_simd` (waves of a workgroup spread over 4 SIMDs)."""
    waves_per_wg = max(1, threads // 64)
    return max(1, (min(waves_per_simd, MAX_WAVES_PER_SIMD) * 4) // waves_per_wg)
