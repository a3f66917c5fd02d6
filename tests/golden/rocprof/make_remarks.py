"""Regenerate resource_remarks.txt: the compiler's kernel-resource report (the remarks that
`-Rpass-analysis=kernel-resource-usage` prints for gfx950) of five representative kernels, kept
as a fixture for the parser and occupancy-model tests.

    python tests/golden/rocprof/make_remarks.py

Compiles phantom-a100_amd/csrc/pa_attn.hip with the library's own device flags (no GPU needed)
and keeps the remark blocks of the kernels KERNELS names (one compiled kernel per name prefix), in
that order.
"""
from __future__ import annotations

import importlib.util
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.abspath(os.path.join(HERE, "..", "..", ".."))
PKG = os.path.join(REPO, "phantom-a100_amd")
# Kernels kept, by the mangled name up to the end of the template arguments (the parameter list
# that follows is not matched, so a change of the kernel's signature keeps the fixture regenerable):
# the naive softmax, the persistent fused_tc d=64 kernel (fp16 in, fp32 out, packed-max check), the persistent C4
# kernel (bf16 d=128, BM=256), a one-stage fused_tuned tile and the fp32 fused kernel.
KERNELS = [
    "_ZN2pa13naive_softmaxE",
    "_ZN2pa11fa_mfma_fwdIDF16_Li64ELi128ELi64ELi2EfLi1ELb1ELb0ELb0ELb1EEEv",
    "_ZN2pa11fa_mfma_fwdIDF16bLi128ELi256ELi64ELi2EDF16bLi1ELb1ELb0ELb0ELb0EEEv",
    "_ZN2pa11fa_mfma_fwdIDF16_Li64ELi128ELi32ELi1EDF16_Li1ELb0ELb0ELb0ELb0EEEv",
    "_ZN2pa10fa_f32_fwdIfLi64ELi4EfEEv",
]


def main() -> str:
    spec = importlib.util.spec_from_file_location("pa_build_native", os.path.join(PKG, "build_native.py"))
    bn = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bn)
    with tempfile.TemporaryDirectory() as tmp:
        cmd = [bn.hipcc(), *bn.DEVICE_FLAGS, *bn.COMMON_FLAGS, "-Rpass-analysis=kernel-resource-usage",
               "--cuda-device-only", "-c", "-I", os.path.join(REPO, "include"), "-I", os.path.join(PKG, "csrc"),
               os.path.join(PKG, "csrc", "pa_attn.hip"), "-o", os.path.join(tmp, "pa_attn.o")]
        text = subprocess.run(cmd, capture_output=True, text=True, check=True, cwd=REPO).stderr
    blocks, cur = {}, None
    for line in text.splitlines():
        if "remark:" not in line or "kernel-resource-usage" not in line:
            continue
        if "Function Name:" in line:
            cur = line.split("Function Name:")[1].split("[")[0].strip()
            blocks[cur] = []
        if cur is not None:
            blocks[cur].append(line)
    chosen = []
    for prefix in KERNELS:
        names = [name for name in blocks if name.startswith(prefix)]
        if len(names) != 1:
            raise SystemExit(f"{prefix}: {len(names)} compiled kernels match (want exactly one): {names[:4]}")
        chosen.append(names[0])
    out = "\n".join(line for k in chosen for line in blocks[k]) + "\n"
    path = os.path.join(HERE, "resource_remarks.txt")
    with open(path, "w") as fh:
        fh.write(out)
    return path


if __name__ == "__main__":
    print(main())
