"""Regenerate resource_remarks.txt: the compiler's kernel-resource report (the remarks that
`-Rpass-analysis=kernel-resource-usage` prints for gfx950) of five representative kernels, kept
as a fixture for the parser and occupancy-model tests.

    python tests/golden/rocprof/make_remarks.py

Compiles phantom-a100_amd/csrc/pa_attn.hip with the library's own device flags (no GPU needed)
and keeps the remark blocks of the kernels named in KERNELS, in that order.
"""
from __future__ import annotations

import importlib.util
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.abspath(os.path.join(HERE, "..", "..", ".."))
PKG = os.path.join(REPO, "phantom-a100_amd")
KERNELS = [
    "_ZN2pa13naive_softmaxEPfi",
    "_ZN2pa11fa_mfma_fwdIDF16_Li64ELi128ELi64ELi2EfLi1ELb0ELb0EEEvPKT_S3_S3_PT4_iiifi",
    "_ZN2pa11fa_mfma_fwdIDF16bLi128ELi256ELi64ELi2EDF16bLi1ELb1ELb0EEEvPKT_S3_S3_PT4_iiifi",
    "_ZN2pa11fa_mfma_fwdIDF16_Li64ELi128ELi32ELi1EDF16_Li1ELb0ELb0EEEvPKT_S3_S3_PT4_iiifi",
    "_ZN2pa10fa_f32_fwdIfLi64ELi4EfEEvPKT_S3_S3_PT2_iiifi",
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
    missing = [k for k in KERNELS if k not in blocks]
    if missing:
        raise SystemExit(f"not compiled: {missing}")
    out = "\n".join(line for k in KERNELS for line in blocks[k]) + "\n"
    path = os.path.join(HERE, "resource_remarks.txt")
    with open(path, "w") as fh:
        fh.write(out)
    return path


if __name__ == "__main__":
    print(main())
