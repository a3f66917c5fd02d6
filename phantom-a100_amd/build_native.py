"""Build libphantom_attn.so (the HIP kernels + C ABI) for gfx950, in-tree.

    python phantom-a100_amd/build_native.py            # -> phantom-a100_amd/cuda_attn/libphantom_attn.so

hipcc cross-compiles without a GPU. Flags:
  --offload-arch=gfx950                  MI355X (CDNA4) only
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                         no packed fp32 (v_pk_*_f32) instructions in device code
  -mllvm -amdgpu-mfma-vgpr-form=1        MFMA accumulators in ordinary VGPRs, so the softmax can
                                         read S and rescale O without accvgpr copies
  -Rpass-analysis=kernel-resource-usage  the compiler's per-kernel resource report (VGPRs, AGPRs,
                                         SGPRs, spills, scratch, LDS, occupancy), saved beside the
                                         library as kernel_resources.json for the tile-choice tool
"""
from __future__ import annotations

import json
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT = os.path.join(HERE, "cuda_attn", "libphantom_attn.so")
# The tile alternatives for the counter-driven tile choice (autotune/select_tiles.py); never loaded
# by cuda_attn.
TILES_OUT = os.path.join(HERE, "cuda_attn", "libphantom_attn_tiles.so")
RESOURCES = os.path.join(HERE, "cuda_attn", "kernel_resources.json")
LIBRARIES = {OUT: ["pa_attn.hip"], TILES_OUT: ["pa_tiles.hip"]}
SOURCES = [src for srcs in LIBRARIES.values() for src in srcs]
ARCH = "gfx950"

DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build libphantom_attn.so)")
    return path


def build(verbose: bool = False) -> str:
    """Compile every source (in parallel) and link libphantom_attn.so and libphantom_attn_tiles.so;
    returns the path of libphantom_attn.so."""
    objs = {}
    os.makedirs(os.path.join(HERE, "_build"), exist_ok=True)
    procs = []
    for src in SOURCES:
        obj = os.path.join(HERE, "_build", os.path.splitext(src)[0] + ".o")
        cmd = [hipcc(), *DEVICE_FLAGS, *COMMON_FLAGS, "-Rpass-analysis=kernel-resource-usage",
               "-I", INCLUDE, "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs[src] = obj
    failed = []
    resources = {}
    for src, p in procs:
        out, _ = p.communicate()
        resources.update(parse_resource_remarks(out))
        # hipcc's host pass does not know the device-only target feature; that warning is noise,
        # and the resource remarks go to kernel_resources.json.
        lines = [ln for ln in out.splitlines() if "unknown target feature" not in ln and ln.strip()
                 and "packed-fp32-ops" not in ln and "kernel-resource-usage" not in ln
                 and not re.match(r"^\s*(\d+ \|.*|\|?\s*\^)$", ln) and not ln.startswith("In file included")]
        if p.returncode != 0:
            failed.append(src)
            print("\n".join(lines), file=sys.stderr)
        elif verbose and lines:
            print("\n".join(lines))
    if failed:
        raise RuntimeError("hipcc failed for: " + ", ".join(failed))
    for lib_path, srcs in LIBRARIES.items():
        tmp = lib_path + ".tmp"
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *(objs[src] for src in srcs), "-o", tmp]
        subprocess.run(cmd, check=True)
        check_no_missing_stubs(tmp)
        os.replace(tmp, lib_path)
    with open(RESOURCES, "w") as fh:
        json.dump(resources, fh, indent=1, sort_keys=True)
        fh.write("\n")
    return OUT


_REMARK = re.compile(r"remark:\s+(Function Name|[A-Za-z][A-Za-z ]*?(?: \[[^\]]+\])?):\s*(\S+)\s*\[-Rpass-analysis")
_FIELDS = {"TotalSGPRs": "sgprs", "VGPRs": "vgprs", "AGPRs": "agprs", "ScratchSize [bytes/lane]": "scratch_bytes",
           "Occupancy [waves/SIMD]": "occupancy_waves_per_simd", "SGPRs Spill": "sgpr_spill",
           "VGPRs Spill": "vgpr_spill", "LDS Size [bytes/block]": "lds_bytes", "Dynamic Stack": "dynamic_stack"}


def parse_resource_remarks(text: str) -> dict:
    """Per-kernel resources from hipcc -Rpass-analysis=kernel-resource-usage output:
    {mangled name: {vgprs, agprs, sgprs, scratch_bytes, occupancy_waves_per_simd, ...}}."""
    out, cur = {}, None
    for m in _REMARK.finditer(text):
        key, val = m.group(1).strip(), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None and key in _FIELDS:
            cur[_FIELDS[key]] = (val == "True") if key == "Dynamic Stack" else int(val)
    return out


def check_no_missing_stubs(path: str) -> None:
    """Fail the build if a kernel's host-side launch stub was not emitted (the library would
    then fail to load with an undefined __device_stub__ symbol)."""
    nm = shutil.which("nm")
    if not nm:
        return
    out = subprocess.run([nm, "-D", "--undefined-only", path], capture_output=True, text=True, check=True).stdout
    missing = [ln.split()[-1] for ln in out.splitlines() if "__device_stub__" in ln]
    if missing:
        os.remove(path)
        raise RuntimeError("kernel launch stubs missing from the host object:\n  " + "\n  ".join(missing[:10]))


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
