"""Host-only checks of the causal walk and the launch model (no GPU): builds and runs
tests/native/launch_model_check.cpp with hipcc, which cross-compiles here without a device."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        pytest.skip("hipcc not found")
    return path


def test_causal_walk_and_launch_model(tmp_path):
    exe = tmp_path / "launch_model_check"
    cmd = [hipcc(), "--offload-arch=gfx950", "-O2", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I", os.path.join(REPO, "include"), "-I", os.path.join(REPO, "phantom-a100_amd", "csrc"),
           os.path.join(HERE, "native", "launch_model_check.cpp"), "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert build.returncode == 0, build.stdout + build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(run.stdout)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip().endswith("ok")


def test_walk_cache_under_thread_sanitizer(tmp_path):
    """The same checks built with ThreadSanitizer on the host code (the walk cache's mutex under
    eight threads); skipped where the toolchain lacks the sanitizer runtime."""
    exe = tmp_path / "launch_model_check_tsan"
    cmd = [hipcc(), "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", *"-Xarch_host -fsanitize=thread".split(), "-I", os.path.join(REPO, "include"),
           "-I", os.path.join(REPO, "phantom-a100_amd", "csrc"), os.path.join(HERE, "native", "launch_model_check.cpp"),
           "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    if build.returncode != 0:
        pytest.skip("no ThreadSanitizer build here: " + (build.stderr.strip().splitlines() or [""])[-1][:200])
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0 and "ThreadSanitizer" not in run.stderr, run.stdout[-2000:] + run.stderr[-4000:]
    assert run.stdout.strip().endswith("ok")
