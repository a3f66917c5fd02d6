"""Host-side checks that need no GPU: the public surface mirrors the reference package, argument
checks raise the reference's messages, and libphantom_attn.so loads and exports every entry point
declared in include/phantom_attn.h. Calls into the library here stop at its argument validation;
no kernel is launched.
"""
import ctypes
import inspect
import os
import re

import pytest
import torch

import cuda_attn
from cuda_attn import _checks, _native

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "phantom_attn.h")


# ---------------------------------------------------------------- public surface
def test_public_names_match_reference():
    # /root/reference/cuda_attn/__init__.py:93-94
    assert cuda_attn.__all__ == ["naive", "tiled", "fused", "fused_tuned", "fused_vec", "fused_db", "fused_tc",
                                 "reference", "KERNELS", "FP16_ONLY"]
    assert list(cuda_attn.KERNELS) == ["naive", "tiled", "fused", "fused_vec", "fused_db", "fused_tc"]
    assert cuda_attn.FP16_ONLY == {"fused_vec", "fused_db", "fused_tc"}
    for name in cuda_attn.__all__:
        assert hasattr(cuda_attn, name)


def test_signatures_and_defaults_match_reference():
    # /root/reference/cuda_attn/__init__.py:40-75 and csrc/bindings.cpp:42-53
    for name in ("naive", "tiled", "fused", "fused_tc", "fused_vec", "fused_db", "reference"):
        params = list(inspect.signature(getattr(cuda_attn, name)).parameters.values())
        assert [p.name for p in params[:4]] == ["q", "k", "v", "causal"]
        assert params[3].default is False
    p = inspect.signature(cuda_attn.fused_tuned).parameters
    assert [n for n in p][:7] == ["q", "k", "v", "causal", "double_buffer", "br", "bc"]
    assert (p["causal"].default, p["double_buffer"].default, p["br"].default, p["bc"].default) == (False, True, 64, 32)
    # extension: keyword-only out_dtype on the fused entry points
    for name in ("fused", "fused_tuned", "fused_tc"):
        od = inspect.signature(getattr(cuda_attn, name)).parameters["out_dtype"]
        assert od.kind is inspect.Parameter.KEYWORD_ONLY and od.default is None


# ---------------------------------------------------------------- argument checks (CPU tensors)
def qkv(shape=(1, 2, 64, 64), dtype=torch.float16):
    return [torch.zeros(shape, dtype=dtype) for _ in range(3)]


def test_cpu_tensors_rejected_before_any_native_call():
    q, k, v = qkv()
    for name, fn in cuda_attn.KERNELS.items():
        with pytest.raises(RuntimeError, match="CUDA tensors"):
            fn(q, k, v)


def test_check_inputs_messages():
    q, k, v = qkv()
    chk = lambda *a: _checks.check_inputs(*a, require_cuda=False)  # noqa: E731
    with pytest.raises(RuntimeError, match="contiguous"):
        chk(q.transpose(2, 3), k, v)
    with pytest.raises(RuntimeError, match="dtype"):
        chk(q, k.float(), v)
    with pytest.raises(RuntimeError, match=r"shaped \(B, H, N, d\)"):
        chk(q[0], k[0], v[0])
    with pytest.raises(RuntimeError, match="same shape"):
        chk(q, k[:, :, :32].contiguous(), v)
    with pytest.raises(RuntimeError, match="non-empty"):
        e = torch.zeros((1, 2, 0, 64), dtype=torch.float16)
        chk(e, e.clone(), e.clone())
    chk(q, k, v)  # valid


def test_head_dim_and_dtype_messages():
    q, k, v = qkv((1, 1, 64, 128))
    with pytest.raises(RuntimeError, match="head dimension"):
        _checks.check_head_dim("fused_forward", q, (64,))
    with pytest.raises(RuntimeError, match="head dimension"):
        _checks.check_fp16_d64_aligned("fused_tuned", q, k, v)
    _checks.check_tc(q, k, v)  # d = 128 is compiled for fused_tc (extension)
    q96, k96, v96 = qkv((1, 1, 64, 96))
    with pytest.raises(RuntimeError, match="head dimension"):
        _checks.check_tc(q96, k96, v96)
    q32, k32, v32 = qkv(dtype=torch.float32)
    with pytest.raises(RuntimeError, match="float16"):
        _checks.check_fp16_d64_aligned("fused_tuned", q32, k32, v32)
    with pytest.raises(RuntimeError, match="float16"):
        _checks.check_tc(q32, k32, v32)
    qb, kb, vb = qkv(dtype=torch.bfloat16)
    _checks.check_tc(qb, kb, vb)
    with pytest.raises(RuntimeError, match="float16"):
        _checks.check_fp16_d64_aligned("fused_tuned", qb, kb, vb)
    with pytest.raises(RuntimeError, match="only float32 and float16"):
        _checks.check_float_half("fused_forward", qb)


def test_alignment_message():
    base = torch.zeros(1 * 1 * 64 * 64 + 1, dtype=torch.float16)
    q = base[1:].view(1, 1, 64, 64)  # 2-byte offset
    _, k, v = qkv((1, 1, 64, 64))
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        _checks.check_fp16_d64_aligned("fused_tuned", q, k, v)


def test_tuned_config_and_lds_messages():
    with pytest.raises(RuntimeError, match="not compiled"):
        _checks.check_tuned_config(32, 32)
    for br, bc in _checks.TUNED_CONFIGS:
        _checks.check_tuned_config(br, bc)
    with pytest.raises(RuntimeError, match="shared memory"):
        _checks.check_lds("fused_tuned", 70000, 65536, "BR=128 BC=64")
    with pytest.raises(RuntimeError, match="shared memory"):
        _checks.check_lds("fused_tc", 70000, 65536)
    _checks.check_lds("fused_tc", 65536, 65536)


def test_out_dtype_resolution():
    q = torch.zeros(1, dtype=torch.float16)
    assert _checks.resolve_out_dtype("fused_tc", q, None) == torch.float16
    assert _checks.resolve_out_dtype("fused_tc", q, torch.float32) == torch.float32
    with pytest.raises(RuntimeError, match="out_dtype"):
        _checks.resolve_out_dtype("fused_tc", q, torch.bfloat16)


# ---------------------------------------------------------------- C ABI
def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pa_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = header_functions()
    assert names == sorted(_native.PROTOTYPES), names


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    for name in header_functions():
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_version_string():
    assert "gfx950" in _native.version()


def test_lds_bytes_queries():
    lib = _native.lib()
    for br, bc in _checks.TUNED_CONFIGS:
        one = lib.pa_fused_tuned_lds_bytes(br, bc, 0, 64, _native.DTYPE_F16)
        two = lib.pa_fused_tuned_lds_bytes(br, bc, 1, 64, _native.DTYPE_F16)
        assert 0 < one < two <= 160 * 1024
        assert two == 2 * one
    assert lib.pa_fused_tuned_lds_bytes(32, 32, 1, 64, _native.DTYPE_F16) == -1
    assert lib.pa_fused_tuned_lds_bytes(64, 32, 1, 128, _native.DTYPE_F16) == -1
    for d in (64, 128):
        for dt in (_native.DTYPE_F16, _native.DTYPE_BF16):
            assert 0 < lib.pa_fused_tc_lds_bytes(d, dt) <= 160 * 1024
    assert lib.pa_fused_tc_lds_bytes(96, _native.DTYPE_F16) == -1
    assert lib.pa_fused_tc_lds_bytes(64, _native.DTYPE_F32) == -1


def test_native_argument_validation_without_gpu():
    """Rejected arguments return a negative status and a message; no HIP call is made."""
    lib = _native.lib()
    rc = lib.pa_fused_tc_fwd(None, None, None, None, _native.DTYPE_F16, _native.DTYPE_F16, 1, 64, 64, 0, None)
    assert rc == _native.ERR_INVALID and "null" in _native.last_error()
    p = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    rc = lib.pa_fused_tc_fwd(p, p, p, p, _native.DTYPE_F32, _native.DTYPE_F32, 1, 64, 64, 0, None)
    assert rc == _native.ERR_UNSUPPORTED and "float16" in _native.last_error()
    rc = lib.pa_fused_tc_fwd(p, p, p, p, _native.DTYPE_F16, _native.DTYPE_F16, 1, 64, 96, 0, None)
    assert rc == _native.ERR_UNSUPPORTED and "head dimension" in _native.last_error()
    rc = lib.pa_fused_tuned_fwd(p, p, p, p, _native.DTYPE_F16, _native.DTYPE_F16, 1, 64, 64, 0, 1, 32, 32, None)
    assert rc == _native.ERR_UNSUPPORTED and "not compiled" in _native.last_error()
    rc = lib.pa_fused_fwd(p, p, p, p, _native.DTYPE_F32, _native.DTYPE_F32, 0, 64, 64, 0, None)
    assert rc == _native.ERR_INVALID and "non-empty" in _native.last_error()
    rc = lib.pa_fused_fwd(p, p, p, p, _native.DTYPE_F32, _native.DTYPE_F32, 1, 64, 80, 0, None)
    assert rc == _native.ERR_UNSUPPORTED and "head dimension" in _native.last_error()
    rc = lib.pa_naive_fwd(p, p, p, p, None, _native.DTYPE_F32, 1, 64, 64, 0, None)
    assert rc == _native.ERR_INVALID and "workspace" in _native.last_error()
    rc = lib.pa_tiled_fwd(p, p, p, p, p, _native.DTYPE_BF16, 1, 64, 64, 0, None)
    assert rc == _native.ERR_UNSUPPORTED and "float32 and float16" in _native.last_error()
    rc = lib.pa_tiled_fwd_noalloc(p, p, p, p, _native.DTYPE_F16, 2, 4096, 64, 0, None)   # 2 x 4096^2 scores
    assert rc == _native.ERR_UNSUPPORTED and "static scratch" in _native.last_error()
    rc = lib.pa_tiled_fwd_noalloc(p, p, p, p, _native.DTYPE_F16, 65535, 262140, 64, 0, None)  # no overflow
    assert rc == _native.ERR_UNSUPPORTED and "static scratch" in _native.last_error()
    rc = lib.pa_tiled_fwd_noalloc(p, p, p, p, _native.DTYPE_BF16, 1, 64, 64, 0, None)
    assert rc == _native.ERR_UNSUPPORTED and "float32 and float16" in _native.last_error()
    q = ctypes.c_void_p(258)  # misaligned
    rc = lib.pa_fused_tc_fwd(q, p, p, p, _native.DTYPE_F16, _native.DTYPE_F16, 1, 64, 64, 0, None)
    assert rc == _native.ERR_INVALID and "16-byte aligned" in _native.last_error()
    with pytest.raises(RuntimeError, match="head dimension"):
        _native.check(lib.pa_fused_tc_fwd(p, p, p, p, _native.DTYPE_F16, _native.DTYPE_F16, 1, 64, 96, 0, None),
                      "fused_tc")


def test_c_abi_example_builds_and_runs(tmp_path):
    """The C integration path: tests/native/c_abi_example.c includes both public headers as C99
    (-Wall -Werror), links against the two libraries with gcc and runs calls that need no GPU."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not installed")
    lib_dir = os.path.dirname(_native.LIB_PATH)
    exe = str(tmp_path / "c_abi_example")
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(REPO, "include"),
                    os.path.join(REPO, "tests", "native", "c_abi_example.c"), "-o", exe, "-L", lib_dir, "-lphantom_attn",
                    "-lphantom_attn_tiles", f"-Wl,-rpath,{lib_dir}"], check=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    assert out.stdout.startswith("c abi ok: phantom_attn")


def test_fused_tc_kernel_description_without_gpu():
    """The launch description follows the dispatch table; with no device the persistent launch is
    not chosen (as in pa_fused_tc_fwd), and the setter reports the previous setting."""
    f16, bf16, f32 = _native.DTYPE_F16, _native.DTYPE_BF16, _native.DTYPE_F32
    d128 = _native.fused_tc_kernel(bf16, bf16, 128, 4096, 128)
    assert d128.startswith("fa_mfma_fwd<bf16, D=128, BM=256, BN=64, 2 stages, out bf16")
    assert "grid 2048 x 512 threads" in d128
    d64 = _native.fused_tc_kernel(f16, f32, 128, 1024, 64)
    assert "D=64, BM=128" in d64 and "out f32" in d64 and "grid 1024 x 256 threads" in d64
    assert "key split 2" in _native.fused_tc_kernel(f16, f16, 42, 128, 64)
    # d = 128, 256-query blocks (one per CU at a time, 256 CUs): the 128-query tile up to half the
    # CUs (causal: all), and non-causal past one round where the last round is at most 85 % full
    tile = lambda bh, n, causal=0: re.search(r"BM=(\d+)", _native.fused_tc_kernel(bf16, bf16, bh, n, 128, causal))[1]
    assert [tile(32, 1024), tile(64, 1024), tile(64, 1024, 1), tile(80, 1024, 1)] == ["128", "256", "128", "256"]
    assert [tile(72, 1024), tile(20, 4096), tile(144, 1024), tile(36, 4096)] == ["128"] * 4   # rounds 1.13-2.25
    assert [tile(112, 1024), tile(64, 2048), tile(56, 4096), tile(128, 4096)] == ["256"] * 4  # rounds 1.75, 2, 3.5, 8
    assert tile(72, 1024, 1) == "256"
    # rows whose last 256-query block is mostly padding: past one round from 14 % padding on
    # (N = 128, 384, 896), within one round for N <= 128 only
    assert [tile(600, 128), tile(512, 384), tile(256, 896), tile(256, 128)] == ["128"] * 4
    assert [tile(256, 1100), tile(100, 384), tile(40, 1100), tile(256, 1536)] == ["256"] * 4
    assert _native.fused_tc_kernel(f16, f16, 1, 64, 96) == ""
    assert _native.fused_tc_kernel(f32, f32, 1, 64, 64) == ""
    prev = _native.set_persistent(False)
    try:
        assert _native.set_persistent(True) is False
    finally:
        _native.set_persistent(prev)


def test_workload_accounting():
    from cuda_attn.workloads import CONFIGS
    # figures of the measurement plan: FLOPs = 4*BH*N^2*d, bytes = (3*in + out) * BH*N*d
    assert CONFIGS["C1"].flops() == 176160768
    assert CONFIGS["C3"].flops() == 34359738368
    assert CONFIGS["C4"].flops() == 1099511627776
    assert CONFIGS["C5"].flops() == 274877906944
    assert CONFIGS["C4"].hbm_bytes() == 536870912
    assert CONFIGS["C1"].hbm_bytes() == 5505024
