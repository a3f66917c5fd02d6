"""Run one entry point a few times on one shape: the target program for rocprofv3.

    rocprofv3 --kernel-trace --stats -d out -- python3 phantom-a100_amd/bench/run_one.py --impl fused_tc --n 4096
    rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE -d out -- \\
        python3 phantom-a100_amd/bench/run_one.py --impl fused_tuned --br 128 --bc 64 --db 1

Mirrors /root/reference/bench/run_one.py:1-28 (there the Nsight target), plus the tile arguments
of fused_tuned, the dtype / head dim of fused_tc, and a first call outside the counted ones so
one-time work (library load) is not in the profile's window of interest.
"""
import argparse
import os
import sys

import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))
import cuda_attn  # noqa: E402

DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def make_call(a, q, k, v):
    if a.candidate:   # an alternative tile of fused_tc (libphantom_attn_tiles.so)
        from autotune import tile_candidates as tc
        index = {c["label"]: c["index"] for c in tc.candidates()}
        if a.candidate not in index:
            raise SystemExit(f"no candidate {a.candidate!r}; compiled: {sorted(index)}")
        return lambda: tc.forward(index[a.candidate], q, k, v, a.causal)
    if a.impl == "fused_tuned":
        return lambda: cuda_attn.fused_tuned(q, k, v, a.causal, bool(a.db), a.br, a.bc)
    fn = cuda_attn.KERNELS[a.impl]
    return lambda: fn(q, k, v, a.causal)


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--impl", choices=list(cuda_attn.KERNELS) + ["fused_tuned"], required=True)
    p.add_argument("--n", type=int, default=4096)
    p.add_argument("--batch", type=int, default=4)
    p.add_argument("--heads", type=int, default=16)
    p.add_argument("--dim", type=int, default=64)
    p.add_argument("--dtype", choices=list(DTYPES), default="fp16")
    p.add_argument("--causal", action="store_true")
    p.add_argument("--br", type=int, default=64)
    p.add_argument("--bc", type=int, default=32)
    p.add_argument("--db", type=int, default=1)
    p.add_argument("--reps", type=int, default=5)
    p.add_argument("--candidate", default="", help="fused_tc: run this alternative of libphantom_attn_tiles.so")
    p.add_argument("--per-block", action="store_true",
                   help="fused_tc: one workgroup per query block (the persistent launch switched off)")
    p.add_argument("--calibrate", action="store_true",
                   help="first copy 1 GiB device-to-device: a known-size transfer that calibrates FETCH_SIZE")
    a = p.parse_args(argv)
    if a.per_block:
        from cuda_attn import _native
        _native.set_persistent(False)
    if a.calibrate:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    gen = torch.Generator().manual_seed(0)
    dt = DTYPES[a.dtype]
    q, k, v = (torch.randn(a.batch, a.heads, a.n, a.dim, generator=gen).to(dt).cuda() for _ in range(3))
    fn = make_call(a, q, k, v)
    for _ in range(a.reps):
        fn()
    torch.cuda.synchronize()
    print(f"ran {a.impl}{' ' + a.candidate if a.candidate else ''}{' per block' if a.per_block else ''} "
          f"N={a.n} d={a.dim} {a.dtype} x{a.reps}", flush=True)


if __name__ == "__main__":
    main()
