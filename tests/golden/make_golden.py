"""Writes the golden fixtures in tests/golden/*.npz (run in this repo; inputs are seeded).

Each fixture holds q, k, v exactly as the kernels receive them (fp32 / fp16 arrays, bf16 as
uint16 bit patterns), the causal flag, and `o`: the float64 attention output of the C brute
force oracle/attn_ref64.c (restating /root/reference/sim/harness.cu:40-64), stored as float32.
The reference repository stores no golden vectors of its own (its tests regenerate seeded
inputs each run), so these are the committed known answers that the CPU oracle tests and the
GPU parity tests both check against.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "phantom-a100_amd"))
sys.path.insert(0, REPO)

from cuda_attn.workloads import make_qkv  # noqa: E402
import oracle  # noqa: E402

# name: (B, H, N, d, dtype, qk_scale, seed, causal)
CASES = {
    "f32_n128_d64": (1, 3, 128, 64, torch.float32, 1.0, 10, False),
    "f32_n333_d64_causal": (1, 1, 333, 64, torch.float32, 1.0, 11, True),
    "f16_n1_d64": (1, 2, 1, 64, torch.float16, 1.0, 12, False),
    "f16_n65_d64_causal": (2, 2, 65, 64, torch.float16, 1.0, 13, True),
    "f16_n333_d64": (1, 1, 333, 64, torch.float16, 1.0, 14, False),
    "f16_n1024_d64_peaked": (1, 1, 1024, 64, torch.float16, 3.0, 15, False),
    "bf16_n200_d128_causal": (1, 2, 200, 128, torch.bfloat16, 1.0, 16, True),
    "bf16_n256_d128": (1, 1, 256, 128, torch.bfloat16, 1.0, 17, False),
    "f32_n200_d80": (1, 1, 200, 80, torch.float32, 1.0, 18, False),
}


def to_store(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def main() -> None:
    for name, (b, h, n, d, dtype, qk, seed, causal) in CASES.items():
        q, k, v = make_qkv(b, h, n, d, dtype, seed=seed, qk_scale=qk)
        o = oracle.attention_ref64(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), q=to_store(q), k=to_store(k), v=to_store(v),
                            o=o.astype(np.float32), causal=np.array(causal), seed=np.array(seed),
                            qk_scale=np.array(qk), dtype=np.array(str(dtype).replace("torch.", "")))
        print(name, q.shape, dtype, "causal" if causal else "", "max|o|=%.3f" % np.abs(o).max())


if __name__ == "__main__":
    main()
