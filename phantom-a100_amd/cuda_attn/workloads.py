"""The five benchmark configurations, their seeded synthetic inputs and work accounting.

Input generation mirrors the reference's test helper (/root/reference/tests/test_correctness.py:17-20):
q, k, v drawn in that order as fp32 randn from one generator, scaled, then cast. Here the
generator is a CPU torch.Generator so the same bits reach the GPU kernel and the CPU oracle.

FLOPs follow the reference's convention 4*B*H*N^2*d, halved when causal
(/root/reference/bench/benchmark.py:63-66). Compulsory HBM bytes = read Q, K, V once and write O once.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Config:
    name: str
    B: int
    H: int
    N: int
    d: int
    dtype: torch.dtype
    qk_scale: float      # Q and K are multiplied by this after the N(0,1) draw
    seed: int
    entry: str           # cuda_attn entry point that serves this config
    out_dtype: torch.dtype

    @property
    def BH(self) -> int:
        return self.B * self.H

    def flops(self, causal: bool = False) -> float:
        return attention_flops(self.B, self.H, self.N, self.d, causal)

    def hbm_bytes(self) -> int:
        return compulsory_bytes(self.BH, self.N, self.d, self.dtype, self.out_dtype)


# BASELINE configs C1..C5 (non-causal, scale 1/sqrt(d)).
CONFIGS = {
    "C1": Config("C1", 1, 42, 128, 64, torch.float32, 1.0, 0, "fused", torch.float32),
    "C2": Config("C2", 1, 42, 128, 64, torch.float16, 1.0, 1, "fused_tc", torch.float32),
    "C3": Config("C3", 8, 16, 1024, 64, torch.float16, 1.0, 2, "fused_tc", torch.float16),
    "C4": Config("C4", 4, 32, 4096, 128, torch.bfloat16, 1.0, 3, "fused_tc", torch.bfloat16),
    "C5": Config("C5", 1, 16, 8192, 64, torch.float16, 3.0, 4, "fused_tc", torch.float32),
}


def attention_flops(b: int, h: int, n: int, d: int, causal: bool = False) -> float:
    """Two matmuls of 2*N*N*d FLOPs per head; causal counts half (FA convention)."""
    f = 4.0 * b * h * n * n * d
    return f / 2 if causal else f


def compulsory_bytes(bh: int, n: int, d: int, in_dtype: torch.dtype, out_dtype: torch.dtype) -> int:
    isz = torch.empty((), dtype=in_dtype).element_size()
    osz = torch.empty((), dtype=out_dtype).element_size()
    return (3 * isz + osz) * bh * n * d


def make_qkv(b: int, h: int, n: int, d: int, dtype: torch.dtype, *, seed: int = 0, qk_scale: float = 1.0,
             device: str | torch.device = "cpu"):
    """q, k, v of shape (b, h, n, d): fp32 N(0,1) draws from a seeded CPU generator, q and k
    multiplied by qk_scale, cast to dtype, then moved to `device`."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    out = []
    for i in range(3):
        x = torch.randn(b, h, n, d, dtype=torch.float32, generator=g)
        if i < 2 and qk_scale != 1.0:
            x = x * qk_scale
        out.append(x.to(dtype).to(device).contiguous())
    return out


def config_inputs(cfg: Config, device: str | torch.device = "cpu"):
    return make_qkv(cfg.B, cfg.H, cfg.N, cfg.d, cfg.dtype, seed=cfg.seed, qk_scale=cfg.qk_scale, device=device)
