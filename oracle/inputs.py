"""Seeded synthetic inputs -- TEST INFRASTRUCTURE (shared by tests and bench).

q, k, v are drawn in that order as fp32 N(0, 1) from a CPU torch.Generator,
multiplied by `scale`, then cast to the target dtype; identical on any box.
(The reference's harness draws on the GPU with seed 42, benchmark.py:1281-1284;
CPU generation makes the inputs machine-independent.)
"""
from __future__ import annotations

import torch


def make_qkv(B: int, Hq: int, Hk: int, M: int, N: int, D: int, *, dtype=torch.float16,
             seed: int = 0, scale: float = 1.0, device="cpu"):
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, Hq, M, D, generator=g, dtype=torch.float32) * scale
    k = torch.randn(B, Hk, N, D, generator=g, dtype=torch.float32) * scale
    v = torch.randn(B, Hk, N, D, generator=g, dtype=torch.float32) * scale
    return tuple(t.to(dtype).to(device) for t in (q, k, v))
