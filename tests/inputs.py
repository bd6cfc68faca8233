"""Seeded input generators shared by the CPU and GPU tests.

The adversarial kinds follow the reference's G1/G2 generator
(src/verify_v3_kernels.py:98-131): random, zeros, one large outlier per group,
all-negative, bf16-denormal territory and mixed magnitudes e^U(-60, 6).
Tensors are produced on the CPU with a seeded torch.Generator and returned as
bf16 (the fused kernels' dtype) unless `dtype` says otherwise.
"""

from __future__ import annotations

import torch

KINDS = ("random", "zeros", "outlier", "negatives", "denormal", "mixed_magnitude")


def make_pair(kind: str, n: int, d: int, group: int = 64, seed: int = 41,
              dtype=torch.bfloat16):
    """Two [n, d] tensors (h_gate-like, h_up-like) of the given kind."""
    g = torch.Generator().manual_seed(seed)

    def randn(scale=1.0):
        return (torch.randn(n, d, generator=g) * scale).to(dtype)

    if kind == "random":
        return randn(3.0), randn(2.0)
    if kind == "zeros":
        z = torch.zeros(n, d, dtype=dtype)
        return z, z.clone()
    if kind == "outlier":
        base = randn(1e-3).float().view(n, d // group, group)
        idx = torch.randint(0, group, (n, d // group), generator=g)
        sign = torch.where(torch.rand(n, d // group, generator=g) > 0.5, 1.0, -1.0)
        base.scatter_(2, idx.unsqueeze(-1), (1e4 * sign).unsqueeze(-1))
        return base.view(n, d).to(dtype), randn(2.0)
    if kind == "negatives":
        return -randn(3.0).abs(), -randn(2.0).abs()
    if kind == "denormal":
        a = (torch.randn(n, d, generator=g) * 1e-38).to(dtype)
        b = (torch.randn(n, d, generator=g) * 1e-40).to(dtype)
        return a, b
    if kind == "mixed_magnitude":
        mag = torch.exp(torch.empty(n, d).uniform_(-60, 6, generator=g))
        a = (torch.randn(n, d, generator=g) * mag).to(dtype)
        b = (torch.randn(n, d, generator=g) * mag.flip(0)).to(dtype)
        return a, b
    raise ValueError(kind)


def randn(shape, seed: int, scale: float = 1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)
