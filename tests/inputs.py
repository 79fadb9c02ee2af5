"""Seeded synthetic inputs shared by the tests, bench.py and smoke().

Draw order for a ConvRot activation (fixed; the seed alone does not fix it):
  x = randn(M, K) in fp32; outlier channels = randperm(K)[:max(1, round(0.001 K))];
  x[:, outliers] *= 20; x -> bf16.
Weights: randint(-127, 128, (N, K)) int8; weight scales uniform(1e-3, 5e-3) fp32;
bias: randn(N) * 0.02 -> bf16 -> fp32.
Attention: q, k, v = randn(B, H, L, D) fp32 (that order); k += randn(B, H, 1, D) * 2
(per-head channel bias, exercising smoothing); all -> bf16.
"""
from __future__ import annotations

import numpy as np
import torch


def activation(m: int, k: int, seed: int, outlier_scale: float = 20.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g, dtype=torch.float32)
    n_out = max(1, round(0.001 * k))
    idx = torch.randperm(k, generator=g)[:n_out]
    x[:, idx] *= outlier_scale
    return x.to(torch.bfloat16)


def weights(n: int, k: int, seed: int, with_bias: bool = True):
    g = torch.Generator().manual_seed(seed + 1000)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    ws = torch.empty(n, dtype=torch.float32).uniform_(1e-3, 5e-3, generator=g)
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16).float() if with_bias else None
    return w, ws, bias


def attention(b: int, h: int, l: int, d: int, seed: int, hkv: int | None = None, lk: int | None = None):
    g = torch.Generator().manual_seed(seed)
    hkv = h if hkv is None else hkv
    lk = l if lk is None else lk
    q = torch.randn(b, h, l, d, generator=g)
    k = torch.randn(b, hkv, lk, d, generator=g)
    v = torch.randn(b, hkv, lk, d, generator=g)
    k = k + torch.randn(b, hkv, 1, d, generator=g) * 2.0
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> numpy uint16 bit patterns (CPU copy)."""
    assert t.dtype == torch.bfloat16
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)
