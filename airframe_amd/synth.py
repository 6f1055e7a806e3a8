"""Seeded synthetic K/V/Q for the INT4 KV path (no model weights exist for this path).

Values are f32 ~N(0,1).  With outliers, each kv head gets ceil(frac*hd) seeded channels
scaled by `factor` (same channels at every position); a query head uses the channels of the
kv head it reads, so the outlier channels line up in q.k.
"""
from __future__ import annotations

import math

import numpy as np


def outlier_dims(n_kv: int, hd: int, seed: int, frac: float = 0.02) -> np.ndarray:
    k = max(1, math.ceil(frac * hd))
    rng = np.random.default_rng(seed + 7919)
    return np.stack([np.sort(rng.choice(hd, size=k, replace=False)) for _ in range(n_kv)])


def channel_scale(n_heads: int, n_kv: int, hd: int, dims: np.ndarray | None,
                  factor: float = 8.0) -> np.ndarray:
    """[n_heads, hd] f32 multiplier: `factor` on the outlier channels of each head's kv head."""
    s = np.ones((n_heads, hd), np.float32)
    if dims is not None:
        group = n_heads // n_kv
        for h in range(n_heads):
            s[h, dims[h // group]] = factor
    return s


def normal(rng: np.random.Generator, shape, scale: np.ndarray | None = None) -> np.ndarray:
    x = rng.standard_normal(shape, dtype=np.float32)
    if scale is not None:
        x = (x * scale).astype(np.float32)
    return x


def normal_torch(shape, gen, device, scale=None):
    """Same distribution drawn on the device with a seeded torch.Generator (bench sizes)."""
    import torch
    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if scale is not None:
        x.mul_(torch.as_tensor(scale, device=device))
    return x
