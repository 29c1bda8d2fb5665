"""Seeded input generation shared by the tests (CPU and GPU)."""

from __future__ import annotations

import numpy as np

from oracle import bf16


def randn_bf16(shape, seed: int, *, std: float = 1.0, offset=None) -> np.ndarray:
    """float32 numpy array of bf16-rounded N(0, std^2) values (torch generator)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g, dtype=torch.float32) * std
    if offset is not None:
        x = x + offset
    return bf16.round_f32(x.numpy())


def key_offset(heads: int, dim: int, seed: int, std: float = 0.5):
    """Per-(head, channel) key offset shared by all tokens (outlier channels)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    return torch.randn(heads, dim, generator=g, dtype=torch.float32) * std


def to_dev(x: np.ndarray, device):
    return bf16.to_torch(x, device)


def err_stats(got: np.ndarray, want: np.ndarray) -> tuple[float, float]:
    d = np.abs(np.asarray(got, dtype=np.float64) - np.asarray(want, dtype=np.float64))
    return float(d.max()), float(d.mean())
