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


LOG2E = 1.4426950408889634

# Inputs whose logits jump by more than 2^8 (in exp2 units) after the first
# 32 keys, so that the attention kernel's running reference has to move (its
# lazy rescale of O and l) for most query rows.  Values use std 0.25: with a
# peaky softmax the output is close to one value row, and the bf16 rounding of
# a unit-scale output alone would average about 1.5e-3, above the 1e-3 gate,
# while a wrong rescale shows as an error of the output's own size.
PEAKY_KINDS = ("q4", "q8", "planted", "low_first", "partial_first")


def peaky_case(kind: str, heads: int, dim: int, lq: int, splits: list[int], seed: int):
    """float32 arrays of bf16 values q [lq, H, D], k, v [sum(splits), H, D].

    q4 / q8        Q ~ N(0, 16) / N(0, 64), K ~ N(0, 1) + per-channel offset
    planted        Q = N(0, 1) + 3 u_h (u_h a unit direction per head); one key
                   24 a u_h as the last key of the last segment (its weight is
                   about that of all other keys together)
    low_first      Q as planted, no planted key; the first 64 keys moved by
                   -16 a u_h and the next 64 by +16 a u_h (a low first tile,
                   then a high one)
    partial_first  as planted, with a first segment shorter than 32 keys
    with a = sqrt(D / 64), so that the logits (scaled by D^-1/2) do not
    depend on the head dim.
    """
    import torch

    n = sum(splits)
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(lq, heads, dim, generator=g)
    k = torch.randn(n, heads, dim, generator=g) + 0.5 * torch.randn(heads, dim, generator=g)
    v = 0.25 * torch.randn(n, heads, dim, generator=g)
    u = torch.randn(heads, dim, generator=g)
    u = u / u.norm(dim=-1, keepdim=True)
    if kind in ("q4", "q8"):
        q = z * (4.0 if kind == "q4" else 8.0)
    elif kind in ("planted", "low_first", "partial_first"):
        if kind == "partial_first" and splits[0] >= 32:
            raise ValueError("partial_first needs a first segment under 32 keys")
        q = z + 3.0 * u
        a = (dim / 64.0) ** 0.5
        if kind == "low_first":
            k[:64] -= 16.0 * a * u
            k[64:128] += 16.0 * a * u
        else:
            k[n - 1] = 24.0 * a * u
    else:
        raise ValueError(kind)
    return (bf16.round_f32(q.numpy()), bf16.round_f32(k.numpy()), bf16.round_f32(v.numpy()))


def rescale_rows_fraction(q: np.ndarray, k: np.ndarray, scale: float, first: int = 32) -> float:
    """Fraction of (row, head) pairs whose largest logit beyond the first
    ``first`` keys exceeds those keys' maximum by more than 8 in log2 units:
    the rows for which a kernel that starts its reference at its first
    sub-tile (the first 32 keys, or fewer when the first segment is shorter)
    must move it at least once."""
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(k, dtype=np.float64)
    hits = []
    for h in range(q64.shape[1]):
        s = q64[:, h] @ k64[:, h].T * (scale * LOG2E)
        hits.append(s[:, first:].max(axis=1) > s[:, :first].max(axis=1) + 8.0)
    return float(np.mean(np.stack(hits)))
