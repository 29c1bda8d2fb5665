"""Q/K RMSNorm + RoPE inside a merged QKV projection (CPU restatement).

Test infrastructure only: tests and the bench's CPU baseline use it as the
checker; the product path never imports it.

Restates fused_qkv_qk_norm_rope_ / _merged_qkv_preprocess_kernel,
src/taomate_hd/inference/fused_kernels.py:425-472 and 826-873, with the
rounding helper _round_bf16 (:58-61).  For every token and head, Q and K
(not V) of the [tokens, 3 * heads * head_dim] bf16 buffer become

    normalized = bf16((x * rsqrt(mean(x^2) + eps)) * weight)
    rope       = bf16(bf16(normalized * cos) + bf16(rotate_half(normalized) * sin))

for the first rotary_dim channels (normalized for the rest), with cos / sin
read at the token's position from a bf16 [positions, rotary_dim] cache
(cos in the first half of a row, sin in the second, channel d using
phase d % (rotary_dim / 2)).

Two things the reference leaves to its compiler are fixed here and in the
HIP kernel:
  * the order of the sum of squares: partial sums over 8 consecutive
    channels (in channel order), then a butterfly over the partials
    (partner index i ^ k for k = n/2, ..., 1);
  * the inverse RMS: 1 / sqrt(variance + eps) with a correctly rounded
    square root and division (the reference's tl.rsqrt is the GPU's
    approximate reciprocal square root).
Parity with the reference is therefore exact up to those two points; see
the pinning tests in tests/test_oracle.py.
"""

from __future__ import annotations

import numpy as np


def round_bf16(x: np.ndarray) -> np.ndarray:
    """The reference's _round_bf16 (fused_kernels.py:58-61): on the fp32 bits,
    add 0x7FFF plus bit 16 (wrapping mod 2^32), then clear the low 16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return (u & 0xFFFFFFFF).astype(np.uint32).view(np.float32)


def sum_squares(x: np.ndarray) -> np.ndarray:
    """Sum of squares over the last axis (a multiple of 8) in the fixed order."""
    x = np.asarray(x, dtype=np.float32)
    n = x.shape[-1] // 8
    chunks = x.reshape(*x.shape[:-1], n, 8)
    part = chunks[..., 0] * chunks[..., 0]
    for e in range(1, 8):
        part = part + chunks[..., e] * chunks[..., e]
    k = n // 2
    idx = np.arange(n)
    while k >= 1:
        part = part + part[..., idx ^ k]
        k //= 2
    return part[..., 0]


def qkv_norm_rope(qkv: np.ndarray, q_weight: np.ndarray, k_weight: np.ndarray, cos_sin: np.ndarray,
                  positions: np.ndarray, eps: float, heads: int) -> np.ndarray:
    """Q/K of a merged [tokens, 3 * heads * head_dim] buffer (bf16 values as
    float32) normalized and rotated; V unchanged.  Returns a new array."""
    qkv = np.asarray(qkv, dtype=np.float32)
    tokens, width = qkv.shape
    head_dim = width // (3 * heads)
    rotary = int(cos_sin.shape[-1])
    half = rotary // 2
    out = qkv.copy()
    x = qkv[:, : 2 * heads * head_dim].reshape(tokens, 2, heads, head_dim)
    variance = sum_squares(x) / np.float32(head_dim)
    inv = np.float32(1.0) / np.sqrt(variance + np.float32(eps))
    w = np.stack([np.asarray(q_weight, np.float32), np.asarray(k_weight, np.float32)])[None, :, None, :]
    normalized = round_bf16((x * inv[..., None]) * w)
    d = np.arange(head_dim)
    rot = d < rotary
    if rotary:
        partner = np.where(d < half, d + half, d - half)
        paired = normalized[..., np.where(rot, partner, d)]
        rotated = np.where(d < half, -paired, paired)
        phase = d % half
        rows = np.asarray(cos_sin, dtype=np.float32)[np.asarray(positions, dtype=np.int64)]  # [tokens, rotary]
        cos = round_bf16(rows[:, np.where(rot, phase, 0)])[:, None, None, :]
        sin = round_bf16(rows[:, np.where(rot, half + phase, 0)])[:, None, None, :]
        rope = round_bf16(round_bf16(normalized * cos) + round_bf16(rotated * sin))
        normalized = np.where(rot, rope, normalized)
    out[:, : 2 * heads * head_dim] = normalized.reshape(tokens, 2 * heads * head_dim)
    return out
