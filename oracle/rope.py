"""Q/K RMSNorm + RoPE (CPU restatement).

Test infrastructure only: tests and the bench's CPU baseline use it as the
checker; the product path never imports it.

Restates fused_qkv_qk_norm_rope_ / _merged_qkv_preprocess_kernel
(qkv_norm_rope), fused_qk_norm_rope / _qk_norm_rope_kernel (qk_norm_rope)
and fused_apply_rope / _rope_kernel (apply_rope, no norm),
src/taomate_hd/inference/fused_kernels.py:257-297, 385-472, 673-692 and
798-873, with the rounding helper _round_bf16 (:58-61).  For every token and
head, Q and K (not V) of the [tokens, 3 * heads * head_dim] bf16 buffer (or
one [tokens, heads, head_dim] projection) become

    normalized = bf16((x * rsqrt(mean(x^2) + eps)) * weight)
    rope       = bf16(bf16(normalized * cos) + bf16(rotate_half(normalized) * sin))

for the first rotary_dim channels (normalized for the rest).  The merged form
reads cos / sin at the token's position from a bf16 [positions, rotary_dim]
cache (cos in the first half of a row, sin in the second, channel d using
phase d % (rotary_dim / 2)); the one-projection form reads per-token,
per-channel tables cos[t][d], sin[t][d].

Two things the reference leaves to its compiler are fixed here and in the
HIP kernel:
  * the order of the sum of squares.  A row's head_dim channels are dealt to
    head_dim / 8 lanes of 8 channels each (lane_channels): lane j < rotary / 8
    holds the 4 channels at 4j and the 4 at rotary / 2 + 4j (a rotation pair
    per position), the remaining lanes hold 8 consecutive channels of the
    unrotated tail.  Each lane sums the squares of its channels in that order
    as a chain of fused multiply-adds (x0 * x0, then s + x * x rounded once),
    and the lane partials are added as a balanced pairwise tree in lane order
    ((l0 + l1) + (l2 + l3)) + ...;
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


def lane_channels(head_dim: int, rotary: int) -> np.ndarray:
    """[head_dim / 8, 8] channel indices of each lane of a row, in summation order."""
    half = rotary // 2
    lanes = []
    for j in range(head_dim // 8):
        if j < rotary // 8:
            lanes.append([4 * j + e for e in range(4)] + [half + 4 * j + e for e in range(4)])
        else:
            base = rotary + 8 * (j - rotary // 8)
            lanes.append(list(range(base, base + 8)))
    return np.array(lanes, dtype=np.int64)


def sum_squares(x: np.ndarray, rotary: int = 0) -> np.ndarray:
    """Sum of squares over the last axis (head_dim, a multiple of 8) in the
    fixed order for a row with the given rotary span."""
    x = np.asarray(x, dtype=np.float32)
    chunks = x[..., lane_channels(x.shape[-1], rotary)]  # [..., lanes, 8]
    part = chunks[..., 0] * chunks[..., 0]
    for e in range(1, 8):
        # fused multiply-add: x * x of a bf16 value is exact in float64 and the
        # float64 sum of it and a float32 partial rounds to float32 as one
        # rounding of the exact sum would (double rounding through a format
        # of 53 >= 2 * 24 + 2 bits is innocuous for addition)
        c = chunks[..., e].astype(np.float64)
        part = (part.astype(np.float64) + c * c).astype(np.float32)
    while part.shape[-1] > 1:
        part = part[..., 0::2] + part[..., 1::2]
    return part[..., 0]


def _norm_rope(x: np.ndarray, w: np.ndarray, cos_d: np.ndarray, sin_d: np.ndarray, rotary: int,
               eps: float) -> np.ndarray:
    """x [..., head_dim] (bf16 values as float32), w broadcastable to it,
    cos_d / sin_d broadcastable to [..., rotary] (channel d's cos and sin)."""
    head_dim = x.shape[-1]
    half = rotary // 2
    variance = sum_squares(x, rotary) / np.float32(head_dim)
    inv = np.float32(1.0) / np.sqrt(variance + np.float32(eps))
    normalized = round_bf16((x * inv[..., None]) * w)
    if rotary:
        d = np.arange(rotary)
        paired = normalized[..., np.where(d < half, d + half, d - half)]
        rotated = np.where(d < half, -paired, paired)
        cos = round_bf16(np.asarray(cos_d, dtype=np.float32))
        sin = round_bf16(np.asarray(sin_d, dtype=np.float32))
        rope = round_bf16(round_bf16(normalized[..., :rotary] * cos) + round_bf16(rotated * sin))
        normalized = np.concatenate([rope, normalized[..., rotary:]], -1)
    return normalized


def qkv_norm_rope(qkv: np.ndarray, q_weight: np.ndarray, k_weight: np.ndarray, cos_sin: np.ndarray,
                  positions: np.ndarray, eps: float, heads: int) -> np.ndarray:
    """Q/K of a merged [tokens, 3 * heads * head_dim] buffer (bf16 values as
    float32) normalized and rotated; V unchanged.  Returns a new array.
    fused_kernels.py:425-472, 824-873."""
    qkv = np.asarray(qkv, dtype=np.float32)
    tokens, width = qkv.shape
    head_dim = width // (3 * heads)
    rotary = int(cos_sin.shape[-1])
    half = rotary // 2
    out = qkv.copy()
    x = qkv[:, : 2 * heads * head_dim].reshape(tokens, 2, heads, head_dim)
    w = np.stack([np.asarray(q_weight, np.float32), np.asarray(k_weight, np.float32)])[None, :, None, :]
    cos_d = sin_d = None
    if rotary:
        phase = np.arange(rotary) % half
        rows = np.asarray(cos_sin, dtype=np.float32)[np.asarray(positions, dtype=np.int64)]  # [tokens, rotary]
        cos_d = rows[:, phase][:, None, None, :]
        sin_d = rows[:, half + phase][:, None, None, :]
    normalized = _norm_rope(x, w, cos_d, sin_d, rotary, eps)
    out[:, : 2 * heads * head_dim] = normalized.reshape(tokens, 2 * heads * head_dim)
    return out


def qk_norm_rope(value: np.ndarray, weight: np.ndarray, cos: np.ndarray, sin: np.ndarray,
                 eps: float) -> np.ndarray:
    """One projection [tokens, heads, head_dim] (bf16 values as float32)
    normalized and rotated with per-token tables cos / sin [tokens, rotary].
    fused_kernels.py:385-422, 798-821."""
    value = np.asarray(value, dtype=np.float32)
    rotary = int(np.asarray(cos).shape[-1])
    cos_d = np.asarray(cos, np.float32)[:, None, :] if rotary else None
    sin_d = np.asarray(sin, np.float32)[:, None, :] if rotary else None
    return _norm_rope(value, np.asarray(weight, np.float32), cos_d, sin_d, rotary, eps)


def apply_rope(value: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """The rotation alone on [tokens, heads, head_dim] (bf16 values as float32)
    with per-token tables cos / sin [tokens, rotary]: channel d < rotary
    becomes R(R(x[d] cos[d]) + R(r[d] sin[d])), r = rotate_half(x); the rest
    is kept.  fused_kernels.py:257-297, 673-692."""
    x = np.asarray(value, dtype=np.float32)
    rotary = int(np.asarray(cos).shape[-1])
    if not rotary:
        return x.copy()
    half = rotary // 2
    d = np.arange(rotary)
    paired = x[..., np.where(d < half, d + half, d - half)]
    rotated = np.where(d < half, -paired, paired)
    c = round_bf16(np.asarray(cos, np.float32))[:, None, :]
    s = round_bf16(np.asarray(sin, np.float32))[:, None, :]
    rope = round_bf16(round_bf16(x[..., :rotary] * c) + round_bf16(rotated * s))
    return np.concatenate([rope, x[..., rotary:]], -1)
