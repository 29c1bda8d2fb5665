"""Bit-exact bf16 <-> fp32 conversions in numpy (test infrastructure only).

bf16 is the upper half of an IEEE fp32; fp32 -> bf16 rounds to nearest even,
as torch's ``Tensor.to(torch.bfloat16)`` and the gfx950 ``v_cvt_pk_bf16_f32``
instruction do.  NaNs stay NaN.
"""

from __future__ import annotations

import numpy as np


def bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def round_f32(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16 value (returned as float32)."""
    return bits_to_f32(f32_to_bits(np.asarray(x, dtype=np.float32)))


def from_torch(tensor) -> np.ndarray:
    """bf16 torch tensor (any device) -> float32 numpy array (exact)."""
    import torch

    bits = tensor.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16)
    return bits_to_f32(bits)


def to_torch(x: np.ndarray, device=None):
    """float32 numpy array of bf16 values -> bf16 torch tensor (exact)."""
    import torch

    bits = f32_to_bits(np.asarray(x, dtype=np.float32)).view(np.int16)
    return torch.from_numpy(bits.copy()).view(torch.bfloat16).to(device)
