"""Row-wise RMSNorm / AdaLN-modulate / residual-gate ops (CPU restatement).

Test infrastructure only: tests and the bench's CPU baseline use it as the
checker; the product path never imports it.

Restates the SOL fused kernels of src/taomate_hd/inference/fused_kernels.py:
_modulate_kernel / fused_modulate (:221-237, 643-656), _gate_add_kernel /
fused_gate_add (:239-255, 658-671), _rms_norm_kernel / fused_rms_norm
(:312-321, 706-721), _rms_norm_modulate_kernel / fused_rms_norm_modulate
(:323-348, 723-755) and _residual_gate_rms_norm_modulate_kernel /
fused_residual_gate_rms_norm_modulate (:350-383, 757-796), and
_swiglu_kernel / fused_swiglu (:299-310, 694-704), with R() the
reference's _round_bf16 (:58-61).  Inputs are bf16 values held as float32.

Fixed here where the reference leaves it to its compiler (and matched by the
HIP kernels): the sum of squares of a row deals its 8-column chunks to 64
partials (chunk c to partial c % 64), each a chain of fused multiply-adds
over its chunks in order (8 columns in order), then adds the partials as a
pairwise tree in order; the inverse RMS is 1 / sqrt(sum / cols + eps) with a
correctly rounded square root and divisions.
"""

from __future__ import annotations

import numpy as np

from .rope import round_bf16

LANES = 64


def sum_squares_row(x: np.ndarray) -> np.ndarray:
    """Sum of squares over the last axis (a multiple of 8) in the fixed order."""
    x = np.asarray(x, dtype=np.float32)
    cols = x.shape[-1]
    nch = cols // 8
    rounds = -(-nch // LANES)
    padded = np.zeros((*x.shape[:-1], rounds * LANES * 8), np.float32)
    padded[..., :cols] = x
    chunks = padded.reshape(*x.shape[:-1], rounds, LANES, 8)  # chunk c = lane + 64 * round
    part = chunks[..., 0, :, 0] * chunks[..., 0, :, 0]
    for i in range(rounds):
        for e in range(8):
            if i == 0 and e == 0:
                continue
            # fused multiply-add (x * x exact in float64; one rounding of the
            # float64 sum to float32 equals one rounding of the exact sum);
            # zero padding adds +0, which changes nothing
            c = chunks[..., i, :, e].astype(np.float64)
            part = (part.astype(np.float64) + c * c).astype(np.float32)
    while part.shape[-1] > 1:
        part = part[..., 0::2] + part[..., 1::2]
    return part[..., 0]


def inverse_rms(x: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    variance = sum_squares_row(x) / np.float32(x.shape[-1])
    return np.float32(1.0) / np.sqrt(variance + np.float32(eps))


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """fused_rms_norm: R((x * inv) * w) (the .to(bfloat16) store rounds to nearest even)."""
    x = np.asarray(x, dtype=np.float32)
    return round_bf16((x * inverse_rms(x, eps)[..., None]) * np.asarray(weight, np.float32))


def modulate(x: np.ndarray, scale: np.ndarray, shift: np.ndarray, index: np.ndarray) -> np.ndarray:
    """R(R(x * R(1 + scale[t])) + shift[t]), t = index[row]."""
    x = np.asarray(x, dtype=np.float32)
    sc = np.asarray(scale, np.float32)[np.asarray(index, np.int64)]
    sh = np.asarray(shift, np.float32)[np.asarray(index, np.int64)]
    return round_bf16(round_bf16(x * round_bf16(np.float32(1.0) + sc)) + sh)


def gate_add(residual: np.ndarray, gate: np.ndarray, branch: np.ndarray, index: np.ndarray) -> np.ndarray:
    """R(residual + R(gate[t] * branch))."""
    g = np.asarray(gate, np.float32)[np.asarray(index, np.int64)]
    return round_bf16(np.asarray(residual, np.float32) + round_bf16(g * np.asarray(branch, np.float32)))


def rms_norm_modulate(x: np.ndarray, weight: np.ndarray, scale: np.ndarray, shift: np.ndarray, index: np.ndarray,
                      eps: float) -> np.ndarray:
    return modulate(rms_norm(x, weight, eps), scale, shift, index)


def residual_gate_rms_norm_modulate(residual: np.ndarray, branch: np.ndarray, gate: np.ndarray, weight: np.ndarray,
                                    scale: np.ndarray, shift: np.ndarray, index: np.ndarray,
                                    eps: float) -> tuple[np.ndarray, np.ndarray]:
    hidden = gate_add(residual, gate, branch, index)
    return hidden, rms_norm_modulate(hidden, weight, scale, shift, index, eps)


def swiglu(x: np.ndarray) -> np.ndarray:
    """R(R(g * s) * u) over the halves (gate | up) of the last axis, with
    s = sigmoid(g) evaluated in float64 and rounded to float32 (the reference's
    tl.sigmoid is its compiler's approximation: parity within one bf16 ulp).
    fused_kernels.py:299-310, 694-704."""
    x = np.asarray(x, dtype=np.float32)
    half = x.shape[-1] // 2
    g, u = x[..., :half], x[..., half:]
    s = (1.0 / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32)
    return round_bf16(round_bf16(g * s) * u)
