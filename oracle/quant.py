"""CPU restatement of the INT8 arithmetic on the W8A8 and INT8-QK paths.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

All inputs are float32 arrays holding bf16 values (see oracle.bf16).  The
rounding steps are written out one operation at a time in float32, the order
the HIP kernels use, so results are comparable bit for bit.
"""

from __future__ import annotations

import numpy as np

from . import bf16

F32 = np.float32


def token_quant(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-token dynamic symmetric INT8 quantization of ``x [M, K]``.

    Restates vLLM ``dynamic_scaled_int8_quant`` as called at
    src/taomate_hd/inference/w8a8.py:71 (and ``scaled_int8_quant`` at :141):
      scale[m] = amax_m / 127 (fp32),  q = sat_int8(rint(x * (127 / amax_m)))
    The vLLM source is not in the container; the formula is the one recalled
    from its public kernel and stated in include/tmhd.h.
    amax = 0 gives scale 0 and q 0.
    Pinned by tests/test_oracle.py (closed forms: max element -> +-127, error
    bound <= scale/2, ties to even, zero rows).
    """
    x = np.asarray(x, dtype=F32)
    amax = np.max(np.abs(x), axis=1).astype(F32)
    scale = (amax / F32(127.0)).astype(F32)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, F32(127.0) / amax, F32(0.0)).astype(F32)
    y = (x * inv[:, None]).astype(F32)
    q = np.clip(np.rint(y), -128, 127).astype(np.int8)
    return q, scale


def weight_quant(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Static per-output-channel INT8 weight quantization of ``w [N, K]``.

    Restates _quantize_cutlass_w8a8_weight, src/taomate_hd/inference/w8a8.py:175-179:
      scale = clamp(amax_row(|W|).float() / 127, min=1e-12)
      q = clamp(round(W / scale), -127, 127).int8      (round = half to even)
    Pinned by tests/test_oracle.py (max element -> +-127, |W/scale - q| <= 1/2,
    ties to even, clamp at -127, tiny rows use the 1e-12 floor).
    """
    w = np.asarray(w, dtype=F32)
    amax = np.max(np.abs(w), axis=1).astype(F32)
    scale = np.maximum((amax / F32(127.0)).astype(F32), F32(1e-12)).astype(F32)
    y = (w / scale[:, None]).astype(F32)
    q = np.clip(np.rint(y), -127, 127).astype(np.int8)
    return q, scale


def int_gemm(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Exact int32 accumulators ``acc[m][n] = sum_k a[m][k] * b[n][k]``.

    The accumulation inside cutlass_scaled_mm (w8a8.py:72, :142-144).  fp64
    matmul of integer-valued operands is exact while |acc| < 2^53; for INT8
    operands |acc| <= 128^2 * K, far below that for any K used here.
    Pinned by tests/test_oracle.py (brute-force loops on small shapes).
    """
    a64 = np.asarray(a, dtype=np.float64)
    b64 = np.asarray(b, dtype=np.float64)
    acc = a64 @ b64.T
    return acc.astype(np.int64).astype(np.int32)


def scaled_mm_epilogue(acc: np.ndarray, a_scale: np.ndarray, b_scale: np.ndarray, bias: np.ndarray | None) -> np.ndarray:
    """bf16(float(acc) * b_scale[n] * a_scale[m] + bias[n]), fp32, left to right.

    The dequantization of cutlass_scaled_mm (w8a8.py:72) with the bf16 bias
    term of the projection's epilogue.  Returns float32 values of the bf16
    result.  Pinned by tests/test_oracle.py (unit scales return acc rounded to
    bf16; bias-only and power-of-two scale cases).
    """
    t = np.asarray(acc).astype(F32)
    t = (t * np.asarray(b_scale, dtype=F32)[None, :]).astype(F32)
    t = (t * np.asarray(a_scale, dtype=F32)[:, None]).astype(F32)
    if bias is not None:
        t = (t + np.asarray(bias, dtype=F32)[None, :]).astype(F32)
    return bf16.round_f32(t)


# ---------------------------------------------------------------------------
# INT8-QK (SageAttention-style) operands.

MEAN_FIX = 2.0 ** 24
QUANT_BLOCK = 128


def smooth_k_mean(k: np.ndarray) -> np.ndarray:
    """bf16 token-mean of keys ``k [N, H, D]`` -> ``[H, D]`` (float32 bf16 values).

    Restates ``mean = k.mean(dim=1, keepdim=True)`` on the bf16 concatenated
    keys, src/taomate_hd/inference/sage_value_padding.py:89.  The sum is exact
    (int64 fixed point: rint(x * 2^24)) so it does not depend on summation
    order; mean = bf16(fp32(sum * 2^-24 / N)).
    Pinned by tests/test_oracle.py (constant keys give that constant; the
    fixed-point sum equals the fp64 sum for bf16 inputs of moderate range).
    """
    k = np.asarray(k, dtype=F32)
    fixed = np.rint((k * F32(MEAN_FIX)).astype(F32)).astype(np.int64)
    total = fixed.sum(axis=0)  # exact
    n = k.shape[0]
    mean = (total.astype(np.float64) / (float(n) * MEAN_FIX)).astype(F32)
    return bf16.round_f32(mean)


def block_quant(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-(128-row block, head) symmetric INT8 quantization of ``x [N, H, D]``.

    SageAttention's per-block INT8 Q/K quantization
    (sage_value_padding.py:90-92 calls its per-thread variant; the INT8-QK
    workload fixes 128-token blocks).  Formula stated in include/tmhd.h:
      scale = amax / 127,  q = sat_int8(rint(x * (127 / amax))),  amax = 0 -> 0.
    Returns q [N, H, D] int8 and scale [H, ceil(N / 128)] float32.
    Pinned by tests/test_oracle.py (as token_quant, per block).
    """
    x = np.asarray(x, dtype=F32)
    n, h, d = x.shape
    nblk = (n + QUANT_BLOCK - 1) // QUANT_BLOCK
    q = np.zeros((n, h, d), dtype=np.int8)
    scale = np.zeros((h, nblk), dtype=F32)
    for b in range(nblk):
        blk = x[b * QUANT_BLOCK : (b + 1) * QUANT_BLOCK]  # [r, H, D]
        amax = np.max(np.abs(blk), axis=(0, 2)).astype(F32)  # [H]
        scale[:, b] = (amax / F32(127.0)).astype(F32)
        with np.errstate(divide="ignore"):
            inv = np.where(amax > 0, F32(127.0) / amax, F32(0.0)).astype(F32)
        y = (blk * inv[None, :, None]).astype(F32)
        q[b * QUANT_BLOCK : (b + 1) * QUANT_BLOCK] = np.clip(np.rint(y), -128, 127).astype(np.int8)
    return q, scale


def smooth_k_segments(segments: list[np.ndarray]) -> tuple[np.ndarray, list[np.ndarray], list[np.ndarray]]:
    """Smooth-K quantization of a call's key segments ([n_i, H, D] each).

    The mean is taken over every key of the call (the concatenation the
    reference builds at attention_hook.py:336-345); each segment is then
    block-quantized on its own 128-token blocks, x = fp32(k) - fp32(mean).
    Returns (mean [H, D], [q_i], [scale_i]).
    """
    mean = smooth_k_mean(np.concatenate(segments, axis=0))
    qs, ss = [], []
    for k in segments:
        q, s = block_quant((np.asarray(k, dtype=F32) - mean[None]).astype(F32))
        qs.append(q)
        ss.append(s)
    return mean, qs, ss
