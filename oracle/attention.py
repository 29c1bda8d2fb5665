"""CPU restatement of the hook's attention backends (test infrastructure only).

* ``attention_fp64``   exact softmax(q k^T * scale) v in float64
* ``sdpa_cpu``         the reference's serial backend, torch SDPA on CPU fp32
* ``i8qk_attention``   the INT8-QK (SageAttention-style) arithmetic in float64
* ``i8qk_attention_cpu`` the same arithmetic in torch fp32 (the timed CPU baseline)
"""

from __future__ import annotations

import numpy as np

from . import quant


def attention_fp64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """Non-causal attention of token-major ``q [Lq, H, D]`` over ``k, v [N, H, D]``.

    Restates _sdpa_from_kv_parts, src/taomate_hd/streaming/attention_hook.py:100-115
    (SDPA with is_causal=False, dropout_p=0, explicit scale) in float64.
    Pinned by tests/test_oracle.py: N = 1 gives v; constant keys give mean(v);
    one dominant logit selects its value row; permuting keys changes nothing;
    splitting keys and merging by log-sum-exp equals the whole; matches torch
    SDPA on CPU.
    """
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(k, dtype=np.float64)
    v64 = np.asarray(v, dtype=np.float64)
    out = np.empty((q64.shape[0], q64.shape[1], v64.shape[2]), dtype=np.float64)
    for h in range(q64.shape[1]):
        s = (q64[:, h, :] @ k64[:, h, :].T) * float(scale)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h, :] = p @ v64[:, h, :]
    return out


def attention_lse_fp64(q: np.ndarray, k: np.ndarray, scale: float) -> np.ndarray:
    """Row log-sum-exp ``[Lq, H]`` of the scaled logits (natural log), float64."""
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(k, dtype=np.float64)
    lse = np.empty((q64.shape[0], q64.shape[1]), dtype=np.float64)
    for h in range(q64.shape[1]):
        s = (q64[:, h, :] @ k64[:, h, :].T) * float(scale)
        m = s.max(axis=1)
        lse[:, h] = m + np.log(np.exp(s - m[:, None]).sum(axis=1))
    return lse


def sdpa_cpu(q, k, v, scale: float):
    """The reference serial backend on CPU: torch SDPA in fp32 on [T, H, D] tensors.

    Same calls as attention_hook.py:107-115 (transpose to [1, H, T, D],
    is_causal=False, dropout_p=0), on CPU float32 tensors.  Used as the CPU
    baseline and as the fp32 reference of the INT8-QK cosine gate.
    """
    import torch
    import torch.nn.functional as F

    out = F.scaled_dot_product_attention(
        q.transpose(0, 1).unsqueeze(0),
        k.transpose(0, 1).unsqueeze(0),
        v.transpose(0, 1).unsqueeze(0),
        dropout_p=0.0,
        is_causal=False,
        scale=scale,
    )
    return out.squeeze(0).transpose(0, 1)


def i8qk_attention(q: np.ndarray, k_segments: list[np.ndarray], v_segments: list[np.ndarray], scale: float):
    """INT8-QK attention of ``q [Lq, H, D]`` over the given key/value segments.

    Restates the accelerated backend (attention_hook.py:335-371,
    sage_value_padding.py:79-97) with the INT8-QK workload's quantization: smooth-K mean
    over all keys of the call, per-128-block INT8 Q and K (K blocks restart at
    each segment), logits = (q_i8 . k_i8) * s_q * s_k * scale exactly, then a
    float64 softmax and P.V.  Returns (out [Lq, H, D] float64, operands dict).
    Pinned by tests/test_oracle.py (shift invariance of the smooth-K step:
    equals attention_fp64 of the dequantized operands with and without the
    mean; within quantization error of attention_fp64 of the inputs).
    """
    mean, kq, ks = quant.smooth_k_segments(k_segments)
    qq, qs = quant.block_quant(np.asarray(q, dtype=np.float32))
    lq, heads, _ = qq.shape
    out = np.empty((lq, heads, v_segments[0].shape[2]), dtype=np.float64)
    v_all = np.concatenate([np.asarray(v, dtype=np.float64) for v in v_segments], axis=0)
    qb = np.arange(lq) // quant.QUANT_BLOCK
    for h in range(heads):
        parts = []
        for kqi, ksi in zip(kq, ks):
            kb = np.arange(kqi.shape[0]) // quant.QUANT_BLOCK
            acc = qq[:, h, :].astype(np.float64) @ kqi[:, h, :].astype(np.float64).T
            parts.append(acc * qs[h, qb][:, None].astype(np.float64) * ksi[h, kb][None, :].astype(np.float64))
        s = np.concatenate(parts, axis=1) * float(scale)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h, :] = p @ v_all[:, h, :]
    return out, {"mean": mean, "k_i8": kq, "k_scale": ks, "q_i8": qq, "q_scale": qs}


def i8qk_attention_cpu(q, k_segments, v, scale: float):
    """The INT8-QK arithmetic on CPU torch fp32 tensors, as the timed CPU
    baseline of the quantized path: the same smooth-K mean and per-128-block
    quantization as ``i8qk_attention`` (fp32 mean of bf16 keys, rounded to
    bf16; q_i8 = sat(rint(x * (127 / amax)))), the integer Q.K^T in fp32 (exact:
    |q_i8 . k_i8| <= 127^2 * 128 < 2^24), then fp32 softmax and P.V.
    ``q [Lq, H, D]``, ``k_segments`` a list of ``[n_i, H, D]``, ``v [N, H, D]``
    (fp32 tensors holding bf16 values).  Returns ``[Lq, H, D]`` fp32.
    Pinned by tests/test_oracle.py against ``i8qk_attention`` (fp64).
    """
    import torch

    def block_quant(x):
        n, h, d = x.shape
        nb = (n + 127) // 128
        pad = torch.zeros((nb * 128 - n, h, d), dtype=x.dtype)
        xb = torch.cat([x, pad]).view(nb, 128, h, d)
        amax = xb.abs().amax(dim=(1, 3))  # [nb, H]
        # tensor / tensor: torch's scalar / tensor form is not correctly rounded on CPU
        inv = torch.where(amax > 0, torch.full_like(amax, 127.0) / amax, torch.zeros_like(amax))
        qi = torch.clamp(torch.round(xb * inv[:, None, :, None]), -128, 127)
        return qi.view(nb * 128, h, d)[:n], (amax / 127.0).repeat_interleave(128, 0)[:n]  # [n, H]

    keys = torch.cat(list(k_segments))
    mean = (keys.double().sum(0) / keys.shape[0]).float().to(torch.bfloat16).float()
    qq, qs = block_quant(q)
    parts = []
    for k in k_segments:
        kq, ks = block_quant(k - mean)
        parts.append((kq, ks))
    out = torch.empty_like(q)
    for h in range(q.shape[1]):
        logits = torch.cat([(qq[:, h] @ kq[:, h].T) * ks[None, :, h] for kq, ks in parts], dim=1)
        logits *= qs[:, h, None] * scale
        out[:, h] = torch.softmax(logits, dim=1) @ v[:, h]
    return out


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))
