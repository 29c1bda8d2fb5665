"""Q/K RMSNorm + RoPE in front of the hook.

``fused_qkv_qk_norm_rope_`` (in place in the merged QKV projection; the
``_stage_`` form also writes the chunk's K/V into a cache slot),
``fused_qk_norm_rope`` (one projection, new output) and ``fused_apply_rope``
(the rotation alone) have the reference's signatures, checks and error
messages (src/taomate_hd/inference/fused_kernels.py:673-692, 798-873) and
run the gfx950 kernels behind ``tmhd_qkv_norm_rope`` / ``tmhd_qk_norm_rope``
/ ``tmhd_apply_rope`` on the current stream.
The arithmetic and bf16 rounding follow the reference's Triton kernels
(``:385-472``); the order of the sum of squares and a correctly rounded
inverse square root are fixed where the reference leaves them to its
compiler (stated in include/tmhd.h).
"""

from __future__ import annotations

from typing import Any

from . import _native


def _merged_qkv_args(torch: Any, qkv: Any, q_weight: Any, k_weight: Any, cos_sin_cache: Any, positions: Any):
    """The reference's checks of the merged-projection form (fused_kernels.py:824-873)."""
    if qkv.ndim != 2 or not qkv.is_contiguous():
        raise ValueError("fused QKV preprocessing requires contiguous [tokens, width]")
    if q_weight.shape != k_weight.shape or q_weight.ndim != 1:
        raise ValueError("fused QKV Q/K norm weights differ")
    if any(value.dtype != torch.bfloat16 for value in (qkv, q_weight, k_weight, cos_sin_cache)):
        raise ValueError("fused QKV preprocessing requires BF16 tensors")
    tokens = int(qkv.shape[0])
    head_dim = int(q_weight.numel())
    projection_width, remainder = divmod(int(qkv.shape[-1]), 3)
    heads, head_remainder = divmod(projection_width, head_dim)
    if remainder or head_remainder:
        raise ValueError("fused QKV width does not contain three complete projections")
    positions = positions.reshape(-1).to(device=qkv.device, dtype=torch.int64).contiguous()
    if int(positions.numel()) != tokens:
        raise ValueError("fused QKV RoPE positions do not cover every token")
    cache = cos_sin_cache.contiguous()
    rotary_dim = int(cache.shape[-1])
    if cache.ndim != 2 or rotary_dim > head_dim or rotary_dim % 2:
        raise ValueError("fused QKV RoPE cache span is invalid")
    for name, t in (("qkv", qkv), ("q_weight", q_weight), ("k_weight", k_weight), ("cos_sin_cache", cache)):
        if t.device != qkv.device or t.device.type != "cuda":
            raise ValueError(f"{name} must be on the GPU of qkv")
    return tokens, heads, head_dim, positions, cache, rotary_dim, q_weight.contiguous(), k_weight.contiguous()


def fused_qkv_qk_norm_rope_(qkv: Any, q_weight: Any, k_weight: Any, cos_sin_cache: Any, positions: Any, eps: float) -> Any:
    """Normalize and rotate Q/K in place in a merged bf16 QKV projection.

    ``qkv`` is ``[tokens, 3 * heads * head_dim]`` (Q, K, V); V is not read or
    written.  ``cos_sin_cache`` is ``[positions, rotary_dim]`` bf16 (cos in the
    first half of a row, sin in the second) and ``positions`` holds one
    position per token.  Returns ``qkv``.
    """
    import torch

    tokens, heads, head_dim, positions, cache, rotary_dim, q_weight, k_weight = _merged_qkv_args(
        torch, qkv, q_weight, k_weight, cos_sin_cache, positions)
    status = _native.load().tmhd_qkv_norm_rope(
        _native.ptr(qkv), tokens, heads, head_dim, qkv.stride(0), _native.ptr(q_weight), _native.ptr(k_weight),
        _native.ptr(cache), cache.stride(0), int(cache.shape[0]), rotary_dim, _native.ptr(positions), float(eps),
        _native.stream_ptr(torch, qkv.device),
    )
    _native.check(status, "tmhd_qkv_norm_rope")
    return qkv


def fused_qkv_qk_norm_rope_stage_(qkv: Any, q_weight: Any, k_weight: Any, cos_sin_cache: Any, positions: Any,
                                  eps: float, slot: Any, *, row0: int = 0, count: int | None = None,
                                  dst: int = 0) -> Any:
    """``fused_qkv_qk_norm_rope_`` that also stages the chunk: the K and V of
    tokens ``row0 .. row0 + count`` land in ``slot`` (a ``KVSlot``) at rows
    ``dst ..``, exactly as ``slot.pack(k, v, row0=row0, count=count, dst=dst)``
    of the processed projection would put them, without a separate pass over
    K.  Returns ``qkv``."""
    import torch

    from .slots import KV_TILE, round_up

    tokens, heads, head_dim, positions, cache, rotary_dim, q_weight, k_weight = _merged_qkv_args(
        torch, qkv, q_weight, k_weight, cos_sin_cache, positions)
    if (slot.heads, slot.head_dim) != (heads, head_dim) or slot.device != qkv.device:
        raise ValueError(f"slot {(slot.heads, slot.head_dim)} on {slot.device} does not take this projection's K/V")
    n = tokens - int(row0) if count is None else int(count)
    if int(row0) < 0 or n < 0 or int(row0) + n > tokens:
        raise ValueError(f"rows [{row0}, {int(row0) + n}) outside the {tokens} tokens")
    dst = int(dst)
    if dst < 0 or dst % KV_TILE or dst + n > slot.capacity:
        raise ValueError(f"{n} rows at slot row {dst} do not fit the slot capacity {slot.capacity} (tile-aligned)")
    slot.key_sums.clear()
    status = _native.load().tmhd_qkv_norm_rope_stage(
        _native.ptr(qkv), tokens, heads, head_dim, qkv.stride(0), _native.ptr(q_weight), _native.ptr(k_weight),
        _native.ptr(cache), cache.stride(0), int(cache.shape[0]), rotary_dim, _native.ptr(positions), float(eps),
        int(row0), n, _native.ptr(slot.k), _native.ptr(slot.vt), slot.capacity * head_dim, slot.capacity * head_dim,
        slot.capacity, dst, dst + round_up(n, KV_TILE), _native.stream_ptr(torch, qkv.device),
    )
    _native.check(status, "tmhd_qkv_norm_rope_stage")
    slot.tokens = dst + n
    return qkv


def fused_qk_norm_rope(value: Any, weight: Any, cos: Any, sin: Any, eps: float) -> Any:
    """RMSNorm + RoPE of one projection ``value [tokens, heads, head_dim]``
    (bf16; rows may be strided, e.g. the Q or K view of a merged projection)
    into a new contiguous bf16 tensor.  ``cos`` / ``sin`` are
    ``[tokens, rotary_dim]`` per-channel tables; a float dtype other than
    bf16 is rounded to bf16 first, which is the reference kernel's own
    rounding of them (``_round_bf16`` on load).  ``weight`` must be bf16: the
    reference uses a wider weight unrounded, which this kernel does not.
    """
    import torch

    tokens, heads, head_dim = value.shape
    rotary_dim = int(cos.shape[-1])
    if rotary_dim > head_dim or rotary_dim % 2:
        raise ValueError("SOL QKNorm/RoPE requires an even rotary span within a head")
    if value.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("fused QK norm/RoPE requires a BF16 value and weight")
    if weight.ndim != 1 or int(weight.numel()) != head_dim:
        raise ValueError("fused QK norm weight does not match head_dim")
    if value.stride(-1) != 1 or value.stride(1) != head_dim:
        value = value.contiguous()
    if int(cos.numel()) != tokens * rotary_dim or int(sin.numel()) != tokens * rotary_dim:
        raise ValueError("fused QK RoPE tables do not cover every token")
    cos = cos.to(torch.bfloat16).reshape(tokens, rotary_dim).contiguous()
    sin = sin.to(torch.bfloat16).reshape(tokens, rotary_dim).contiguous()
    for name, t in (("value", value), ("weight", weight), ("cos", cos), ("sin", sin)):
        if t.device != value.device or t.device.type != "cuda":
            raise ValueError(f"{name} must be on the GPU of value")
    weight = weight.contiguous()
    out = torch.empty((tokens, heads, head_dim), dtype=torch.bfloat16, device=value.device)
    status = _native.load().tmhd_qk_norm_rope(
        _native.ptr(value), tokens, heads, head_dim, value.stride(0), _native.ptr(out), out.stride(0),
        _native.ptr(weight), _native.ptr(cos), cos.stride(0), _native.ptr(sin), sin.stride(0), rotary_dim,
        float(eps), _native.stream_ptr(torch, value.device),
    )
    _native.check(status, "tmhd_qk_norm_rope")
    return out


def fused_apply_rope(value: Any, cos: Any, sin: Any) -> Any:
    """The rotation alone (no RMSNorm) of ``value [tokens, heads, head_dim]``
    bf16 with per-token tables ``cos`` / ``sin`` ``[tokens, rotary_dim]``, into a
    new contiguous bf16 tensor (fused_kernels.py:257-297, 673-692).  Wider
    tables are rounded to bf16 first, as the reference kernel does on load."""
    import torch

    tokens, heads, head_dim = value.shape
    rotary_dim = int(cos.shape[-1])
    if value.dtype != torch.bfloat16:
        raise ValueError("fused RoPE requires a BF16 value")
    if rotary_dim > head_dim or rotary_dim % 2:
        raise ValueError("fused RoPE requires an even rotary span within a head")
    if value.stride(-1) != 1 or value.stride(1) != head_dim:
        value = value.contiguous()
    if int(cos.numel()) != tokens * rotary_dim or int(sin.numel()) != tokens * rotary_dim:
        raise ValueError("fused RoPE tables do not cover every token")
    cos = cos.to(torch.bfloat16).reshape(tokens, rotary_dim).contiguous()
    sin = sin.to(torch.bfloat16).reshape(tokens, rotary_dim).contiguous()
    for name, t in (("value", value), ("cos", cos), ("sin", sin)):
        if t.device != value.device or t.device.type != "cuda":
            raise ValueError(f"{name} must be on the GPU of value")
    out = torch.empty((tokens, heads, head_dim), dtype=torch.bfloat16, device=value.device)
    status = _native.load().tmhd_apply_rope(
        _native.ptr(value), tokens, heads, head_dim, value.stride(0), _native.ptr(out), out.stride(0),
        _native.ptr(cos), cos.stride(0), _native.ptr(sin), sin.stride(0), rotary_dim,
        _native.stream_ptr(torch, value.device),
    )
    _native.check(status, "tmhd_apply_rope")
    return out
