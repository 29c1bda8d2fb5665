"""Ulysses sequence <-> heads layouts either side of the streaming attention
(src/taomate_hd/distributed/ulysses_layout.py and the inference paths of
distributed/ulysses.py:113-212), on the gfx950 kernels behind
``tmhd_ulysses_*``.

A rank holds ``T`` tokens with all ``H`` heads; one all-to-all over the
Ulysses group gives it all ``U * T`` tokens of ``L = ceil(H / U)`` heads
(padded heads are zero), and a second one brings the attention output back.
The collective itself is the caller's (``torch.distributed.all_to_all_single``
over RCCL on a multi-GPU node); these functions build and read its buffers:

* ``qkv_send_layout`` / ``attention_receive_layout``: the reference's two
  layout functions, same names, arguments and results;
* ``qkv_receive_layout``: the reference's ``movedim(0, 1).contiguous()`` of the
  received QKV, as a merged ``[U * T, 3 * L * D]`` projection;
* ``token_major=True`` sends ``[U, T, 3, L, D]`` instead, whose received
  buffer already is that merged projection (``qkv_received_views``: zero
  copies);
* ``qkv_norm_rope_send_layout``: Q/K RMSNorm + RoPE of the merged projection
  written straight into the send buffer;
* ``merged_qkv_sequence_to_heads`` / ``heads_to_sequence``: both directions
  around a given ``all_to_all(output, input)`` callable.
"""

from __future__ import annotations

from typing import Any, Callable

from . import _native


def _local_heads(num_heads: int, world_size: int) -> int:
    if int(world_size) < 1:
        raise ValueError("Ulysses world size must be positive")
    return (int(num_heads) + int(world_size) - 1) // int(world_size)


def _check_merged(torch: Any, value: Any, num_heads: int, head_dim: int) -> None:
    _native.require_device_tensor(torch, value, "value")
    if value.dtype != torch.bfloat16 or value.ndim != 2 or value.stride(1) != 1:
        raise ValueError("merged QKV must be a [tokens, 3 * heads * head_dim] bf16 view with unit column stride")
    if int(value.shape[1]) != 3 * int(num_heads) * int(head_dim):
        raise ValueError("merged QKV width differs from heads * head_dim")


def qkv_send_layout(value: Any, *, num_heads: int, head_dim: int, world_size: int, token_major: bool = False,
                    out: Any | None = None) -> Any:
    """Send buffer ``[U, 3, T, L, D]`` (``token_major``: ``[U, T, 3, L, D]``) of
    the merged projection ``value [T, 3 * H * D]`` (ulysses_layout.py:34-41)."""
    import torch

    _check_merged(torch, value, num_heads, head_dim)
    tokens, local = int(value.shape[0]), _local_heads(num_heads, world_size)
    shape = (world_size, tokens, 3, local, head_dim) if token_major else (world_size, 3, tokens, local, head_dim)
    if out is None:
        out = torch.empty(shape, dtype=value.dtype, device=value.device)
    elif tuple(out.shape) != shape or out.dtype != value.dtype or not out.is_contiguous():
        raise ValueError(f"send buffer must be a contiguous bf16 {shape}")
    _native.require_same_gpu(torch, value.device, out=out)
    lib = _native.load()
    _native.check(lib.tmhd_ulysses_qkv_send(_native.ptr(value), value.stride(0), tokens, int(num_heads),
                                            int(head_dim), int(world_size), 1 if token_major else 0,
                                            _native.ptr(out), _native.stream_ptr(torch, value.device)),
                  "tmhd_ulysses_qkv_send")
    return out


def qkv_norm_rope_send_layout(qkv: Any, q_weight: Any, k_weight: Any, cos_sin_cache: Any, positions: Any,
                              eps: float, *, world_size: int, token_major: bool = False,
                              out: Any | None = None) -> Any:
    """``fused_qkv_qk_norm_rope_`` then ``qkv_send_layout`` in one pass over Q and
    K (fused_kernels.py:824-873 then ulysses.py:183-212): the normalised,
    rotated rows go to the send buffer, ``qkv`` itself is not modified.
    Bit-identical to the two steps."""
    import torch

    from .rope import _merged_qkv_args

    tokens, heads, head_dim, positions, cache, rotary_dim, q_weight, k_weight = _merged_qkv_args(
        torch, qkv, q_weight, k_weight, cos_sin_cache, positions)
    local = _local_heads(heads, world_size)
    shape = (world_size, tokens, 3, local, head_dim) if token_major else (world_size, 3, tokens, local, head_dim)
    if out is None:
        out = torch.empty(shape, dtype=qkv.dtype, device=qkv.device)
    elif tuple(out.shape) != shape or out.dtype != qkv.dtype or not out.is_contiguous():
        raise ValueError(f"send buffer must be a contiguous bf16 {shape}")
    _native.require_same_gpu(torch, qkv.device, out=out)
    lib = _native.load()
    _native.check(lib.tmhd_ulysses_qkv_norm_rope_send(
        _native.ptr(qkv), qkv.stride(0), tokens, heads, head_dim, _native.ptr(q_weight), _native.ptr(k_weight),
        _native.ptr(cache), cache.stride(0), int(cache.shape[0]), rotary_dim, _native.ptr(positions), float(eps),
        int(world_size), 1 if token_major else 0, _native.ptr(out), _native.stream_ptr(torch, qkv.device),
    ), "tmhd_ulysses_qkv_norm_rope_send")
    return out


def qkv_receive_layout(received: Any, out: Any | None = None) -> Any:
    """The received layout-0 buffer ``[U, 3, T, L, D]`` as the merged projection
    ``[U * T, 3 * L * D]`` of the rank's heads (the reference's
    ``outputs.movedim(0, 1).contiguous()``, ulysses.py:209-211, row-merged)."""
    import torch

    if (received.ndim != 5 or int(received.shape[1]) != 3 or not received.is_contiguous()
            or received.dtype != torch.bfloat16):
        raise ValueError("received QKV must be a contiguous bf16 [world, 3, tokens, local_heads, head_dim] buffer")
    world, _, tokens, local, head_dim = (int(v) for v in received.shape)
    if out is None:
        out = torch.empty((world * tokens, 3 * local * head_dim), dtype=received.dtype, device=received.device)
    elif (tuple(out.shape) != (world * tokens, 3 * local * head_dim) or out.stride(1) != 1
            or out.dtype != torch.bfloat16):
        raise ValueError("out must be a bf16 [world * tokens, 3 * local_heads * head_dim] view with unit column stride")
    _native.require_device_tensor(torch, received, "received")
    _native.require_same_gpu(torch, received.device, out=out)
    lib = _native.load()
    _native.check(lib.tmhd_ulysses_qkv_receive(_native.ptr(received), tokens, local, head_dim, world,
                                               _native.ptr(out), out.stride(0),
                                               _native.stream_ptr(torch, received.device)),
                  "tmhd_ulysses_qkv_receive")
    return out


def qkv_received_views(merged: Any, *, local_heads: int, head_dim: int) -> tuple[Any, Any, Any]:
    """Q, K, V ``[U * T, L, D]`` views of a received merged projection (the
    token-major layout's received buffer viewed as ``[U * T, 3 * L * D]``, or
    ``qkv_receive_layout``'s result); no copy."""
    rows = int(merged.shape[0])
    flat = merged.reshape(rows, 3, int(local_heads), int(head_dim))
    return flat[:, 0], flat[:, 1], flat[:, 2]


def attention_receive_layout(value: Any, *, num_heads: int, out: Any | None = None) -> Any:
    """Received attention output ``[U, T, L, D]`` -> ``[T, num_heads, D]``
    (ulysses_layout.py:59-67); ``out`` may be any token-major view."""
    import torch

    if value.ndim != 4 or not value.is_contiguous() or value.dtype != torch.bfloat16:
        raise ValueError("received attention output must be a contiguous bf16 [world, tokens, local_heads, dim]")
    world, tokens, local, dim = (int(v) for v in value.shape)
    if _local_heads(num_heads, world) != local:
        raise ValueError(f"{num_heads} heads over {world} ranks do not give {local} local heads")
    if out is None:
        out = torch.empty((tokens, int(num_heads), dim), dtype=value.dtype, device=value.device)
    elif tuple(out.shape) != (tokens, int(num_heads), dim) or out.stride(2) != 1 or out.dtype != torch.bfloat16:
        raise ValueError("out must be a bf16 [tokens, heads, dim] view with unit dim stride")
    _native.require_device_tensor(torch, value, "value")
    _native.require_same_gpu(torch, value.device, out=out)
    lib = _native.load()
    _native.check(lib.tmhd_ulysses_attention_receive(_native.ptr(value), tokens, int(num_heads), dim, world,
                                                     _native.ptr(out), out.stride(0), out.stride(1),
                                                     _native.stream_ptr(torch, value.device)),
                  "tmhd_ulysses_attention_receive")
    return out


def merged_qkv_sequence_to_heads(value: Any, *, num_heads: int, head_dim: int, world_size: int,
                                 all_to_all: Callable[[Any, Any], Any], token_major: bool = True,
                                 norm_rope: tuple[Any, ...] | None = None) -> tuple[Any, Any, Any]:
    """Exchange a merged projection ``[T, 3 * H * D]`` for ``U * T`` tokens of the
    rank's ``L`` heads (ulysses.py:183-212): returns Q, K, V ``[U * T, L, D]``.

    ``all_to_all(output, input)`` performs the collective on the flat send
    buffer (``torch.distributed.all_to_all_single`` over the Ulysses group).
    With ``token_major`` the received buffer is read in place; otherwise it is
    reordered as the reference does.  ``norm_rope = (q_weight, k_weight,
    cos_sin_cache, positions, eps)`` also applies the Q/K RMSNorm + RoPE on
    the way into the send buffer."""
    import torch

    local = _local_heads(num_heads, world_size)
    if norm_rope is not None:
        send = qkv_norm_rope_send_layout(value, *norm_rope, world_size=world_size, token_major=token_major)
    else:
        send = qkv_send_layout(value, num_heads=num_heads, head_dim=head_dim, world_size=world_size,
                               token_major=token_major)
    received = torch.empty_like(send)
    all_to_all(received, send)
    tokens = int(value.shape[0])
    if token_major:
        merged = received.view(world_size * tokens, 3 * local * head_dim)
    else:
        merged = qkv_receive_layout(received)
    return qkv_received_views(merged, local_heads=local, head_dim=head_dim)


def heads_to_sequence(value: Any, *, num_heads: int, world_size: int, all_to_all: Callable[[Any, Any], Any],
                      out: Any | None = None) -> Any:
    """The attention output ``[U * T, L, D]`` of the rank's heads back to its
    ``T`` tokens with all ``num_heads`` heads (ulysses.py:113-138)."""
    import torch

    rows, local, dim = (int(v) for v in value.shape)
    if rows % world_size:
        raise ValueError("attention rows are not a multiple of the Ulysses world size")
    send = value.contiguous().view(world_size, rows // world_size, local, dim)
    received = torch.empty_like(send)
    all_to_all(received, send)
    return attention_receive_layout(received, num_heads=num_heads, out=out)
