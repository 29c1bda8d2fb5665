"""Dense attention over the documents of a packed sequence.

``packed_sdpa`` is the drop-in for the reference's ``_packed_sdpa``
(src/taomate_hd/model/layers.py:202-255): the token refiner and non-streamed
forwards attend within each ``cu_seqlens`` document, non-causally, with SDPA
or FlashAttention-3.  Same arguments, validation and errors; the output is
``[tokens, heads, head_dim]`` bf16 in document order (empty documents add no
rows, as the reference's concatenation does).

Each non-empty document's K/V rows are packed once into one slot of a pooled
head-major buffer (at a 64-row-aligned offset, tile tail zeroed); one BF16
kernel launch per document then reads its query rows in place and writes its
output rows in place, with no per-document concatenation.
"""

from __future__ import annotations

from typing import Any

from . import _native
from .attention import segment_attention
from .slots import KV_TILE, SlotPool, SlotView, round_up

_POOLS: dict[tuple[str, int, int, int], SlotPool] = {}


def _pool(torch: Any, device: Any, heads: int, head_dim: int) -> SlotPool:
    """Slots per (device, stream, shape): a released slot is reused only by
    work queued after its readers on the same stream."""
    key = (str(torch.device(device)), _native.stream_ptr(torch, device), int(heads), int(head_dim))
    if key not in _POOLS:
        _POOLS[key] = SlotPool(torch, heads=heads, head_dim=head_dim, device=device)
    return _POOLS[key]


def packed_sdpa(q: Any, k: Any, v: Any, *, cu_seqlens: Any, cu_seqlens_host: tuple[int, ...] | None,
                max_seqlen: int, scale: float) -> Any:
    """Non-causal attention of each ``cu_seqlens`` document of ``q``/``k``/``v``
    (``[tokens, heads, head_dim]`` bf16 views, unit dim stride) over itself."""
    import torch

    bounds = (
        tuple(int(item) for item in cu_seqlens_host)
        if cu_seqlens_host is not None
        else tuple(int(item) for item in cu_seqlens.detach().cpu().tolist())
    )
    lengths = tuple(stop - start for start, stop in zip(bounds[:-1], bounds[1:]))
    if (
        len(bounds) < 2
        or bounds[0] != 0
        or bounds[-1] != int(q.shape[0])
        or any(length < 0 for length in lengths)
        or max_seqlen != max(lengths, default=0)
    ):
        raise ValueError("packed-attention cumulative lengths are invalid")
    docs = [(start, stop) for start, stop in zip(bounds[:-1], bounds[1:]) if stop > start]
    if not docs:
        raise ValueError("packed attention has no live segment")
    if q.ndim != 3 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("packed attention Q/K/V must share one [tokens, heads, head_dim] shape")
    _native.require_same_gpu(torch, q.device, q=q, k=k, v=v)
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"packed attention {name} must be bfloat16")
    heads, head_dim = int(q.shape[1]), int(q.shape[2])
    if k.stride() != v.stride():  # the pack kernel takes one stride pair for K and V
        k, v = k.contiguous(), v.contiguous()
    offsets, total = [], 0
    for start, stop in docs:
        offsets.append(total)
        total += round_up(stop - start, KV_TILE)
    pool = _pool(torch, q.device, heads, head_dim)
    slot = pool.acquire(total)
    try:
        for (start, stop), dst in zip(docs, offsets):
            slot.pack(k, v, row0=start, count=stop - start, dst=dst)
        out = torch.empty((int(q.shape[0]), heads, head_dim), dtype=torch.bfloat16, device=q.device)
        for (start, stop), dst in zip(docs, offsets):
            segment_attention(torch, q, [SlotView(slot, stop - start, dst)], scale=float(scale), backend="bf16",
                              q_row0=start, lq=stop - start, out=out, o_row0=start)
    finally:
        pool.release(slot)
    return out
