"""Head-major K/V slots: the storage unit of the streaming KV cache.

A slot holds one block of keys and values for one layer:

* ``k``  bf16 ``[H, cap, D]``  - key row ``t`` of head ``h`` is ``k[h, t]``;
* ``vt`` bf16 ``[H, D, cap]``  - values transposed; token ``t`` sits at column
  ``vt_position(t)`` (the middle two 4-token chunks of every 16-token group
  swapped), which is the order one MFMA lane consumes in ``P . V``.

``cap`` is a multiple of 64 (the kernels' key tile) and rows ``[tokens,
round_up(tokens, 64))`` are kept zero, so a tile never reads stale data.
Slots are filled only by ``tmhd_kv_pack`` (``KVSlot.pack``) and the staged
norm + RoPE, which also drop the slot's memo of key sums (``key_sums``, kept
for the INT8-QK smooth-K mean); attention reads them in place.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

from . import _native

KV_TILE = _native.KV_TILE
# the attention kernels address a V^T row as row * 2 * capacity in 24-bit
# multiplies: a slot holds fewer than 2^23 tokens
MAX_SLOT_CAPACITY = (1 << 23) - KV_TILE


def round_up(value: int, multiple: int) -> int:
    return (int(value) + multiple - 1) // multiple * multiple


def vt_position(t: int) -> int:
    """Column of token ``t`` inside a transposed value row (an involution)."""
    chunk = (t >> 2) & 3
    perm = (0, 2, 1, 3)[chunk]
    return (t & ~15) | (perm << 2) | (t & 3)


def vt_columns(torch: Any, count: int, device: Any) -> Any:
    """``vt_position`` of tokens ``0 .. count - 1`` as a long tensor on ``device``."""
    t = torch.arange(int(count), device=device)
    chunk = (t >> 2) & 3
    perm = torch.where(chunk == 1, 2, torch.where(chunk == 2, 1, chunk))
    return (t & ~15) | (perm << 2) | (t & 3)


@dataclass
class SlotView:
    """Rows ``row0 .. row0 + tokens`` of a slot, as one attention segment.

    ``row0`` is a multiple of 64 (a key tile; the transposed value order
    repeats every 16 tokens), and the slot rows up to the next multiple of 64
    after the view are zero.
    """

    slot: "KVSlot"
    tokens: int
    row0: int = 0

    def to_segment(self) -> _native.KVSegment:
        s = self.slot
        if self.row0 % KV_TILE or self.row0 + round_up(self.tokens, KV_TILE) > s.capacity:
            raise ValueError(f"slot view rows [{self.row0}, {self.row0 + self.tokens}) are not a tile-aligned part of the slot")
        return _native.KVSegment(
            k=_native.ptr(s.k) + 2 * self.row0 * s.head_dim,
            vt=_native.ptr(s.vt) + 2 * self.row0,
            k_head_stride=s.capacity * s.head_dim,
            vt_head_stride=s.capacity * s.head_dim,
            vt_row_stride=s.capacity,
            tokens=int(self.tokens),
        )


class KVSlot:
    """One head-major key/value block (see module docstring)."""

    def __init__(self, torch: Any, *, heads: int, head_dim: int, capacity: int, device: Any) -> None:
        self._torch = torch
        self.heads = int(heads)
        self.head_dim = int(head_dim)
        self.capacity = max(KV_TILE, round_up(capacity, KV_TILE))
        if self.capacity > MAX_SLOT_CAPACITY:
            raise ValueError(f"slot capacity {self.capacity} above the {MAX_SLOT_CAPACITY} tokens a slot can hold")
        self.device = torch.device(device)
        self.k = torch.empty((self.heads, self.capacity, self.head_dim), dtype=torch.bfloat16, device=self.device)
        self.vt = torch.empty((self.heads, self.head_dim, self.capacity), dtype=torch.bfloat16, device=self.device)
        self.tokens = 0
        # handle of the stream a pool last took this slot back on
        self.released_on: int | None = None
        # exact fixed-point key sums of views of this slot, (row0, tokens, stream) ->
        # int64 [H, D]; dropped whenever the slot is written (pack, staged norm + RoPE)
        self.key_sums: dict[tuple[int, int, int], Any] = {}

    @property
    def nbytes(self) -> int:
        return 2 * self.k.numel() * self.k.element_size()

    def view(self, tokens: int | None = None) -> SlotView:
        count = self.tokens if tokens is None else int(tokens)
        if not 0 < count <= self.tokens:
            raise ValueError(f"slot view of {count} tokens outside the {self.tokens} packed rows")
        return SlotView(self, count)

    def pack(self, key: Any, value: Any, *, rows: Any | None = None, row0: int = 0, count: int | None = None,
             dst: int = 0, rows_checked: bool = False) -> None:
        """Copy token-major rows of ``key``/``value`` ([T, H, D] bf16) into the slot.

        ``rows`` is an int32/int64 GPU index tensor; without it rows
        ``row0 .. row0 + count`` are copied.  They land at slot rows
        ``dst ..`` (``dst`` a multiple of 64) and the slot rows after them up to
        the next multiple of 64 are zeroed; ``tokens`` becomes the end row.
        The range of ``rows`` is checked (one sync) unless ``rows_checked``.
        """
        torch = self._torch
        for name, t in (("key", key), ("value", value)):
            _native.require_device_tensor(torch, t, name)
            if t.dtype != torch.bfloat16 or t.ndim != 3 or t.stride(2) != 1:
                raise ValueError(f"{name} must be a [tokens, heads, dim] bf16 view with unit dim stride")
        if key.shape != value.shape or key.stride() != value.stride():
            raise ValueError("key and value must share shape and strides")
        if tuple(key.shape[1:]) != (self.heads, self.head_dim):
            raise ValueError(f"K/V heads x dim {tuple(key.shape[1:])} differ from slot {(self.heads, self.head_dim)}")
        rows_ptr = None
        if rows is not None:
            from .attention import _row_list

            rows = _row_list(torch, rows, key.device, int(key.shape[0]), "rows", rows_checked)
            n = int(rows.numel())
            rows_ptr = _native.ptr(rows) if n else None
        else:
            n = int(key.shape[0]) - int(row0) if count is None else int(count)
            if int(row0) < 0 or n < 0 or int(row0) + n > int(key.shape[0]):
                raise ValueError(f"rows [{row0}, {int(row0) + n}) outside the {int(key.shape[0])} K/V rows")
        dst = int(dst)
        if dst < 0 or dst % KV_TILE or dst + n > self.capacity:
            raise ValueError(f"{n} rows at slot row {dst} do not fit the slot capacity {self.capacity} (tile-aligned)")
        self.key_sums.clear()
        lib = _native.load()
        status = lib.tmhd_kv_pack(
            _native.ptr(key), _native.ptr(value), key.stride(0), key.stride(1), rows_ptr, int(row0), n,
            _native.ptr(self.k), _native.ptr(self.vt), self.capacity * self.head_dim,
            self.capacity * self.head_dim, self.capacity, dst, dst + round_up(n, KV_TILE), self.heads,
            self.head_dim, _native.stream_ptr(torch, key.device),
        )
        _native.check(status, "tmhd_kv_pack")
        self.tokens = dst + n

    def token_major(self, tokens: int | None = None, order: Any | None = None) -> tuple[Any, Any]:
        """Materialise ``[tokens, H, D]`` key/value copies (compatibility path)."""
        torch = self._torch
        n = self.tokens if tokens is None else int(tokens)
        key = self.k[:, :n, :].permute(1, 0, 2).contiguous()
        cols = vt_columns(torch, n, self.device)
        value = self.vt.index_select(2, cols).permute(2, 0, 1).contiguous()
        if order is not None:
            key = key.index_select(0, order)
            value = value.index_select(0, order)
        return key, value


class SlotPool:
    """Pool of slots of one shape family, recycled without copies.

    ``acquire`` hands out the smallest free slot that fits (or a new one);
    ``release`` takes it back.  At most ``max_free`` slots are kept free:
    beyond that the smallest free slot is returned to the allocator, so a
    pool's idle memory stays bounded (``free_bytes``).

    Streams: a slot is handed out again only on the stream it was released
    on, where the kernels that last read it are queued ahead of any new
    writer; and ``release`` records that stream on the slot's memory, so a
    slot returned to the allocator is not reused on its allocation stream
    before those kernels end.  A slot in use (between ``acquire`` and
    ``release``) is the caller's to order across streams.
    """

    def __init__(self, torch: Any, *, heads: int, head_dim: int, device: Any, max_free: int = 8) -> None:
        if int(max_free) < 0:
            raise ValueError("max_free must be non-negative")
        self._torch = torch
        self.heads = heads
        self.head_dim = head_dim
        self.device = device
        self.max_free = int(max_free)
        self._free: list[KVSlot] = []

    @property
    def free_bytes(self) -> int:
        return sum(slot.nbytes for slot in self._free)

    def acquire(self, tokens: int) -> KVSlot:
        need = round_up(max(int(tokens), 1), KV_TILE)
        stream = self._stream_key()
        best = None
        for slot in self._free:
            if slot.released_on != stream:
                continue
            if slot.capacity >= need and (best is None or slot.capacity < best.capacity):
                best = slot
        if best is not None:
            self._free.remove(best)
            best.tokens = 0
            return best
        return KVSlot(self._torch, heads=self.heads, head_dim=self.head_dim, capacity=need, device=self.device)

    def _stream_key(self) -> int:
        """Handle of the current stream on the pool's device (0 off the GPU)."""
        torch = self._torch
        if torch.device(self.device).type != "cuda":
            return 0
        return int(torch.cuda.current_stream(device=self.device).cuda_stream)

    def release(self, slot: KVSlot) -> None:
        slot.tokens = 0
        torch = self._torch
        if slot.k.is_cuda:
            stream = torch.cuda.current_stream(device=slot.k.device)
            slot.k.record_stream(stream)
            slot.vt.record_stream(stream)
        slot.released_on = self._stream_key()
        self._free.append(slot)
        if len(self._free) > self.max_free:
            self._free.remove(min(self._free, key=lambda s: s.capacity))

    def clear(self) -> None:
        self._free.clear()
