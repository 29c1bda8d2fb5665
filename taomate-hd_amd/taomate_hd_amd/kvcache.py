"""Head-major in-place KV cache with the public API of the reference's
``CleanAVKVCache`` (src/taomate_hd/streaming/cache.py:68-392).

The reference keeps each layer's history as one token-major ``[tokens, H, D]``
tensor: a commit ``torch.cat``s the staged rows onto it (cache.py:293-296) and
eviction ``index_select``s the survivors into a new tensor (cache.py:339-378).
Here every committed block owns one slot per layer (head-major keys,
transposed values, see slots.py):

* ``stage`` packs the commit rows straight into a free slot (the only copy);
* ``commit`` only appends the block to the ledger;
* ``retain_sink_and_recent_commits`` returns evicted slots to the pool, and
  the video-only sink filter shortens block 0 in place, because block 0 is
  packed with its video rows first;
* the hook reads ``history_views`` / ``fused_current_views``: slot views that
  the attention kernel consumes in place.

The reference-shaped readers (``history``, ``history_blocks``, ...) return
token-major copies in the reference's row order, for callers outside the hook.
Ledger semantics (counts, tags, block order, sink filtering, validation and
errors) follow cache.py line by line.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

from .slots import KVSlot, SlotPool, SlotView

MAIN_LAYER_NAMES = tuple(f"blocks.{index}.attn" for index in range(50))
VIDEO_TOKEN_TAG = 0
AUDIO_TOKEN_TAG = 2
AV_TOKEN_TAGS = frozenset({VIDEO_TOKEN_TAG, AUDIO_TOKEN_TAG})


@dataclass(frozen=True)
class KVContract:
    """Post-Ulysses K/V shape contract (cache.py:12-17)."""

    layer_names: tuple[str, ...] = MAIN_LAYER_NAMES
    local_heads: int = 14
    head_dim: int = 128
    dtype: str = "torch.bfloat16"


def kv_contract_from_model(model: Any) -> KVContract:
    """Resolve post-Ulysses local K/V heads from the live topology (cache.py:20-33)."""
    arch = getattr(model, "arch", None)
    context = getattr(model, "parallel_context", None)
    total_heads = int(getattr(arch, "num_attention_heads", 0))
    head_dim = int(getattr(arch, "attention_head_dim", 0))
    tp_size = int(getattr(context, "tp_world_size", 0))
    ulysses_size = int(getattr(context, "ulysses_world_size", 0))
    parallel_size = tp_size * ulysses_size
    if total_heads <= 0 or head_dim <= 0 or parallel_size <= 0 or total_heads % tp_size:
        raise ValueError("live H3 attention topology cannot resolve local K/V heads")
    return KVContract(
        local_heads=(total_heads // tp_size + ulysses_size - 1) // ulysses_size, head_dim=head_dim
    )


@dataclass(frozen=True)
class AVKV:
    """Token-major audio-video key/value pair (cache.py:36-40)."""

    key: Any
    value: Any
    modality: str = "audio_video"


def _validate_committed_media_tags(tags: tuple[int, ...]) -> None:
    """cache.py:63-65."""
    if not tags or frozenset(tags) != AV_TOKEN_TAGS:
        raise ValueError("clean H3 commit must contain both video and audio rows")


@dataclass
class _Block:
    """One committed (or staged) clean block.

    ``tags`` is the reference ledger entry (original row order).  ``order``
    lists, for each slot row, the original row it holds; block 0 of a cache
    is packed video rows first so the sink filter is a prefix.
    """

    tags: tuple[int, ...]
    order: tuple[int, ...]
    slots: dict[str, KVSlot] = field(default_factory=dict)

    @property
    def count(self) -> int:
        return len(self.tags)


class HeadMajorRingKVCache:
    """Persistent post-RoPE media history committed only from clean AV states."""

    def __init__(self, contract: KVContract | None = None) -> None:
        self.contract = contract or KVContract()
        self._blocks: list[_Block] = []
        self._staged: _Block | None = None
        self._staged_commit_indices: Any | None = None
        self._staged_rows_host: tuple[int, ...] | None = None
        self._block_index = 0
        self._sink_video_only = False
        self._pool: SlotPool | None = None
        self._device: Any | None = None

    # ---- ledger properties (cache.py:85-107)
    @property
    def committed_blocks(self) -> int:
        return self._block_index

    @property
    def history_tokens(self) -> int:
        return sum(block.count for block in self._blocks)

    @property
    def retained_blocks(self) -> int:
        return len(self._blocks)

    @property
    def history_audio_tokens(self) -> int:
        return sum(tag == AUDIO_TOKEN_TAG for block in self._blocks for tag in block.tags)

    @property
    def history_video_tokens(self) -> int:
        return sum(tag == VIDEO_TOKEN_TAG for block in self._blocks for tag in block.tags)

    @property
    def clean_commit_active(self) -> bool:
        return self._staged is not None

    @property
    def commit_token_counts(self) -> tuple[int, ...]:
        return tuple(block.count for block in self._blocks)

    @property
    def commit_token_tags(self) -> tuple[tuple[int, ...], ...]:
        return tuple(block.tags for block in self._blocks)

    @property
    def slot_bytes(self) -> int:
        """Device bytes held by committed and staged slots."""
        blocks = [*self._blocks, *([self._staged] if self._staged is not None else [])]
        return sum(slot.nbytes for block in blocks for slot in block.slots.values())

    def _check_layer(self, layer: str) -> None:
        if layer not in self.contract.layer_names:
            raise KeyError(f"unknown H3 attention layer: {layer}")

    # ---- zero-copy readers used by the hook
    def _block_view(self, block: _Block, layer: str, rows: int | None = None) -> SlotView:
        slot = block.slots[layer]
        return slot.view(block.count if rows is None else rows)

    def history_views(self, layer: str) -> tuple[SlotView, ...]:
        """All retained blocks of ``layer`` as slot views (the ``history`` prefix)."""
        self._check_layer(layer)
        return tuple(self._block_view(block, layer) for block in self._blocks)

    def fused_current_views(
        self, layer: str, *, use_sink: bool = False, recent_blocks: int | None = None
    ) -> tuple[SlotView, ...]:
        """Slot views of ``history_for_fused_current`` (cache.py:179-207)."""
        self._check_layer(layer)
        if recent_blocks is None:
            return self.history_views(layer)
        persistent_recent = max(0, recent_blocks - 1)
        if use_sink:
            selected = self._sink_and_recent_indices(persistent_recent)
            if not selected:
                return ()
            views = [self._block_view(self._blocks[i], layer) for i in selected]
            if (
                self._sink_video_only
                and self.retained_blocks + 1 > recent_blocks
                and AUDIO_TOKEN_TAG in self._blocks[0].tags
            ):
                video_rows = sum(tag == VIDEO_TOKEN_TAG for tag in self._blocks[0].tags)
                views[0] = self._block_view(self._blocks[0], layer, video_rows)
            return tuple(views)
        return tuple(self._block_view(self._blocks[i], layer) for i in self._recent_indices(persistent_recent))

    def staged_view(self, layer: str) -> SlotView | None:
        """The rows staged for ``layer`` in the active clean commit, if any."""
        if self._staged is None or layer not in self._staged.slots:
            return None
        return self._block_view(self._staged, layer)

    # ---- reference readers (token-major copies in reference row order)
    def _materialize(self, blocks: list[tuple[_Block, int]], layer: str) -> AVKV | None:
        import torch

        if not blocks:
            return None
        keys, values = [], []
        for block, rows in blocks:
            slot = block.slots[layer]
            order = block.order[:rows]
            inverse = sorted(range(rows), key=lambda i: order[i])
            index = None
            if inverse != list(range(rows)):
                index = torch.tensor(inverse, dtype=torch.long, device=slot.device)
            key, value = slot.token_major(rows, order=index)
            keys.append(key)
            values.append(value)
        if len(keys) == 1:
            return AVKV(key=keys[0], value=values[0])
        return AVKV(key=torch.cat(keys, dim=0), value=torch.cat(values, dim=0))

    def history(self, layer: str) -> AVKV | None:
        """Complete retained prefix for attention (cache.py:109-123)."""
        self._check_layer(layer)
        if not self._blocks:
            return None
        return self._materialize([(b, b.count) for b in self._blocks], layer)

    def _recent_indices(self, count: int) -> list[int]:
        if count == 0 or not self._blocks:
            return []
        if count >= len(self._blocks):
            return list(range(len(self._blocks)))
        return list(range(len(self._blocks) - count, len(self._blocks)))

    def recent_history(self, layer: str, count: int) -> AVKV | None:
        """Suffix holding at most ``count`` committed blocks (cache.py:125-135)."""
        if isinstance(count, bool) or not isinstance(count, int) or count < 0:
            raise ValueError("recent H3 history count must be non-negative")
        self._check_layer(layer)
        idx = self._recent_indices(count)
        return self._materialize([(self._blocks[i], self._blocks[i].count) for i in idx], layer)

    def _sink_and_recent_indices(self, recent_count: int) -> list[int]:
        if not self._blocks:
            return []
        recent_start = max(1, len(self._blocks) - recent_count)
        return [0, *range(recent_start, len(self._blocks))]

    def sink_and_recent_history(self, layer: str, recent_count: int) -> AVKV | None:
        """Block-zero sink plus the newest non-sink commits (cache.py:137-149)."""
        blocks = self.sink_and_recent_history_blocks(layer, recent_count)
        if not blocks:
            return None
        if len(blocks) == 1:
            return blocks[0]
        import torch

        return AVKV(
            key=torch.cat(tuple(pair.key for pair in blocks), dim=0),
            value=torch.cat(tuple(pair.value for pair in blocks), dim=0),
        )

    def sink_and_recent_history_blocks(self, layer: str, recent_count: int) -> tuple[AVKV, ...]:
        """cache.py:151-159."""
        if isinstance(recent_count, bool) or not isinstance(recent_count, int) or recent_count < 0:
            raise ValueError("recent H3 history count must be non-negative")
        self._check_layer(layer)
        return tuple(
            self._materialize([(self._blocks[i], self._blocks[i].count)], layer)
            for i in self._sink_and_recent_indices(recent_count)
        )

    def history_blocks(self, layer: str) -> tuple[AVKV, ...]:
        """Retained history, one pair per block (cache.py:161-177)."""
        self._check_layer(layer)
        return tuple(self._materialize([(b, b.count)], layer) for b in self._blocks)

    def history_for_fused_current(
        self, layer: str, *, use_sink: bool = False, recent_blocks: int | None = None
    ) -> AVKV | None:
        """Persistent part of the hypothetical post-commit view (cache.py:179-207)."""
        self._check_layer(layer)
        if recent_blocks is None:
            return self.history(layer)
        persistent_recent = max(0, recent_blocks - 1)
        if use_sink:
            selected = self._sink_and_recent_indices(persistent_recent)
            if not selected:
                return None
            rows = [self._blocks[i].count for i in selected]
            if (
                self._sink_video_only
                and self.retained_blocks + 1 > recent_blocks
                and AUDIO_TOKEN_TAG in self._blocks[0].tags
            ):
                rows[0] = sum(tag == VIDEO_TOKEN_TAG for tag in self._blocks[0].tags)
            return self._materialize([(self._blocks[i], r) for i, r in zip(selected, rows)], layer)
        return self.recent_history(layer, persistent_recent)

    # ---- write side
    def begin_clean_commit(self, block_index: int) -> None:
        """cache.py:209-218."""
        if block_index != self._block_index:
            raise ValueError(f"clean block order mismatch: expected {self._block_index}, got {block_index}")
        if self._staged is not None:
            raise RuntimeError("a clean commit is already active")
        self._staged = _Block(tags=(), order=())
        self._staged_commit_indices = None
        self._staged_rows_host = None

    def _slot_pool(self, device: Any) -> SlotPool:
        import torch

        if self._pool is None:
            # evicting a block frees one slot per layer, which the next stage takes
            # back: keep up to two blocks' worth free
            self._pool = SlotPool(
                torch, heads=self.contract.local_heads, head_dim=self.contract.head_dim, device=device,
                max_free=2 * len(self.contract.layer_names),
            )
            self._device = torch.device(device)
        elif torch.device(device) != self._device:
            raise ValueError(f"K/V must share one CUDA device ({self._device})")
        return self._pool

    def stage(
        self,
        layer: str,
        key: Any,
        value: Any,
        token_tags: Any,
        commit_mask: Any,
        *,
        commit_indices: Any | None = None,
    ) -> None:
        """Stage one layer's commit rows into a free slot (cache.py:220-277)."""
        import torch

        if self._staged is None:
            raise RuntimeError("K/V may be staged only during a clean sigma=0 forward")
        if layer not in self.contract.layer_names or layer in self._staged.slots:
            raise ValueError(f"invalid or duplicate clean K/V layer: {layer}")
        if (
            not torch.is_tensor(token_tags)
            or not torch.is_tensor(commit_mask)
            or token_tags.ndim != 1
            or commit_mask.ndim != 1
            or commit_mask.dtype != torch.bool
        ):
            raise TypeError("token_tags and commit_mask must be one-dimensional tensors")
        if (
            key.shape[0] != token_tags.shape[0]
            or value.shape[0] != token_tags.shape[0]
            or commit_mask.shape[0] != token_tags.shape[0]
        ):
            raise ValueError("token metadata and post-Ulysses K/V rows differ")
        if not torch.is_tensor(key) or not torch.is_tensor(value) or key.shape != value.shape or key.ndim != 3:
            raise ValueError(f"{layer} K/V must have the same [tokens, heads, dim] shape")
        if tuple(key.shape[1:]) != (self.contract.local_heads, self.contract.head_dim):
            raise ValueError(
                f"{layer} K/V local shape must be [{self.contract.local_heads}, {self.contract.head_dim}]"
            )
        if key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
            raise ValueError(f"{layer} K/V must be bfloat16")
        if not key.is_cuda or not value.is_cuda or key.device != value.device:
            raise ValueError(f"{layer} K/V must share one CUDA device")
        if self._staged_commit_indices is None:
            if commit_indices is None:
                commit_indices = torch.nonzero(commit_mask, as_tuple=False).view(-1)
            if (
                not torch.is_tensor(commit_indices)
                or commit_indices.ndim != 1
                or commit_indices.dtype != torch.long
                or commit_indices.device != key.device
                or int(commit_indices.numel()) == 0
            ):
                raise ValueError("clean H3 block contains no valid audio/video rows")
            tags = tuple(int(t) for t in token_tags.index_select(0, commit_indices).detach().cpu().tolist())
            _validate_committed_media_tags(tags)
            order = tuple(range(len(tags)))
            if not self._blocks:
                # block 0 becomes the sink: video rows first, so the
                # video-only filter of retain_sink_and_recent_commits is a prefix
                order = tuple(i for i, t in enumerate(tags) if t == VIDEO_TOKEN_TAG) + tuple(
                    i for i, t in enumerate(tags) if t != VIDEO_TOKEN_TAG
                )
            indices = commit_indices.detach()
            if order != tuple(range(len(tags))):
                indices = indices.index_select(0, torch.tensor(order, dtype=torch.long, device=indices.device))
            self._staged.tags = tags
            self._staged.order = order
            self._staged_commit_indices = indices.to(torch.int32).contiguous()
            self._staged_rows_host = tuple(int(r) for r in indices.cpu().tolist())
        rows = self._staged_commit_indices
        slot = self._slot_pool(key.device).acquire(int(rows.numel()))
        try:
            slot.pack(key, value, rows=rows, rows_checked=True)  # index_select above bounds-checked them
        except BaseException:
            self._pool.release(slot)
            raise
        self._staged.slots[layer] = slot

    def staged_rows(self) -> Any | None:
        """Packed-sequence rows of the active commit, in slot order (int32)."""
        return self._staged_commit_indices

    def staged_rows_host(self) -> tuple[int, ...] | None:
        """Host copy of ``staged_rows`` (taken once per commit)."""
        return self._staged_rows_host

    def commit(self) -> None:
        """Atomically append the staged block (cache.py:279-316)."""
        if self._staged is None:
            raise RuntimeError("no clean commit is active")
        missing = [name for name in self.contract.layer_names if name not in self._staged.slots]
        if missing:
            raise RuntimeError(f"clean commit is missing attention layers: {missing}")
        if self._staged.count <= 0:
            raise RuntimeError("clean H3 commit did not append media tokens")
        block = self._staged
        self._staged = None
        self._staged_commit_indices = None
        self._staged_rows_host = None
        self._blocks.append(block)
        self._block_index += 1

    def retain_sink_and_recent_commits(self, recent_count: int, *, sink_video_only: bool = True) -> None:
        """Keep the block-zero sink plus the newest complete AV blocks (cache.py:318-378)."""
        if isinstance(recent_count, bool) or not isinstance(recent_count, int) or recent_count < 0:
            raise ValueError("recent clean commit count must be non-negative")
        if self._staged is not None:
            raise RuntimeError("cannot evict H3 history during a clean commit")
        self._sink_video_only = bool(sink_video_only)
        block_count = len(self._blocks)
        if block_count == 0:
            return
        recent_start = max(0, block_count - recent_count)
        selections = [
            (0, bool(sink_video_only and recent_start > 0)),
            *((index, False) for index in range(max(1, recent_start), block_count)),
        ]
        if selections == [(index, False) for index in range(block_count)]:
            return
        kept = {index for index, _ in selections}
        for index, block in enumerate(self._blocks):
            if index not in kept:
                for slot in block.slots.values():
                    self._pool.release(slot)
        retained: list[_Block] = []
        for index, video_only in selections:
            block = self._blocks[index]
            if video_only:
                # the sink slot holds its video rows first: shorten in place
                video = tuple(i for i in block.order if block.tags[i] == VIDEO_TOKEN_TAG)
                block.order = tuple(range(len(video)))
                block.tags = tuple(VIDEO_TOKEN_TAG for _ in video)
            retained.append(block)
        self._blocks = retained

    def rollback(self) -> None:
        """Drop the staged block (cache.py:380-383)."""
        if self._staged is not None and self._pool is not None:
            for slot in self._staged.slots.values():
                self._pool.release(slot)
        self._staged = None
        self._staged_commit_indices = None
        self._staged_rows_host = None

    def clear(self) -> None:
        """cache.py:385-392."""
        if self._staged is not None:
            raise RuntimeError("cannot clear H3 history during a clean commit")
        if self._pool is not None:
            for block in self._blocks:
                for slot in block.slots.values():
                    self._pool.release(slot)
        self._blocks = []
        self._block_index = 0
        self._sink_video_only = False

    def release_memory(self) -> None:
        """Free the pooled (unused) slots back to the allocator."""
        if self._pool is not None:
            self._pool.clear()


# the reference's class name, for call sites that construct it by name
CleanAVKVCache = HeadMajorRingKVCache

__all__ = [
    "AVKV",
    "AV_TOKEN_TAGS",
    "AUDIO_TOKEN_TAG",
    "CleanAVKVCache",
    "HeadMajorRingKVCache",
    "KVContract",
    "MAIN_LAYER_NAMES",
    "VIDEO_TOKEN_TAG",
    "kv_contract_from_model",
]

