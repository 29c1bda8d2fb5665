"""CPU restatement of the streaming hook, KV cache and their ledger semantics.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

``CacheOracle`` restates CleanAVKVCache (src/taomate_hd/streaming/cache.py:68-392)
and ``HookOracle`` restates H3StreamingAttentionHook.__call__
(src/taomate_hd/streaming/attention_hook.py:236-483) on numpy arrays, keeping
the reference's data flow: token-major ``[tokens, H, D]`` histories grown by
concatenation, K/V parts concatenated in plan order, attention computed by
``attention_fp64`` (SDPA backend) or ``i8qk_attention`` (Sage backend).
Pinned by tests/test_oracle.py with hand-derived ledgers and row plans.
"""

from __future__ import annotations

import numpy as np

from . import attention

VIDEO = 0
AUDIO = 2


class CacheOracle:
    """cache.py:68-392 on numpy arrays (one history array pair per layer)."""

    def __init__(self, layer_names):
        self.layer_names = tuple(layer_names)
        self.history_kv: dict[str, tuple[np.ndarray, np.ndarray]] = {}
        self.staged: dict | None = None
        self.staged_indices = None
        self.staged_tags = None
        self.block_index = 0
        self.counts: list[int] = []
        self.tags: list[tuple[int, ...]] = []
        self.sink_video_only = False

    @property
    def retained_blocks(self) -> int:
        return len(self.counts)

    def history(self, layer):
        """cache.py:109-123."""
        return self.history_kv.get(layer)

    def blocks(self, layer):
        """cache.py:161-177."""
        pair = self.history(layer)
        if pair is None:
            return []
        out, off = [], 0
        for c in self.counts:
            out.append((pair[0][off : off + c], pair[1][off : off + c]))
            off += c
        return out

    def recent_history(self, layer, count):
        """cache.py:125-135."""
        pair = self.history(layer)
        if pair is None or count == 0:
            return None
        if count >= len(self.counts):
            return pair
        n = sum(self.counts[-count:])
        return (pair[0][-n:], pair[1][-n:])

    def sink_and_recent_blocks(self, layer, recent_count):
        """cache.py:151-159."""
        blocks = self.blocks(layer)
        if not blocks:
            return []
        start = max(1, len(blocks) - recent_count)
        return [blocks[0], *blocks[start:]]

    def sink_and_recent_history(self, layer, recent_count):
        """cache.py:137-149."""
        sel = self.sink_and_recent_blocks(layer, recent_count)
        if not sel:
            return None
        return (np.concatenate([b[0] for b in sel]), np.concatenate([b[1] for b in sel]))

    def history_for_fused_current(self, layer, use_sink=False, recent_blocks=None):
        """cache.py:179-207."""
        if recent_blocks is None:
            return self.history(layer)
        persistent_recent = max(0, recent_blocks - 1)
        if use_sink:
            pair = self.sink_and_recent_history(layer, persistent_recent)
            if (
                pair is not None
                and self.sink_video_only
                and self.retained_blocks + 1 > recent_blocks
                and AUDIO in self.tags[0]
            ):
                sink_tags = self.tags[0]
                rows = [r for r, t in enumerate(sink_tags) if t == VIDEO]
                rows.extend(range(len(sink_tags), pair[0].shape[0]))
                return (pair[0][rows], pair[1][rows])
            return pair
        return self.recent_history(layer, persistent_recent)

    def begin_clean_commit(self, block_index):
        """cache.py:209-218."""
        if block_index != self.block_index:
            raise ValueError("clean block order mismatch")
        if self.staged is not None:
            raise RuntimeError("a clean commit is already active")
        self.staged = {}
        self.staged_indices = None
        self.staged_tags = None

    def stage(self, layer, key, value, token_tags, commit_mask, commit_indices=None):
        """cache.py:220-277."""
        if self.staged is None:
            raise RuntimeError("K/V may be staged only during a clean sigma=0 forward")
        if layer not in self.layer_names or layer in self.staged:
            raise ValueError("invalid or duplicate clean K/V layer")
        if self.staged_indices is None:
            if commit_indices is None:
                commit_indices = np.nonzero(commit_mask)[0]
            if len(commit_indices) == 0:
                raise ValueError("clean H3 block contains no valid audio/video rows")
            tags = tuple(int(t) for t in np.asarray(token_tags)[commit_indices])
            if not tags or frozenset(tags) != frozenset({VIDEO, AUDIO}):
                raise ValueError("clean H3 commit must contain both video and audio rows")
            self.staged_indices = np.asarray(commit_indices)
            self.staged_tags = tags
        self.staged[layer] = (key[self.staged_indices].copy(), value[self.staged_indices].copy())

    def commit(self):
        """cache.py:279-316."""
        if self.staged is None:
            raise RuntimeError("no clean commit is active")
        missing = [n for n in self.layer_names if n not in self.staged]
        if missing:
            raise RuntimeError(f"clean commit is missing attention layers: {missing}")
        for name in self.layer_names:
            cur = self.staged.pop(name)
            prev = self.history_kv.pop(name, None)
            self.history_kv[name] = cur if prev is None else (
                np.concatenate([prev[0], cur[0]]), np.concatenate([prev[1], cur[1]])
            )
        counts = {pair[0].shape[0] for pair in self.history_kv.values()}
        if len(counts) != 1:
            raise RuntimeError("per-layer H3 history token counts diverged")
        current = counts.pop() - sum(self.counts)
        if current <= 0:
            raise RuntimeError("clean H3 commit did not append media tokens")
        tags = self.staged_tags
        self.staged = None
        self.staged_indices = None
        self.staged_tags = None
        self.block_index += 1
        self.counts.append(current)
        self.tags.append(tags)

    def retain_sink_and_recent_commits(self, recent_count, sink_video_only=True):
        """cache.py:318-378."""
        if self.staged is not None:
            raise RuntimeError("cannot evict H3 history during a clean commit")
        self.sink_video_only = bool(sink_video_only)
        n = len(self.counts)
        if n == 0:
            return
        recent_start = max(0, n - recent_count)
        selections = [(0, bool(sink_video_only and recent_start > 0))] + [
            (i, False) for i in range(max(1, recent_start), n)
        ]
        if selections == [(i, False) for i in range(n)]:
            return
        new_tags = [
            tuple(t for t in self.tags[i] if t == VIDEO) if vo else self.tags[i] for i, vo in selections
        ]
        offsets = np.cumsum([0] + self.counts[:-1])
        rows = [
            offsets[i] + r for i, vo in selections for r, t in enumerate(self.tags[i]) if not vo or t == VIDEO
        ]
        for name in self.layer_names:
            k, v = self.history_kv[name]
            self.history_kv[name] = (k[rows], v[rows])
        self.counts = [len(t) for t in new_tags]
        self.tags = new_tags

    def rollback(self):
        """cache.py:380-383."""
        self.staged = None
        self.staged_indices = None
        self.staged_tags = None


class HookOracle:
    """attention_hook.py:150-483 on numpy; returns float64 outputs."""

    def __init__(self, cache: CacheOracle, backend: str = "sdpa"):
        self.cache = cache
        self.backend = backend
        self.mode = "idle"
        self.fused_use_sink = None
        self.fused_recent = None

    def activate(self, mode, block_index, fused_current_use_sink=None, fused_current_recent_blocks=None):
        if self.mode != "idle":
            raise RuntimeError("H3 streaming attention hook is already active")
        if block_index != self.cache.block_index:
            raise ValueError("streaming attention block differs from clean history")
        self.mode = mode
        self.fused_use_sink = fused_current_use_sink
        self.fused_recent = fused_current_recent_blocks

    def deactivate(self):
        self.mode = "idle"
        self.fused_use_sink = None
        self.fused_recent = None

    def _exact(self, q, parts, scale):
        ks = [p[0] for p in parts]
        vs = [p[1] for p in parts]
        if self.backend == "sage_attn":
            out, _ = attention.i8qk_attention(q, ks, vs, scale)
            return out
        return attention.attention_fp64(q, np.concatenate(ks), np.concatenate(vs), scale)

    def __call__(self, layer, q, k, v, token_tags, commit_mask, boundaries, scale, live_documents_hint=None,
                 cached_documents=(), compact_rows=None):
        """q/k/v float32 [T, H, D] (bf16 values), commit_mask bool [T].

        ``cached_documents``: live documents whose condition attention the
        condition cache reuses (condition_cache.py:322-329): their condition
        query rows are not computed and read zero (attention_hook.py:445-450),
        while media queries still attend over their condition keys.
        ``compact_rows``: the sorted rows the condition cache keeps in its
        compact order (condition_cache.py:173-228); the output then holds only
        those rows, in that order (rows nobody writes stay zero)."""
        if self.mode == "idle":
            raise RuntimeError("patched H3 attention called outside a streaming step")
        bounds = tuple(int(b) for b in boundaries)
        if live_documents_hint is None:
            live = tuple(
                i for i, (a, b) in enumerate(zip(bounds, bounds[1:])) if bool(np.any(commit_mask[a:b]))
            )
        else:
            live = tuple(live_documents_hint)
        fused = self.mode == "fused_progress_denoise"
        if len(live) != (2 if fused else 1):
            raise ValueError("streaming session target-document count differs from hook mode")
        live_doc = live[-1]
        prev_doc = live[0] if fused else None
        persistent = self.cache.history(layer)
        out = np.zeros(q.shape, dtype=np.float64)
        prev_media_idx = None
        if fused:
            a, b = bounds[prev_doc], bounds[prev_doc + 1]
            prev_media_idx = np.nonzero(commit_mask[a:b])[0] + a
        for index, (start, stop) in enumerate(zip(bounds, bounds[1:])):
            if start == stop:
                continue
            qs, ks, vs = q[start:stop], k[start:stop], v[start:stop]
            if index not in live:
                out[start:stop] = self._exact(qs, [(ks, vs)], scale)
                continue
            mask = commit_mask[start:stop]
            cond = np.nonzero(~mask)[0]
            media = np.nonzero(mask)[0]
            cond_kv = (ks[cond], vs[cond])
            prefixes = []
            previous = None
            if fused and index == live_doc:
                cur = self.cache.history_for_fused_current(
                    layer,
                    **({} if self.fused_recent is None else {
                        "use_sink": bool(self.fused_use_sink), "recent_blocks": self.fused_recent}),
                )
                if cur is not None:
                    prefixes.append(cur)
                previous = (k[prev_media_idx], v[prev_media_idx])
            elif persistent is not None:
                prefixes.append(persistent)
            media_parts = [cond_kv, *prefixes]
            if previous is not None:
                media_parts.append(previous)
            media_parts.append((ks[media], vs[media]))
            media_parts = [p for p in media_parts if p[0].shape[0] > 0]
            if len(cond) and index not in cached_documents:
                out[start + cond] = self._exact(qs[cond], [cond_kv], scale)
            if len(media):
                out[start + media] = self._exact(qs[media], media_parts, scale)
        if self.mode == "clean_commit":
            self.cache.stage(layer, k, v, token_tags, commit_mask)
        elif fused:
            self.cache.stage(layer, k, v, token_tags, commit_mask, commit_indices=prev_media_idx)
        if compact_rows is not None:
            return out[np.asarray(compact_rows, dtype=np.int64)]
        return out


def packed_layout(text: int, cond: int, audio: int, video: int, align: int = 64):
    """One packed document [text, cond, audio, video, pad] and its metadata.

    Restates minimax_h3_packed_sequence (src/taomate_hd/model/packed_sequence.py:113-194)
    and the commit mask of _native_attention_metadata
    (src/taomate_hd/streaming/runtime.py:711-714): tags text 1, audio 2,
    video and cond 0, pad -1; commit rows = target video + target audio;
    cu_seqlens = [0, used, seq_len].
    """
    used = text + cond + audio + video
    seq_len = (used + align - 1) // align * align
    tags = np.full(seq_len, -1, dtype=np.int64)
    tags[:text] = 1
    tags[text : text + cond] = 0
    tags[text + cond : text + cond + audio] = 2
    tags[text + cond + audio : used] = 0
    mask = np.zeros(seq_len, dtype=bool)
    mask[text + cond : used] = True
    return tags, mask, (0, used, seq_len)
