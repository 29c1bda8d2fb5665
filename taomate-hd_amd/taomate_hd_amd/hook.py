"""Per-layer streaming attention hook: drop-in for the reference's
``H3StreamingAttentionHook`` (src/taomate_hd/streaming/attention_hook.py:150-483).

Same constructor, ``activate`` / ``deactivate`` state machine, ``__call__``
keyword signature, validation and errors, document walk and visibility:

* non-live (padding) documents attend to themselves (attention_hook.py:384-390);
* condition queries (rows with ``commit_mask`` False) attend to the
  document's condition rows only;
* media queries attend to [condition, *history prefix, (previous media),
  current media] (``_plan_live_document_kv``, attention_hook.py:31-53);
* CLEAN_COMMIT stages the ``commit_mask`` rows of every layer, FUSED stages
  the previous document's media rows (attention_hook.py:469-482).

What differs is where the bytes go.  The reference concatenates every K/V
part into a dense buffer per call (``_materialize_dense_kv_parts``, :56-97)
and runs SDPA or SageAttention.  Here the history is read in place from the
cache's slots, the chunk's own K/V rows are packed once into a slot (for a
commit, that slot *is* the staged block), and one HIP kernel launch computes
each attention over the segment table.  Query rows are read and output rows
written in place through contiguous ranges or row lists.

Backends: ``"sdpa"`` -> BF16 kernel (serial mode); ``"sage_attn"`` -> INT8-QK
kernel (accelerated mode: smooth-K, per-128-block INT8 Q/K, bf16 P.V).
"""

from __future__ import annotations

from enum import Enum
from typing import Any, Callable

from . import _native, condition
from .attention import QKQuantWorkspace, segment_attention
from .kvcache import HeadMajorRingKVCache
from .profiling import ComponentTimer, maybe_region
from .rope import fused_qkv_qk_norm_rope_stage_
from .slots import SlotPool, SlotView

ATTENTION_BACKENDS = ("sdpa", "sage_attn")


class HookMode(str, Enum):
    """attention_hook.py:10-14."""

    IDLE = "idle"
    NOISY = "noisy"
    CLEAN_COMMIT = "clean_commit"
    FUSED_PROGRESS_DENOISE = "fused_progress_denoise"


def _live_documents_from_mask_or_hint(
    *, boundaries: tuple[int, ...], commit_mask: Any, live_documents_hint: tuple[int, ...] | None
) -> tuple[int, ...]:
    """Resolve target documents (attention_hook.py:118-147)."""
    if live_documents_hint is None:
        return tuple(
            index
            for index, (start, stop) in enumerate(zip(boundaries, boundaries[1:]))
            if bool(commit_mask[start:stop].any().item())
        )
    if not isinstance(live_documents_hint, tuple):
        raise TypeError("live document hint must be a tuple")
    document_count = len(boundaries) - 1
    if any(
        isinstance(index, bool) or not isinstance(index, int) or index < 0 or index >= document_count
        for index in live_documents_hint
    ):
        raise ValueError("live document hint contains an invalid document index")
    if tuple(sorted(set(live_documents_hint))) != live_documents_hint:
        raise ValueError("live document hint must be sorted and unique")
    if any(boundaries[index] == boundaries[index + 1] for index in live_documents_hint):
        raise ValueError("live document hint references an empty document")
    return live_documents_hint


class _Rows:
    """A set of packed-sequence rows: a contiguous range or a device row list
    (built from in-range host rows, so its kernels skip the range check)."""

    def __init__(self, torch: Any, absolute: list[int], device: Any) -> None:
        self.count = len(absolute)
        self.start = absolute[0] if absolute else 0
        self.contiguous = bool(absolute) and absolute[-1] - absolute[0] + 1 == len(absolute)
        self.index = None
        if self.count and not self.contiguous:
            self.index = torch.tensor(absolute, dtype=torch.int32, device=device)

    def query_kwargs(self) -> dict[str, Any]:
        if self.index is not None:
            return {"q_rows": self.index, "rows_checked": True}
        return {"q_row0": self.start, "lq": self.count}

    def out_kwargs(self) -> dict[str, Any]:
        if self.index is not None:
            return {"o_rows": self.index}  # covered by query_kwargs' rows_checked
        return {"o_row0": self.start}

    def pack_kwargs(self) -> dict[str, Any]:
        if self.index is not None:
            return {"rows": self.index, "rows_checked": True}
        return {"row0": self.start, "count": self.count}

    def host_rows(self) -> list[int]:
        if self.index is None:
            return list(range(self.start, self.start + self.count))
        return self.index.cpu().tolist()


class StreamingAttentionHook:
    """Consumes post-QK-norm / post-RoPE / post-Ulysses Q/K/V tensors."""

    def __init__(
        self,
        cache: HeadMajorRingKVCache,
        *,
        attention_backend: str = "sdpa",
        condition_attention_cached: Callable[[str, int], bool] | None = None,
        compact_condition_attention_output: Callable[[str, Any], Any] | None = None,
        timer: ComponentTimer | None = None,
    ) -> None:
        if attention_backend not in ATTENTION_BACKENDS:
            raise ValueError(f"unsupported streaming attention backend: {attention_backend}")
        self.cache = cache
        self.attention_backend = attention_backend
        self.mode = HookMode.IDLE
        self.block_index: int | None = None
        self.fused_current_use_sink: bool | None = None
        self.fused_current_recent_blocks: int | None = None
        self._denoise_step_index: int | None = None
        self._live_documents: tuple[int, ...] | None = None
        self._live_document_boundaries: tuple[int, ...] | None = None
        self._fused_previous_media_indices: Any | None = None
        self._live_document_rows: dict[int, tuple[_Rows, _Rows]] = {}
        self._staged_match: dict[int, bool] = {}
        # the condition-cache queries (attention_hook.py:322-324, 445-465): the
        # runtime's own unless injected (condition.resolve)
        if condition_attention_cached is None or compact_condition_attention_output is None:
            resolved_cached, resolved_compact = condition.resolve()
            condition_attention_cached = condition_attention_cached or resolved_cached
            compact_condition_attention_output = compact_condition_attention_output or resolved_compact
        self._condition_attention_cached = condition_attention_cached
        self._compact_output = compact_condition_attention_output
        self._scratch: SlotPool | None = None
        self._prestaged: dict[str, tuple[Any, tuple[int, ...], int, int]] = {}
        self._quant_ws: QKQuantWorkspace | None = None
        self.sage_attn_calls = 0
        self.sage_attn_query_tokens = 0
        self.sage_attn_key_tokens = 0
        self.kernel_calls = 0
        self.timer = timer

    # ---- receipts (attention_hook.py:174-191)
    def sage_attn_receipt(self) -> dict[str, Any] | None:
        if self.attention_backend != "sage_attn":
            return None
        return {
            "backend": "tmhd_attn_fwd_i8qk_gfx950",
            "tensor_layout": "NHD",
            "is_causal": False,
            "qk_quant_granularity": "per_block_128",
            "pv_accum_dtype": "bf16_pv_fp32_accum",
            "smooth_k": True,
            "kernel_calls": self.sage_attn_calls,
            "query_tokens": self.sage_attn_query_tokens,
            "key_tokens": self.sage_attn_key_tokens,
        }

    def attention_backend_receipt(self) -> dict[str, Any] | None:
        return self.sage_attn_receipt()

    # ---- state machine (attention_hook.py:193-234)
    def activate(
        self,
        *,
        mode: HookMode,
        block_index: int,
        fused_current_use_sink: bool | None = None,
        fused_current_recent_blocks: int | None = None,
        denoise_step_index: int | None = None,
    ) -> None:
        if self.mode is not HookMode.IDLE:
            raise RuntimeError("H3 streaming attention hook is already active")
        if block_index != self.cache.committed_blocks:
            raise ValueError("streaming attention block differs from clean history")
        if (
            fused_current_use_sink is not None or fused_current_recent_blocks is not None
        ) and mode is not HookMode.FUSED_PROGRESS_DENOISE:
            raise ValueError("fused current history policy requires fused progress-denoise mode")
        if denoise_step_index is not None and mode not in {HookMode.NOISY, HookMode.FUSED_PROGRESS_DENOISE}:
            raise ValueError("denoise step index requires noisy or fused progress-denoise mode")
        self.mode = mode
        self.block_index = block_index
        self.fused_current_use_sink = fused_current_use_sink
        self.fused_current_recent_blocks = fused_current_recent_blocks
        self._denoise_step_index = denoise_step_index
        self._live_documents = None
        self._live_document_boundaries = None
        self._fused_previous_media_indices = None
        self._live_document_rows = {}
        self._staged_match = {}

    def deactivate(self) -> None:
        for slot, *_ in self._prestaged.values():  # staged but never consumed
            if self._scratch is not None and slot.device == self._scratch.device:
                self._scratch.release(slot)
        self._prestaged = {}
        self.mode = HookMode.IDLE
        self.block_index = None
        self.fused_current_use_sink = None
        self.fused_current_recent_blocks = None
        self._denoise_step_index = None
        self._live_documents = None
        self._live_document_boundaries = None
        self._fused_previous_media_indices = None
        self._live_document_rows = {}
        self._staged_match = {}

    # ---- pre-staging (no counterpart in the reference)
    def preprocess_qkv_(self, layer_name: str, qkv: Any, q_weight: Any, k_weight: Any, cos_sin_cache: Any,
                        positions: Any, eps: float, *, row0: int, count: int) -> Any:
        """``fused_qkv_qk_norm_rope_`` of a layer's merged projection that also
        packs the K/V of tokens ``row0 .. row0 + count`` into a scratch slot.

        The next call of this hook for ``layer_name`` reads that slot in place
        of packing, when the K/V it receives are the K and V thirds of this
        ``qkv`` and the rows it would pack are exactly these (the media rows
        of the live document in the noisy and fused-progress modes); any
        other rows are packed as usual, and the slot is recycled after that
        call either way.  Returns ``qkv``.
        """
        import torch

        if layer_name not in self.cache.contract.layer_names:
            raise ValueError(f"streaming hook reached a non-main attention layer: {layer_name}")
        heads, head_dim = self.cache.contract.local_heads, self.cache.contract.head_dim
        pool = self._pool(torch, qkv.device, heads, head_dim)
        stale = self._prestaged.pop(layer_name, None)
        if stale is not None and stale[0].device == pool.device:
            pool.release(stale[0])
        slot = pool.acquire(int(count))
        try:
            fused_qkv_qk_norm_rope_stage_(qkv, q_weight, k_weight, cos_sin_cache, positions, eps, slot,
                                          row0=int(row0), count=int(count))
        except BaseException:
            pool.release(slot)
            raise
        width = heads * head_dim
        key_at = (_native.ptr(qkv) + 2 * width, _native.ptr(qkv) + 4 * width, int(qkv.stride(0)))
        self._prestaged[layer_name] = (slot, key_at, int(row0), int(count))
        return qkv

    # ---- helpers
    def _pool(self, torch: Any, device: Any, heads: int, head_dim: int) -> SlotPool:
        if self._scratch is None or self._scratch.device != device:
            self._scratch = SlotPool(torch, heads=int(heads), head_dim=int(head_dim), device=device)
        return self._scratch

    def _attend(self, torch: Any, query: Any, q_rows: _Rows, views: list[SlotView], out: Any, scale: float) -> None:
        backend = "bf16" if self.attention_backend == "sdpa" else "i8qk"
        if backend == "i8qk" and self._quant_ws is None:
            self._quant_ws = QKQuantWorkspace(torch)
        segment_attention(
            torch, query, views, scale=scale, backend=backend, out=out, workspace=self._quant_ws,
            timer=self.timer, **q_rows.query_kwargs(), **q_rows.out_kwargs(),
        )
        self.kernel_calls += 1
        if backend == "i8qk":
            self.sage_attn_calls += 1
            self.sage_attn_query_tokens += q_rows.count
            self.sage_attn_key_tokens += sum(v.tokens for v in views)

    def _document_rows(self, torch: Any, index: int, start: int, stop: int, commit_mask: Any) -> tuple[_Rows, _Rows]:
        rows = self._live_document_rows.get(index)
        if rows is None:
            mask = commit_mask[start:stop].detach().cpu().tolist()
            condition = [start + i for i, m in enumerate(mask) if not m]
            media = [start + i for i, m in enumerate(mask) if m]
            rows = (_Rows(torch, condition, commit_mask.device), _Rows(torch, media, commit_mask.device))
            self._live_document_rows[index] = rows
        return rows

    # ---- the hook (attention_hook.py:236-483)
    def __call__(
        self,
        *,
        attention: Any,
        layer_name: str,
        query: Any,
        key: Any,
        value: Any,
        token_tags: Any,
        commit_mask: Any,
        cu_seqlens: Any,
        cu_seqlens_host: tuple[int, ...] | None,
        max_seqlen: int,
        live_documents_hint: tuple[int, ...] | None = None,
    ) -> Any:
        import torch

        del max_seqlen
        if self.mode is HookMode.IDLE:
            raise RuntimeError("patched H3 attention called outside a streaming step")
        if layer_name not in self.cache.contract.layer_names:
            raise ValueError(f"streaming hook reached a non-main attention layer: {layer_name}")
        if any(not torch.is_tensor(item) for item in (query, key, value, token_tags, commit_mask)):
            raise TypeError("H3 streaming Q/K/V and token metadata must be tensors")
        expected_tail = (self.cache.contract.local_heads, self.cache.contract.head_dim)
        if (
            query.ndim != 3
            or key.shape != query.shape
            or value.shape != query.shape
            or tuple(query.shape[1:]) != expected_tail
        ):
            raise ValueError(f"post-Ulysses Q/K/V must be [tokens, {expected_tail[0]}, {expected_tail[1]}]")
        if query.dtype != torch.bfloat16 or not query.is_cuda:
            raise ValueError("official H3 streaming attention requires CUDA bfloat16 Q/K/V")
        if key.dtype != query.dtype or value.dtype != query.dtype:
            raise ValueError("H3 streaming Q/K/V dtypes differ")
        if key.device != query.device or value.device != query.device:
            raise ValueError("H3 streaming Q/K/V devices differ")
        if token_tags.ndim != 1 or token_tags.shape[0] != query.shape[0]:
            raise ValueError("post-Ulysses token tags do not cover Q/K/V rows")
        if commit_mask.ndim != 1 or commit_mask.dtype != torch.bool or commit_mask.shape[0] != query.shape[0]:
            raise ValueError("post-Ulysses clean commit mask does not cover Q/K/V rows")
        if cu_seqlens_host is None:
            boundaries = tuple(int(item) for item in cu_seqlens.tolist())
        else:
            boundaries = tuple(int(item) for item in cu_seqlens_host)
        if (
            len(boundaries) < 2
            or boundaries[0] != 0
            or boundaries[-1] != query.shape[0]
            or any(left > right for left, right in zip(boundaries, boundaries[1:]))
        ):
            raise ValueError("invalid packed H3 sequence boundaries")
        if self._live_documents is None:
            live_documents = _live_documents_from_mask_or_hint(
                boundaries=boundaries, commit_mask=commit_mask, live_documents_hint=live_documents_hint
            )
            self._live_documents = live_documents
            self._live_document_boundaries = boundaries
        else:
            if boundaries != self._live_document_boundaries:
                raise ValueError("packed H3 boundaries changed within one streaming step")
            live_documents = self._live_documents
            if live_documents_hint is not None and live_documents_hint != live_documents:
                raise ValueError("live document hint changed within one streaming step")
        fused = self.mode is HookMode.FUSED_PROGRESS_DENOISE
        expected_live_documents = 2 if fused else 1
        if len(live_documents) != expected_live_documents:
            raise ValueError(
                "streaming session target-document count differs from hook mode: "
                f"expected={expected_live_documents}, actual={len(live_documents)}"
            )
        for t in (query, key, value):
            if t.stride(2) != 1 or t.stride(0) % 8 or t.stride(1) % 8:
                raise ValueError("Q/K/V views must have unit dim stride and 16-byte aligned rows")
        live_document = live_documents[-1]
        previous_live_document = live_documents[0] if fused else None
        scale = float(attention.softmax_scale)
        pool = self._pool(torch, query.device, int(query.shape[1]), int(query.shape[2]))
        acquired: list[Any] = []
        prestaged = self._prestaged.pop(layer_name, None)
        if prestaged is not None:
            if prestaged[0].device != query.device:
                prestaged = None  # staged on another GPU: dropped, never pooled here
            else:
                acquired.append(prestaged[0])
                at = (_native.ptr(key), _native.ptr(value), int(key.stride(0)))
                if at != prestaged[1] or key.stride(1) != int(key.shape[2]):
                    prestaged = None

        def scratch_pack(rows: _Rows) -> SlotView:
            nonlocal prestaged
            if prestaged is not None and rows.index is None and (rows.start, rows.count) == prestaged[2:]:
                view = prestaged[0].view()
                prestaged = None  # one use
                return view
            slot = pool.acquire(rows.count)
            acquired.append(slot)
            with maybe_region(self.timer, "pack"):
                slot.pack(key, value, **rows.pack_kwargs())
            return slot.view()

        # ---- staging first: the staged slot doubles as a K/V segment
        if self.mode is HookMode.CLEAN_COMMIT:
            with maybe_region(self.timer, "stage"):
                self.cache.stage(layer_name, key, value, token_tags, commit_mask)
        elif fused:
            if self._fused_previous_media_indices is None:
                p_start = boundaries[previous_live_document]
                p_stop = boundaries[previous_live_document + 1]
                previous_media = torch.nonzero(commit_mask[p_start:p_stop], as_tuple=False).view(-1)
                self._fused_previous_media_indices = previous_media.add(p_start)
            with maybe_region(self.timer, "stage"):
                self.cache.stage(
                    layer_name, key, value, token_tags, commit_mask,
                    commit_indices=self._fused_previous_media_indices,
                )
        staged_view = self.cache.staged_view(layer_name)

        compact = self._compact_output(layer_name, query)
        out = torch.empty_like(query) if compact is None else None
        try:
            history = self.cache.history_views(layer_name)
            for index, (start, stop) in enumerate(zip(boundaries, boundaries[1:])):
                if start == stop:
                    continue
                if index not in live_documents:
                    doc = _Rows(torch, list(range(start, stop)), query.device)
                    self._emit(torch, compact, out, query, doc, [scratch_pack(doc)], scale, index, start, stop, "document")
                    continue
                condition_rows, media_rows = self._document_rows(torch, index, start, stop, commit_mask)
                condition_view = scratch_pack(condition_rows) if condition_rows.count else None
                # current media: the staged slot when it holds exactly these rows
                if staged_view is not None and (
                    (fused and index == previous_live_document)
                    or (not fused and self._staged_holds(index, media_rows))
                ):
                    current_view = staged_view
                else:
                    current_view = scratch_pack(media_rows) if media_rows.count else None
                previous_view = None
                if fused and index == live_document:
                    prefixes = list(
                        self.cache.fused_current_views(
                            layer_name,
                            **(
                                {}
                                if self.fused_current_recent_blocks is None
                                else {
                                    "use_sink": bool(self.fused_current_use_sink),
                                    "recent_blocks": self.fused_current_recent_blocks,
                                }
                            ),
                        )
                    )
                    previous_view = staged_view
                else:
                    prefixes = list(history)
                cached = bool(self._condition_attention_cached(layer_name, index))
                if condition_rows.count:
                    if cached:
                        if out is not None:
                            self._zero_rows(torch, out, condition_rows)
                    else:
                        self._emit(torch, compact, out, query, condition_rows, [condition_view], scale, index,
                                   start, stop, "condition")
                if media_rows.count:
                    plan = [
                        *([condition_view] if condition_view is not None else []),
                        *prefixes,
                        *([previous_view] if previous_view is not None else []),
                        current_view,
                    ]
                    self._emit(torch, compact, out, query, media_rows, plan, scale, index, start, stop, "media")
        finally:
            for slot in acquired:
                pool.release(slot)
        return out if compact is None else compact.output

    def _emit(self, torch, compact, out, query, rows: _Rows, views, scale, index, start, stop, kind) -> None:
        if compact is None:
            self._attend(torch, query, rows, views, out, scale)
            return
        # compact condition-cache writer: compute into a dense buffer first
        dense = torch.empty((rows.count, int(query.shape[1]), int(query.shape[2])), dtype=query.dtype,
                            device=query.device)
        backend = "bf16" if self.attention_backend == "sdpa" else "i8qk"
        if backend == "i8qk" and self._quant_ws is None:
            self._quant_ws = QKQuantWorkspace(torch)
        segment_attention(torch, query, views, scale=scale, backend=backend, out=dense, o_row0=0,
                          workspace=self._quant_ws, **rows.query_kwargs())
        self.kernel_calls += 1
        if kind == "document":
            compact.write_document(start, stop, dense)
        else:
            relative = (
                torch.arange(rows.start, rows.start + rows.count, device=query.device)
                if rows.index is None
                else rows.index.to(torch.long)
            ) - start
            compact.write_rows(index, kind, start, relative, dense)

    def _staged_holds(self, index: int, rows: _Rows) -> bool:
        """True when the active commit staged exactly ``rows`` (cached per step)."""
        hit = self._staged_match.get(index)
        if hit is None:
            staged = self.cache.staged_rows_host()
            hit = staged is not None and sorted(staged) == rows.host_rows()
            self._staged_match[index] = hit
        return hit

    @staticmethod
    def _zero_rows(torch: Any, out: Any, rows: _Rows) -> None:
        if rows.index is None:
            out[rows.start : rows.start + rows.count].zero_()
        else:
            out.index_fill_(0, rows.index.to(torch.long), 0)


# the reference's class name
H3StreamingAttentionHook = StreamingAttentionHook
