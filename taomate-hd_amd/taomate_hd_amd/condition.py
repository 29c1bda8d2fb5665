"""What the streaming hook asks of the condition cache.

The reference's LOW-stage condition cache (src/taomate_hd/model/condition_cache.py)
lets a request reuse the condition rows of a document whose condition did not
change: the model restores those rows' K/V from the cache, the hook skips
their condition-query attention, and with the compact option the hook writes
its output straight into the cross-layer compact row order.  The hook only
consults two functions per layer call (attention_hook.py:322-324, 445-465):

* ``condition_attention_cached(layer_name, document_index)``
  (condition_cache.py:322-329): True when this layer's plan reuses that
  document's condition rows;
* ``compact_condition_attention_output(layer_name, query)``
  (condition_cache.py:214-228): None, or a writer with ``output``,
  ``write_rows(document, kind, start, rows, value)`` and
  ``write_document(start, stop, value)`` (condition_cache.py:173-211).

The model side (the bank, its K/V restore and hidden-state reuse) is not part
of this path.  ``resolve`` returns the reference's two functions when the hook
runs inside the reference runtime (its module is importable), so the hook
sees the scope that runtime's layers set; otherwise the functions of this
module, whose scope a caller opens with ``condition_layer``.
"""

from __future__ import annotations

import importlib
from contextlib import contextmanager
from contextvars import ContextVar
from typing import Any, Callable, Iterable, Iterator

import numpy as np

_REFERENCE_MODULE = "taomate_hd.model.condition_cache"


class ConditionLayerState:
    """The condition cache's decisions for one attention layer of one forward.

    ``layer``            the layer's module name without the ``.attn`` suffix
                         (what the reference's layer plan records);
    ``cached_documents`` document indices whose condition attention is reused;
    ``compact_rows``     None, or the sorted global rows kept in the compact
                         order (host sequence): the hook's output then has
                         one row per kept row, in that order.
    ``attention_output_compact`` becomes True once the hook has taken a compact
    writer for this layer (the flag the reference sets on its layer plan,
    condition_cache.py:224), so the caller knows the output's row order.
    """

    def __init__(self, layer: str, cached_documents: Iterable[int] = (), compact_rows: Iterable[int] | None = None,
                 seq_len: int | None = None) -> None:
        self.layer = str(layer).removesuffix(".attn")
        self.cached_documents = frozenset(int(d) for d in cached_documents)
        self.compact_rows = None
        self.attention_output_compact = False
        self._to_compact: np.ndarray | None = None
        self._device_rows: dict[tuple[Any, ...], Any] = {}
        if compact_rows is not None:
            rows = np.asarray(list(compact_rows), dtype=np.int64)
            if rows.size and (np.any(np.diff(rows) <= 0) or rows[0] < 0):
                raise ValueError("compact rows must be sorted, unique and non-negative")
            if seq_len is not None and rows.size and rows[-1] >= seq_len:
                raise ValueError("compact rows exceed the packed sequence")
            self.compact_rows = rows

    def matches(self, layer_name: str) -> bool:
        return self.layer == str(layer_name).removesuffix(".attn")

    def to_compact(self, total_rows: int) -> np.ndarray:
        """Global row -> compact position (-1 for rows that are not kept)."""
        if self._to_compact is None or self._to_compact.shape[0] != total_rows:
            table = np.full(total_rows, -1, dtype=np.int64)
            if self.compact_rows[-1:].size and self.compact_rows[-1] >= total_rows:
                raise ValueError("compact rows exceed the attention call's rows")
            table[self.compact_rows] = np.arange(self.compact_rows.size)
            self._to_compact = table
        return self._to_compact


_ACTIVE: ContextVar[ConditionLayerState | None] = ContextVar("tmhd_condition_layer", default=None)


@contextmanager
def condition_layer(state: ConditionLayerState) -> Iterator[ConditionLayerState]:
    """Make ``state`` the condition-cache decision the hook sees while the
    block runs (the role of the reference's ``condition_layer_plan`` scope)."""
    token = _ACTIVE.set(state)
    try:
        yield state
    finally:
        _ACTIVE.reset(token)


class CompactAttentionOutput:
    """Attention rows written in the compact order of ``state.compact_rows``
    (condition_cache.py:173-211): rows that are not kept are never written,
    kept rows nobody writes stay zero."""

    def __init__(self, state: ConditionLayerState, query: Any) -> None:
        self._state = state
        self._total = int(query.shape[0])
        self._device = query.device
        state.to_compact(self._total)
        self.output = query.new_zeros((int(state.compact_rows.size), *query.shape[1:]))

    def _device_index(self, key: tuple[Any, ...], host: np.ndarray) -> Any:
        import torch

        cached = self._state._device_rows.get(key)
        if cached is None:
            cached = torch.from_numpy(host).to(self._device)
            self._state._device_rows[key] = cached
        return cached

    def destinations(self, start: int, rows: Any) -> np.ndarray:
        """Compact positions of the document-relative ``rows`` (host array)."""
        rel = np.asarray(rows.detach().cpu().numpy() if hasattr(rows, "detach") else rows, dtype=np.int64)
        dest = self._state.to_compact(self._total)[rel + int(start)]
        if dest.size and dest.min() < 0:
            raise ValueError("attention rows outside the compact row set")
        return dest

    def write_rows(self, document: int, kind: str, start: int, rows: Any, value: Any) -> None:
        key = ("rows", int(document), str(kind), int(start), int(self._total))
        index = self._state._device_rows.get(key)
        if index is None:
            index = self._device_index(key, self.destinations(start, rows))
        self.output.index_copy_(0, index, value)

    def write_document(self, start: int, stop: int, value: Any) -> None:
        key = ("document", int(start), int(stop), int(self._total))
        pair = self._state._device_rows.get(key)
        if pair is None:
            kept = self._state.compact_rows
            sel = np.nonzero((kept >= start) & (kept < stop))[0]
            pair = (self._device_index(key + ("dst",), sel), self._device_index(key + ("src",), kept[sel] - start))
            self._state._device_rows[key] = pair
        dst, src = pair
        self.output.index_copy_(0, dst, value.index_select(0, src))


def condition_attention_cached(layer_name: str, document_index: int) -> bool:
    """condition_cache.py:322-329."""
    state = _ACTIVE.get()
    return bool(state is not None and state.matches(layer_name) and int(document_index) in state.cached_documents)


def compact_condition_attention_output(layer_name: str, query: Any) -> CompactAttentionOutput | None:
    """condition_cache.py:214-228."""
    state = _ACTIVE.get()
    if state is None or state.compact_rows is None or not state.matches(layer_name):
        return None
    state.attention_output_compact = True
    return CompactAttentionOutput(state, query)


def resolve() -> tuple[Callable[[str, int], bool], Callable[[str, Any], Any]]:
    """The pair of condition-cache queries the hook consults: the reference
    runtime's own when its module is importable (the hook then runs inside
    that runtime, whose layers set the scope), else this module's."""
    try:
        module = importlib.import_module(_REFERENCE_MODULE)
    except ImportError:
        return condition_attention_cached, compact_condition_attention_output
    return module.condition_attention_cached, module.compact_condition_attention_output
