"""Segment attention: the functional entry to the HIP attention kernels.

``segment_attention`` computes ``softmax(q k^T * scale) v`` for a selection of
token-major query rows over an ordered table of slot segments (no mask), as
``torch.nn.functional.scaled_dot_product_attention(..., is_causal=False)``
does over the concatenated K/V in the reference
(src/taomate_hd/streaming/attention_hook.py:100-115).  ``backend="i8qk"`` runs
the SageAttention-style variant (smooth-K, per-128-block INT8 Q/K, bf16 P.V;
ref attention_hook.py:335-371, inference/sage_value_padding.py:79-97).
"""

from __future__ import annotations

from typing import Any, Sequence

from . import _native
from .profiling import ComponentTimer, maybe_region
from .slots import KV_TILE, KVSlot, SlotView, round_up, vt_columns

BACKENDS = ("bf16", "i8qk")


class QKQuantWorkspace:
    """Grow-only INT8-QK operand storage, keyed by (device, stream).

    Work on one stream is ordered, so a call may reuse the buffers of the
    previous call on that stream without synchronising.  ``nbytes`` reports
    what it holds and ``release`` returns it to the allocator.
    """

    def __init__(self, torch: Any) -> None:
        self._torch = torch
        self._buffers: dict[tuple[Any, ...], dict[str, Any]] = {}

    @property
    def nbytes(self) -> int:
        return sum(int(t.numel()) * t.element_size() for store in self._buffers.values() for t in store.values())

    def release(self) -> None:
        self._buffers.clear()

    def _grow(self, store: dict[str, Any], name: str, numel: int, dtype: Any, device: Any) -> Any:
        buf = store.get(name)
        if buf is None or buf.numel() < numel:
            buf = self._torch.empty(max(numel, 1), dtype=dtype, device=device)
            store[name] = buf
        return buf

    def quant_struct(self, *, heads: int, head_dim: int, lq: int, tokens: Sequence[int], device: Any) -> tuple[Any, dict[str, Any]]:
        torch = self._torch
        key = (str(device), _native.stream_ptr(torch, device))
        store = self._buffers.setdefault(key, {})
        qcap = round_up(max(lq, 1), _native.QUERY_TILE)
        caps = [round_up(t, KV_TILE) for t in tokens]
        nblk = [round_up(c, _native.QUANT_BLOCK) // _native.QUANT_BLOCK for c in caps]
        # 256-byte aligned carve-out offsets inside one int8 buffer and one fp32 buffer
        k_off, total = [], 0
        for c in caps:
            k_off.append(total)
            total += round_up(heads * c * head_dim, 256)
        s_off, stotal = [], 0
        for b in nblk:
            s_off.append(stotal)
            stotal += round_up(heads * b, 64)
        q_i8 = self._grow(store, "q_i8", heads * qcap * head_dim, torch.int8, device)
        q_scale = self._grow(store, "q_scale", heads * (qcap // _native.QUANT_BLOCK), torch.float32, device)
        k_i8 = self._grow(store, "k_i8", total, torch.int8, device)
        k_scale = self._grow(store, "k_scale", stotal, torch.float32, device)
        k_mean = self._grow(store, "k_mean", heads * head_dim, torch.bfloat16, device)
        ws = self._grow(store, "mean_ws", heads * head_dim, torch.int64, device)
        qq = _native.QKQuant()
        qq.q_i8 = _native.ptr(q_i8)
        qq.q_scale = _native.ptr(q_scale)
        qq.q_head_stride = qcap * head_dim
        qq.q_scale_head_stride = qcap // _native.QUANT_BLOCK
        for i, c in enumerate(caps):
            qq.k_i8[i] = _native.ptr(k_i8) + k_off[i]
            qq.k_scale[i] = _native.ptr(k_scale) + 4 * s_off[i]
            qq.k_head_stride[i] = c * head_dim
            qq.k_scale_head_stride[i] = nblk[i]
        qq.k_mean = _native.ptr(k_mean)
        qq.mean_workspace = _native.ptr(ws)
        views = {
            "q_i8": q_i8[: heads * qcap * head_dim].view(heads, qcap, head_dim),
            "q_scale": q_scale[: heads * (qcap // _native.QUANT_BLOCK)].view(heads, -1),
            "k_mean": k_mean[: heads * head_dim].view(heads, head_dim),
            "k_i8": [k_i8[o : o + heads * c * head_dim].view(heads, c, head_dim) for o, c in zip(k_off, caps)],
            "k_scale": [k_scale[o : o + heads * b].view(heads, b) for o, b in zip(s_off, nblk)],
        }
        return qq, views


_SPLIT_WORKSPACES: dict[tuple[Any, ...], Any] = {}


def split_workspace(torch: Any, device: Any, head_dim: int) -> Any:
    """Scratch for the key-range split of an attention call's last round.

    One uint8 buffer per (device, stream), grown to what the library asks for
    on that device; calls on one stream are ordered, so they share it.
    """
    need = int(_native.load().tmhd_attn_split_workspace_bytes(int(head_dim)))
    key = (str(device), _native.stream_ptr(torch, device))
    buf = _SPLIT_WORKSPACES.get(key)
    if buf is None or buf.numel() < need:
        buf = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
        _SPLIT_WORKSPACES[key] = buf
    return buf


def split_workspace_bytes() -> int:
    """Bytes held by the split workspaces of every (device, stream) so far."""
    return sum(int(buf.numel()) for buf in _SPLIT_WORKSPACES.values())


def release_split_workspaces() -> None:
    """Return the split workspaces to the allocator (the next call regrows its own)."""
    _SPLIT_WORKSPACES.clear()


def _validate_tokens_major(torch: Any, tensor: Any, name: str) -> None:
    _native.require_device_tensor(torch, tensor, name)
    if tensor.dtype != torch.bfloat16 or tensor.ndim != 3 or tensor.stride(2) != 1:
        raise ValueError(f"{name} must be a [tokens, heads, dim] bf16 view with unit dim stride")


def _row_list(torch: Any, rows: Any, device: Any, limit: int, name: str, checked: bool) -> Any:
    """A row list as a contiguous int32 tensor on ``device`` with entries in
    [0, limit).  The range check reads the list's min / max back (one sync);
    callers whose lists are valid by construction pass ``checked``."""
    if not torch.is_tensor(rows) or rows.device != torch.device(device):
        raise ValueError(f"{name} must be a tensor on the GPU of the rows it indexes")
    if rows.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{name} must be an int32 or int64 tensor")
    rows = rows.reshape(-1)
    if not checked and rows.numel():
        # on the list as given: an int64 entry past 2^31 must not wrap into range
        lo, hi = (int(v) for v in torch.aminmax(rows))
        if lo < 0 or hi >= limit:
            raise ValueError(f"{name} entries must lie in [0, {limit})")
    return rows.to(torch.int32).contiguous()


def _key_sum(torch: Any, lib: Any, view: SlotView, stream: int) -> int:
    """Device address of the exact fixed-point key sums of a slot view (the
    smooth-K mean's term for that segment), memoised on the slot per (row0,
    tokens, stream): a cached block's keys are summed once, not on every call.
    The slot drops the memo whenever it is written."""
    slot = view.slot
    key = (int(view.row0), int(view.tokens), int(stream))
    hit = slot.key_sums.get(key)
    if hit is None:
        seg = view.to_segment()
        hit = torch.empty((slot.heads, slot.head_dim), dtype=torch.int64, device=slot.device)
        _native.check(lib.tmhd_k_fixed_sum(seg.k, seg.k_head_stride, seg.tokens, slot.heads, slot.head_dim,
                                           _native.ptr(hit), stream), "tmhd_k_fixed_sum")
        slot.key_sums[key] = hit
    return _native.ptr(hit)


def _coalesce_segments(torch: Any, segments: list[SlotView], limit: int) -> list[SlotView]:
    """One launch takes at most ``limit`` segments; the reference has no such
    bound (it concatenates every part).  With more, the oldest segments are
    copied, in order, into one temporary slot: their keys stay the same keys,
    so the result is the attention over the same set (the INT8-QK key blocks
    then run over the merged rows, as they run over any segment)."""
    n_merge = len(segments) - limit + 1
    head, rest = segments[:n_merge], segments[n_merge:]
    keys, values = [], []
    for view in head:
        slot, r0, n = view.slot, int(view.row0), int(view.tokens)
        keys.append(slot.k[:, r0 : r0 + n, :].permute(1, 0, 2))
        cols = r0 + vt_columns(torch, n, slot.device)  # r0 is a multiple of 64: whole 16-token groups
        values.append(slot.vt.index_select(2, cols).permute(2, 0, 1))
    key, value = torch.cat(keys, 0).contiguous(), torch.cat(values, 0).contiguous()
    first = head[0].slot
    merged = KVSlot(torch, heads=first.heads, head_dim=first.head_dim, capacity=int(key.shape[0]), device=first.device)
    merged.pack(key, value)
    return [merged.view(), *rest]


def segment_attention(
    torch: Any,
    query: Any,
    segments: Sequence[SlotView],
    *,
    scale: float,
    backend: str = "bf16",
    q_rows: Any | None = None,
    q_row0: int = 0,
    lq: int | None = None,
    out: Any | None = None,
    o_rows: Any | None = None,
    o_row0: int = 0,
    workspace: QKQuantWorkspace | None = None,
    split: bool = True,
    return_quant: bool = False,
    timer: ComponentTimer | None = None,
    rows_checked: bool = False,
) -> Any:
    """Attention of the selected query rows over ``segments`` (in place, no mask).

    Query row ``i`` is ``query[q_rows[i]]`` (or ``query[q_row0 + i]``); its
    output goes to ``out[o_rows[i]]`` (or ``out[o_row0 + i]``).  Without
    ``out`` a new ``[lq, H, D]`` tensor is returned.  ``split`` lets the
    library run the items of a partial last round as key ranges (merged on
    the same stream); results agree with the unsplit run to fp32 rounding.
    Row lists are device tensors; their range is checked (one sync) unless
    ``rows_checked`` says the caller built them in range.
    """
    if backend not in BACKENDS:
        raise ValueError(f"unknown attention backend {backend!r}")
    _validate_tokens_major(torch, query, "query")
    heads, head_dim = int(query.shape[1]), int(query.shape[2])
    keep: list[Any] = []
    if q_rows is not None:
        q_rows = _row_list(torch, q_rows, query.device, int(query.shape[0]), "q_rows", rows_checked)
        keep.append(q_rows)
        n = int(q_rows.numel())
        if lq is not None and int(lq) != n:
            raise ValueError("lq differs from the query row list")
        lq = n
    elif lq is None:
        lq = int(query.shape[0]) - int(q_row0)
    lq = int(lq)
    if out is None:
        out = torch.empty((lq, heads, head_dim), dtype=torch.bfloat16, device=query.device)
        o_rows, o_row0 = None, 0
    _validate_tokens_major(torch, out, "out")
    if tuple(out.shape[1:]) != (heads, head_dim):
        raise ValueError("out heads/dim differ from query")
    if o_rows is not None:
        o_rows = _row_list(torch, o_rows, out.device, int(out.shape[0]), "o_rows", rows_checked)
        keep.append(o_rows)
        if int(o_rows.numel()) != lq:
            raise ValueError("output row list length differs from the query rows")
    elif not (0 <= int(o_row0) and int(o_row0) + lq <= int(out.shape[0])):
        raise ValueError(f"output rows [{o_row0}, {int(o_row0) + lq}) outside out ({int(out.shape[0])} rows)")
    if q_rows is None and not (0 <= int(q_row0) and int(q_row0) + lq <= int(query.shape[0])):
        raise ValueError(f"query rows [{q_row0}, {int(q_row0) + lq}) outside query ({int(query.shape[0])} rows)")
    segments = [s for s in segments if s.tokens > 0]
    if not segments:
        raise ValueError("attention needs at least one key/value token")
    for s in segments:
        if s.slot.heads != heads or s.slot.head_dim != head_dim or s.slot.device != query.device:
            raise ValueError("segment heads/dim/device differ from the query")
    if len(segments) > _native.MAX_SEGMENTS:
        segments = _coalesce_segments(torch, segments, _native.MAX_SEGMENTS)
    args = _native.AttnArgs()
    args.q = _native.ptr(query)
    args.q_token_stride = query.stride(0)
    args.q_head_stride = query.stride(1)
    args.q_rows = _native.ptr(q_rows) if q_rows is not None and lq else None
    args.q_row0 = int(q_row0)
    args.lq = lq
    args.o = _native.ptr(out)
    args.o_token_stride = out.stride(0)
    args.o_head_stride = out.stride(1)
    args.o_rows = _native.ptr(o_rows) if o_rows is not None and lq else None
    args.o_row0 = int(o_row0)
    args.heads = heads
    args.head_dim = head_dim
    args.scale = float(scale)
    args.n_segments = len(segments)
    for i, s in enumerate(segments):
        args.seg[i] = s.to_segment()
    lib = _native.load()
    stream = _native.stream_ptr(torch, query.device)
    if split and lq:
        ws = split_workspace(torch, query.device, head_dim)
        args.split_workspace = _native.ptr(ws)
        args.split_workspace_bytes = int(ws.numel())
    if backend == "bf16":
        with maybe_region(timer, "attention"):
            status = lib.tmhd_attn_fwd_bf16(args, stream)
        _native.check(status, "tmhd_attn_fwd_bf16")
        return out
    if workspace is None:
        workspace = QKQuantWorkspace(torch)
    qq, views = workspace.quant_struct(
        heads=heads, head_dim=head_dim, lq=lq, tokens=[s.tokens for s in segments], device=query.device
    )
    with maybe_region(timer, "qk_quant"):
        for i, seg in enumerate(segments):
            qq.k_sum[i] = _key_sum(torch, lib, seg, stream)
        status = lib.tmhd_qk_smooth_quant(args, qq, stream)
    _native.check(status, "tmhd_qk_smooth_quant")
    with maybe_region(timer, "attention"):
        status = lib.tmhd_attn_fwd_i8qk(args, qq, stream)
    _native.check(status, "tmhd_attn_fwd_i8qk")
    if return_quant:
        return out, views
    return out
