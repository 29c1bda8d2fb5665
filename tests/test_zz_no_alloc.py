"""tmhd_attn_fwd_bf16_noalloc (static scratch, no allocation) against
tmhd_attn_fwd_bf16 with a caller workspace, through the C ABI, bit for bit:
two calls in a row, the second smaller, both with a split last round."""

from __future__ import annotations

import pytest

from tests.helpers import key_offset, randn_bf16, to_dev

pytestmark = pytest.mark.gpu


def _args(torch, q, views, out, scale):
    from taomate_hd_amd import _native

    a = _native.AttnArgs()
    a.q = _native.ptr(q)
    a.q_token_stride, a.q_head_stride = q.stride(0), q.stride(1)
    a.q_rows, a.q_row0, a.lq = None, 0, int(q.shape[0])
    a.o = _native.ptr(out)
    a.o_token_stride, a.o_head_stride = out.stride(0), out.stride(1)
    a.o_rows, a.o_row0 = None, 0
    a.heads, a.head_dim, a.scale = int(q.shape[1]), int(q.shape[2]), float(scale)
    a.n_segments = len(views)
    for i, v in enumerate(views):
        a.seg[i] = v.to_segment()
    return a


def split_parts(items: int, cus: int, key_tiles: int) -> int:
    """Key ranges per item of the last round, as the launch chooses them: as
    many as fit the CUs the whole items leave free, at most 8, each at least
    4 key tiles of 64 long; 1 = no split."""
    rem = items % cus
    if rem == 0:
        return 1
    return max(1, min(cus // rem, 8, key_tiles // 4))


def heads_for_a_split_round(cus: int, query_tiles: int) -> int:
    """Heads whose items (heads x query tiles) fill one round of ``cus`` CUs
    and leave about an eighth of the next one, so that round is split."""
    return (cus + cus // 8 + query_tiles - 1) // query_tiles


def test_noalloc_attention_equals_workspace_entry_point(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import KVSlot, _native

    lib = _native.load()
    stream = _native.stream_ptr(torch, dev)
    cus = int(torch.cuda.get_device_properties(dev).multi_processor_count)
    # one whole round of items plus a split partial one (on 256 CUs: 42 heads x 7
    # query tiles = 294 items); then 5 heads x 3 tiles = 15 items, every one
    # split, with head_dim 64
    cases = ((heads_for_a_split_round(cus, 7), 128, 1792, [1000, 1560]), (5, 64, 600, [64, 900, 3]))
    for heads, dim, lq, splits in cases:
        n = sum(splits)
        items = heads * ((lq + 255) // 256)
        assert split_parts(items, cus, (n + 63) // 64) > 1, (heads, lq, n, cus)  # the static scratch is used
        q = to_dev(randn_bf16((lq, heads, dim), 80 + dim), dev)
        kd = to_dev(randn_bf16((n, heads, dim), 81 + dim, offset=key_offset(heads, dim, 83)), dev)
        vd = to_dev(randn_bf16((n, heads, dim), 82 + dim), dev)
        views, off = [], 0
        for c in splits:
            slot = KVSlot(torch, heads=heads, head_dim=dim, capacity=c, device=dev)
            slot.pack(kd, vd, row0=off, count=c)
            views.append(slot.view())
            off += c
        ref = torch.empty((lq, heads, dim), dtype=torch.bfloat16, device=dev)
        got = torch.full((lq, heads, dim), 7.0, dtype=torch.bfloat16, device=dev)
        ws = torch.empty(int(lib.tmhd_attn_split_workspace_bytes(dim)), dtype=torch.uint8, device=dev)
        a = _args(torch, q, views, ref, dim ** -0.5)
        a.split_workspace, a.split_workspace_bytes = _native.ptr(ws), int(ws.numel())
        _native.check(lib.tmhd_attn_fwd_bf16(a, stream), "tmhd_attn_fwd_bf16")
        b = _args(torch, q, views, got, dim ** -0.5)
        _native.check(lib.tmhd_attn_fwd_bf16_noalloc(b, stream), "tmhd_attn_fwd_bf16_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(ref.view(torch.int16), got.view(torch.int16)), (heads, dim, lq)
        # a caller workspace is refused: the entry point uses its own scratch only
        b.split_workspace, b.split_workspace_bytes = _native.ptr(ws), int(ws.numel())
        assert lib.tmhd_attn_fwd_bf16_noalloc(b, stream) == 1
