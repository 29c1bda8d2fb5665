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


def test_noalloc_attention_equals_workspace_entry_point(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import KVSlot, _native

    lib = _native.load()
    stream = _native.stream_ptr(torch, dev)
    # 40 heads x 7 query tiles = 280 items: one round of 256 CUs plus 24 split items;
    # then 5 heads x 3 tiles = 15 items, every one split, with head_dim 64
    for heads, dim, lq, splits in ((40, 128, 1792, [1000, 1560]), (5, 64, 600, [64, 900, 3])):
        n = sum(splits)
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
