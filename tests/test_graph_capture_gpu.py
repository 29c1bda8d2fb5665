"""The attention entry point that allocates nothing, captured into a HIP graph
(the callers it is for): three replays, each after new queries were written
into the captured input buffer by eager work, each bit-identical to an eager
call of the workspace entry point on the same inputs."""

from __future__ import annotations

import pytest

from tests.helpers import key_offset, randn_bf16, to_dev
from tests.test_zz_no_alloc import _args, heads_for_a_split_round, split_parts

pytestmark = pytest.mark.gpu


def test_noalloc_attention_replays_in_a_graph(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import KVSlot, _native

    lib = _native.load()
    cus = int(torch.cuda.get_device_properties(dev).multi_processor_count)
    dim, lq, splits = 128, 1792, [1000, 1560]
    heads = heads_for_a_split_round(cus, 7)  # the last round is split, so the static scratch is used
    n = sum(splits)
    assert split_parts(heads * 7, cus, (n + 63) // 64) > 1
    kd = to_dev(randn_bf16((n, heads, dim), 91, offset=key_offset(heads, dim, 93)), dev)
    vd = to_dev(randn_bf16((n, heads, dim), 92), dev)
    views, off = [], 0
    for c in splits:
        slot = KVSlot(torch, heads=heads, head_dim=dim, capacity=c, device=dev)
        slot.pack(kd, vd, row0=off, count=c)
        views.append(slot.view())
        off += c
    q = to_dev(randn_bf16((lq, heads, dim), 90), dev)  # the captured input buffer
    got = torch.zeros((lq, heads, dim), dtype=torch.bfloat16, device=dev)
    ref = torch.empty_like(got)
    ws = torch.empty(int(lib.tmhd_attn_split_workspace_bytes(dim)), dtype=torch.uint8, device=dev)
    b = _args(torch, q, views, got, dim ** -0.5)

    def eager_reference():
        a = _args(torch, q, views, ref, dim ** -0.5)
        a.split_workspace, a.split_workspace_bytes = _native.ptr(ws), int(ws.numel())
        _native.check(lib.tmhd_attn_fwd_bf16(a, _native.stream_ptr(torch, dev)), "tmhd_attn_fwd_bf16")

    # one eager call first: it looks up the static scratch's address on this device
    _native.check(lib.tmhd_attn_fwd_bf16_noalloc(b, _native.stream_ptr(torch, dev)), "noalloc")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _native.check(lib.tmhd_attn_fwd_bf16_noalloc(b, _native.stream_ptr(torch, dev)), "noalloc (captured)")
    torch.cuda.synchronize()
    for r in range(3):
        q.copy_(to_dev(randn_bf16((lq, heads, dim), 100 + r), dev))  # eager work between replays
        got.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        eager_reference()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), r
