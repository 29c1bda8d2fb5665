"""Calls in flight on two streams at once use separate scratch (the attention's
split workspace and INT8-QK operands, the W8A8 activation arena and the
GEMM's split workspace are kept per (device, stream)): each stream's results
equal, bit for bit, the same call run alone."""

from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import key_offset, randn_bf16, to_dev

pytestmark = pytest.mark.gpu


def _views(torch, dev, k, v, splits):
    from taomate_hd_amd import KVSlot

    views, off = [], 0
    kd, vd = to_dev(k, dev), to_dev(v, dev)
    for n in splits:
        slot = KVSlot(torch, heads=k.shape[1], head_dim=k.shape[2], capacity=n, device=dev)
        slot.pack(kd, vd, row0=off, count=n)
        views.append(slot.view())
        off += n
    return views


@pytest.mark.parametrize("backend", ["bf16", "i8qk"])
def test_attention_on_two_streams_matches_single_stream(torch_mod, dev, backend):
    torch = torch_mod
    from taomate_hd_amd import segment_attention

    heads, dim, lq, splits = 3, 128, 600, [700, 900]  # 9 items: the split round runs
    cases = []
    for c in range(2):
        n = sum(splits)
        q = to_dev(randn_bf16((lq, heads, dim), 60 + 10 * c), dev)
        k = randn_bf16((n, heads, dim), 61 + 10 * c, offset=key_offset(heads, dim, 63 + 10 * c))
        v = randn_bf16((n, heads, dim), 62 + 10 * c)
        cases.append((q, _views(torch, dev, k, v, splits)))
    alone = [segment_attention(torch, q, views, scale=dim ** -0.5, backend=backend) for q, views in cases]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev) for _ in range(2)]  # default priority
    outs = [[], []]
    for _ in range(4):  # interleaved launches keep both streams busy at once
        for i, (q, views) in enumerate(cases):
            with torch.cuda.stream(streams[i]):
                outs[i].append(segment_attention(torch, q, views, scale=dim ** -0.5, backend=backend))
    torch.cuda.synchronize()
    for i in range(2):
        for o in outs[i]:
            assert torch.equal(o.view(torch.int16), alone[i].view(torch.int16))


def test_w8a8_linear_on_two_streams_matches_single_stream(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import W8A8Workspace, cutlass_w8a8_linear, quantize_cutlass_w8a8_weight

    m, k, n = 15 * 256 - 100, 1024, 18 * 256 - 32  # 270 tiles: the split round runs
    ws = W8A8Workspace(torch)
    cases = []
    for c in range(2):
        x = to_dev(randn_bf16((m, k), 70 + c), dev)
        w = to_dev(randn_bf16((n, k), 72 + c, std=0.03), dev)
        qw, sw = quantize_cutlass_w8a8_weight(torch, w)
        bias = to_dev(randn_bf16((n,), 74 + c, std=0.02), dev)
        cases.append((x, qw, sw, bias))
    alone = [cutlass_w8a8_linear(torch, x, qw, sw, bias=b).clone() for x, qw, sw, b in cases]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev) for _ in range(2)]
    outs = [[], []]
    for _ in range(3):
        for i, (x, qw, sw, b) in enumerate(cases):
            with torch.cuda.stream(streams[i]):
                # the workspace's output buffer is reused by the next call on its stream: copy it out
                outs[i].append(cutlass_w8a8_linear(torch, x, qw, sw, bias=b, workspace=ws).clone())
    torch.cuda.synchronize()
    assert ws.nbytes > 0 and len(ws._streams) == 2  # one arena per stream
    for i in range(2):
        for o in outs[i]:
            assert torch.equal(o.view(torch.int16), alone[i].view(torch.int16))
