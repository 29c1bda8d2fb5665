"""Ulysses sequence <-> heads layouts on the GPU (called through the C ABI)
against the oracle's restatement of the reference's layout kernels, bit for
bit, for world sizes 2 and 4 with and without padded heads; the fused norm +
RoPE send against norm + RoPE then the send; and attention through emulated
exchanges on one GPU against attention over the whole sequence."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16
from oracle import ulysses as oul
from tests.helpers import randn_bf16, to_dev

pytestmark = pytest.mark.gpu

LAYOUT_CASES = [
    # heads, head_dim, world, tokens
    (40, 128, 2, 300),
    (28, 128, 4, 257),  # 56 heads over TP 2: 7 local heads per rank at Ulysses 4
    (7, 128, 2, 64),  # 4 local heads, one of them padding
    (10, 64, 4, 130),  # 3 local heads, two padded on the last rank
    (5, 128, 4, 33),  # the last rank holds only padding
]


def _merged(tokens, heads, dim, seed, extra=0):
    """bf16 merged projection [T, 3 H D] as a strided view (row stride 3 H D + extra)."""
    x = randn_bf16((tokens, 3 * heads * dim + extra), seed)
    return x, x[:, : 3 * heads * dim]


@pytest.mark.parametrize("token_major", [False, True])
@pytest.mark.parametrize("heads,dim,world,tokens", LAYOUT_CASES)
def test_qkv_send_bit_exact(torch_mod, dev, heads, dim, world, tokens, token_major):
    torch = torch_mod
    from taomate_hd_amd import ulysses

    full, x = _merged(tokens, heads, dim, 1 + heads, extra=8)
    xd = to_dev(full, dev)[:, : 3 * heads * dim]
    out = ulysses.qkv_send_layout(xd, num_heads=heads, head_dim=dim, world_size=world, token_major=token_major)
    out2 = torch.full_like(out, 5.0)  # into a caller buffer with stale contents (padding must be written)
    ulysses.qkv_send_layout(xd, num_heads=heads, head_dim=dim, world_size=world, token_major=token_major, out=out2)
    torch.cuda.synchronize()
    want = (oul.qkv_send_token_major if token_major else oul.qkv_send)(np.ascontiguousarray(x), heads, dim, world)
    assert np.array_equal(bf16.from_torch(out), want)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


@pytest.mark.parametrize("heads,dim,world,tokens", LAYOUT_CASES)
def test_receive_layouts_bit_exact(torch_mod, dev, heads, dim, world, tokens):
    torch = torch_mod
    from taomate_hd_amd import ulysses

    local = oul.local_heads(heads, world)
    recv = randn_bf16((world, 3, tokens, local, dim), 7 + heads)
    merged = ulysses.qkv_receive_layout(to_dev(recv, dev))
    att = randn_bf16((world, tokens, local, dim), 8 + heads)
    big = torch.full((tokens, heads + 3, dim + 8), 9.0, dtype=torch.bfloat16, device=dev)
    view = big[:, 1 : heads + 1, :dim]  # strided output: untouched around it
    ulysses.attention_receive_layout(to_dev(att, dev), num_heads=heads, out=view)
    torch.cuda.synchronize()
    want = oul.qkv_receive(recv)  # [3, U T, L, D]
    got = bf16.from_torch(merged).reshape(world * tokens, 3, local, dim).transpose(1, 0, 2, 3)
    assert np.array_equal(got, want)
    got_att = bf16.from_torch(big)
    assert np.array_equal(got_att[:, 1 : heads + 1, :dim], oul.attention_receive(att, heads))
    assert np.all(got_att[:, 0] == 9.0) and np.all(got_att[:, heads + 1 :] == 9.0) and np.all(got_att[:, :, dim:] == 9.0)


@pytest.mark.parametrize("token_major", [False, True])
@pytest.mark.parametrize("heads,dim,world,tokens,rotary", [(28, 128, 4, 257, 96), (7, 128, 2, 100, 128),
                                                           (10, 64, 4, 130, 32)])
def test_norm_rope_send_equals_norm_rope_then_send(torch_mod, dev, heads, dim, world, tokens, rotary, token_major):
    torch = torch_mod
    from taomate_hd_amd import fused_qkv_qk_norm_rope_, ulysses

    rng = np.random.default_rng(heads + dim)
    x = to_dev(randn_bf16((tokens, 3 * heads * dim), 20 + heads), dev)
    qw = bf16.to_torch(bf16.round_f32(1.0 + 0.1 * rng.standard_normal(dim).astype(np.float32)), dev)
    kw = bf16.to_torch(bf16.round_f32(1.0 + 0.1 * rng.standard_normal(dim).astype(np.float32)), dev)
    ang = rng.uniform(-4, 4, (512, rotary // 2))
    table = bf16.to_torch(bf16.round_f32(np.concatenate([np.cos(ang), np.sin(ang)], -1).astype(np.float32)), dev)
    pos = torch.from_numpy(rng.integers(0, 512, tokens)).to(dev)
    before = x.clone()
    fused = ulysses.qkv_norm_rope_send_layout(x, qw, kw, table, pos, 1e-6, world_size=world, token_major=token_major)
    torch.cuda.synchronize()
    assert torch.equal(x.view(torch.int16), before.view(torch.int16))  # the projection is not modified
    fused_qkv_qk_norm_rope_(x, qw, kw, table, pos, 1e-6)
    plain = ulysses.qkv_send_layout(x, num_heads=heads, head_dim=dim, world_size=world, token_major=token_major)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), plain.view(torch.int16))


@pytest.mark.parametrize("token_major", [False, True])
@pytest.mark.parametrize("heads,world", [(8, 2), (10, 4)])
def test_attention_through_emulated_exchanges_equals_whole_sequence(torch_mod, dev, heads, world, token_major):
    """U ranks emulated on one GPU: sequence -> heads, attention of each
    rank's heads over all tokens, heads -> sequence.  Each rank's result
    equals its rows of attention over the whole sequence, bit for bit (every
    (head, query tile) runs the same kernel code on the same rows)."""
    torch = torch_mod
    from taomate_hd_amd import KVSlot, segment_attention, ulysses

    dim, tokens = 128, 192
    local = oul.local_heads(heads, world)
    x = [to_dev(randn_bf16((tokens, 3 * heads * dim), 40 + r), dev) for r in range(world)]
    sends = [ulysses.qkv_send_layout(xi, num_heads=heads, head_dim=dim, world_size=world, token_major=token_major)
             for xi in x]
    outs = []
    for r in range(world):  # the collective: rank r receives chunk r of every send buffer
        received = torch.stack([s[r] for s in sends])
        merged = (received.view(world * tokens, 3 * local * dim) if token_major
                  else ulysses.qkv_receive_layout(received))
        q, k, v = ulysses.qkv_received_views(merged, local_heads=local, head_dim=dim)
        slot = KVSlot(torch, heads=local, head_dim=dim, capacity=world * tokens, device=dev)
        slot.pack(k, v)
        outs.append(segment_attention(torch, q, [slot.view()], scale=dim ** -0.5, split=False))
    back = [ulysses.attention_receive_layout(torch.stack([o.view(world, tokens, local, dim)[r] for o in outs]),
                                             num_heads=heads) for r in range(world)]
    whole = torch.cat(x).view(world * tokens, 3, heads, dim)
    slot = KVSlot(torch, heads=heads, head_dim=dim, capacity=world * tokens, device=dev)
    slot.pack(whole[:, 1], whole[:, 2])
    want = segment_attention(torch, whole[:, 0], [slot.view()], scale=dim ** -0.5, split=False)
    torch.cuda.synchronize()
    for r in range(world):
        assert torch.equal(back[r].view(torch.int16), want[r * tokens : (r + 1) * tokens].view(torch.int16))
