"""Q/K RMSNorm + RoPE in the merged QKV projection: the HIP kernel (through
the C ABI) against the oracle, bit for bit."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16
from oracle import rope as orope

pytestmark = pytest.mark.gpu


def _case(tokens, heads, head_dim, rotary, seed, npos=23):
    rng = np.random.default_rng(seed)
    qkv = bf16.round_f32(rng.standard_normal((tokens, 3 * heads * head_dim)).astype(np.float32) * 3)
    qkv[0, :head_dim] *= 1e4  # a large row and a tiny row
    qkv[-1, head_dim : 2 * head_dim] *= 1e-4
    qkv = bf16.round_f32(qkv)
    qw = bf16.round_f32(1.0 + 0.2 * rng.standard_normal(head_dim).astype(np.float32))
    kw = bf16.round_f32(1.0 + 0.2 * rng.standard_normal(head_dim).astype(np.float32))
    half = rotary // 2
    ang = rng.uniform(-7, 7, (npos, half))
    cache = bf16.round_f32(np.concatenate([np.cos(ang), np.sin(ang)], -1).astype(np.float32))
    pos = rng.integers(0, npos, tokens)
    return qkv, qw, kw, cache, pos


@pytest.mark.parametrize(
    "tokens,heads,head_dim,rotary,eps",
    [(37, 5, 128, 128, 1e-6), (64, 3, 128, 64, 1e-5), (20, 4, 64, 64, 1e-6), (9, 2, 64, 32, 1e-6), (5, 3, 128, 0, 1e-6),
     (33, 6, 128, 96, 1e-6), (11, 7, 64, 40, 1e-6), (3, 1, 128, 8, 0.0)],
)
def test_qkv_norm_rope_bit_exact(torch_mod, dev, tokens, heads, head_dim, rotary, eps):
    torch = torch_mod
    from taomate_hd_amd import fused_qkv_qk_norm_rope_

    qkv, qw, kw, cache, pos = _case(tokens, heads, head_dim, rotary, seed=tokens + heads + rotary)
    t = bf16.to_torch(qkv, dev)
    before_v = t[:, 2 * heads * head_dim :].clone()
    out = fused_qkv_qk_norm_rope_(
        t, bf16.to_torch(qw, dev), bf16.to_torch(kw, dev), bf16.to_torch(cache, dev).reshape(cache.shape[0], rotary),
        torch.tensor(pos, device=dev), eps,
    )
    torch.cuda.synchronize()
    assert out is t
    got = bf16.from_torch(t)
    want = orope.qkv_norm_rope(qkv, qw, kw, cache, pos, eps, heads)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert torch.equal(t[:, 2 * heads * head_dim :], before_v)


def test_qkv_norm_rope_positions_clamped_and_checks(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import fused_qkv_qk_norm_rope_

    qkv, qw, kw, cache, pos = _case(6, 2, 128, 128, seed=9, npos=5)
    pos = np.array([-3, 0, 4, 5, 100, 2])
    t = bf16.to_torch(qkv, dev)
    fused_qkv_qk_norm_rope_(t, bf16.to_torch(qw, dev), bf16.to_torch(kw, dev), bf16.to_torch(cache, dev),
                            torch.tensor(pos, device=dev), 1e-6)
    torch.cuda.synchronize()
    want = orope.qkv_norm_rope(qkv, qw, kw, cache, np.clip(pos, 0, 4), 1e-6, 2)
    assert np.array_equal(bf16.from_torch(t).view(np.uint32), want.view(np.uint32))
    with pytest.raises(ValueError, match="three complete projections"):
        fused_qkv_qk_norm_rope_(t[:, :-8].contiguous(), bf16.to_torch(qw, dev), bf16.to_torch(kw, dev),
                                bf16.to_torch(cache, dev), torch.tensor(pos, device=dev), 1e-6)
    with pytest.raises(ValueError, match="positions do not cover"):
        fused_qkv_qk_norm_rope_(t, bf16.to_torch(qw, dev), bf16.to_torch(kw, dev), bf16.to_torch(cache, dev),
                                torch.tensor(pos[:3], device=dev), 1e-6)


@pytest.mark.parametrize("tokens,heads,head_dim,rotary", [(29, 5, 128, 96), (16, 3, 64, 64), (7, 4, 128, 0), (13, 2, 64, 24)])
def test_qk_norm_rope_bit_exact_strided_views(torch_mod, dev, tokens, heads, head_dim, rotary):
    torch = torch_mod
    from taomate_hd_amd import fused_qk_norm_rope

    qkv, qw, kw, _, _ = _case(tokens, heads, head_dim, rotary, seed=3 * tokens + rotary)
    rng = np.random.default_rng(tokens)
    ang = rng.uniform(-5, 5, (tokens, rotary))  # per-channel tables: both halves differ
    cos = bf16.round_f32(np.cos(ang).astype(np.float32))
    sin = bf16.round_f32(np.sin(ang).astype(np.float32))
    t = bf16.to_torch(qkv, dev)
    width = heads * head_dim
    q = t[:, :width].view(tokens, heads, head_dim)          # strided rows of the merged buffer
    k = t[:, width : 2 * width].view(tokens, heads, head_dim)
    before = t.clone()
    for view, w, part in ((q, qw, 0), (k, kw, 1)):
        out = fused_qk_norm_rope(view, bf16.to_torch(w, dev), bf16.to_torch(cos, dev).reshape(tokens, rotary),
                                 bf16.to_torch(sin, dev).reshape(tokens, rotary), 1e-6)
        torch.cuda.synchronize()
        assert out.is_contiguous() and tuple(out.shape) == (tokens, heads, head_dim)
        x = qkv[:, part * width : (part + 1) * width].reshape(tokens, heads, head_dim)
        want = orope.qk_norm_rope(x, w, cos, sin, 1e-6)
        assert np.array_equal(bf16.from_torch(out).view(np.uint32), want.view(np.uint32))
    assert torch.equal(t, before)  # the source projection is only read
    # float32 tables: rounded to bf16 first, as the reference kernel rounds them on load
    out32 = fused_qk_norm_rope(q, bf16.to_torch(qw, dev), torch.tensor(np.cos(ang), dtype=torch.float32, device=dev),
                               torch.tensor(np.sin(ang), dtype=torch.float32, device=dev), 1e-6)
    want = orope.qk_norm_rope(qkv[:, :width].reshape(tokens, heads, head_dim), qw, cos, sin, 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(bf16.from_torch(out32).view(np.uint32), want.view(np.uint32))


def test_qk_norm_rope_in_place_and_overlap_refused(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import _native

    tokens, heads, head_dim, rotary = 10, 3, 128, 96
    qkv, qw, _, _, _ = _case(tokens, heads, head_dim, rotary, seed=4)
    rng = np.random.default_rng(5)
    ang = rng.uniform(-5, 5, (tokens, rotary))
    cos = bf16.round_f32(np.cos(ang).astype(np.float32))
    sin = bf16.round_f32(np.sin(ang).astype(np.float32))
    width = heads * head_dim
    x = bf16.to_torch(np.ascontiguousarray(qkv[:, :width]), dev)
    w, c, s = bf16.to_torch(qw, dev), bf16.to_torch(cos, dev), bf16.to_torch(sin, dev)
    lib = _native.load()
    stream = _native.stream_ptr(torch, dev)
    st = lib.tmhd_qk_norm_rope(_native.ptr(x), tokens, heads, head_dim, width, _native.ptr(x), width, _native.ptr(w),
                               _native.ptr(c), rotary, _native.ptr(s), rotary, rotary, 1e-6, stream)
    assert st == 0
    torch.cuda.synchronize()
    want = orope.qk_norm_rope(qkv[:, :width].reshape(tokens, heads, head_dim), qw, cos, sin, 1e-6)
    assert np.array_equal(bf16.from_torch(x).reshape(tokens, heads, head_dim).view(np.uint32), want.view(np.uint32))
    # out shifted by one row onto value: refused, nothing launched
    st = lib.tmhd_qk_norm_rope(_native.ptr(x), tokens - 1, heads, head_dim, width, _native.ptr(x) + 2 * width, width,
                               _native.ptr(w), _native.ptr(c), rotary, _native.ptr(s), rotary, rotary, 1e-6, stream)
    assert st != 0 and b"overlaps" in lib.tmhd_last_error()
    st = lib.tmhd_qk_norm_rope(_native.ptr(x), tokens, heads, head_dim, width, _native.ptr(x), width, _native.ptr(w),
                               _native.ptr(c), rotary, _native.ptr(s), rotary, 12, 1e-6, stream)
    assert st != 0 and b"rotary_dim" in lib.tmhd_last_error()


def test_rounding_helpers_exhaustive(torch_mod, dev):
    # all 2^32 patterns: the bf16 conversion equals the reference's integer
    # rounding and the square root is correctly rounded
    torch = torch_mod
    from taomate_hd_amd import _native

    counts = torch.zeros(2, dtype=torch.int64, device=dev)
    _native.check(_native.load().tmhd_selfcheck_rounding(_native.ptr(counts), _native.stream_ptr(torch, dev)),
                  "tmhd_selfcheck_rounding")
    torch.cuda.synchronize()
    assert counts.tolist() == [0, 0]


@pytest.mark.parametrize("tokens,heads,head_dim,rotary", [(21, 5, 128, 96), (8, 2, 64, 64), (4, 3, 128, 0)])
def test_apply_rope_bit_exact(torch_mod, dev, tokens, heads, head_dim, rotary):
    torch = torch_mod
    from taomate_hd_amd import fused_apply_rope

    qkv, _, _, _, _ = _case(tokens, heads, head_dim, rotary, seed=tokens * 7 + rotary)
    rng = np.random.default_rng(tokens + 1)
    ang = rng.uniform(-5, 5, (tokens, rotary))
    cos = bf16.round_f32(np.cos(ang).astype(np.float32))
    sin = bf16.round_f32(np.sin(ang).astype(np.float32))
    width = heads * head_dim
    t = bf16.to_torch(qkv, dev)
    q = t[:, :width].view(tokens, heads, head_dim)
    out = fused_apply_rope(q, bf16.to_torch(cos, dev).reshape(tokens, rotary), bf16.to_torch(sin, dev).reshape(tokens, rotary))
    torch.cuda.synchronize()
    want = orope.apply_rope(qkv[:, :width].reshape(tokens, heads, head_dim), cos, sin)
    assert np.array_equal(bf16.from_torch(out).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize(
    "tokens,heads,head_dim,rotary,row0,count,dst",
    [(200, 3, 128, 96, 37, 130, 64), (64, 2, 128, 128, 0, 64, 0), (90, 4, 64, 40, 5, 0, 0), (150, 2, 64, 64, 20, 77, 128),
     (33, 5, 128, 0, 0, 33, 0)],
)
def test_qkv_norm_rope_stage_equals_norm_rope_then_pack(torch_mod, dev, tokens, heads, head_dim, rotary, row0, count,
                                                        dst):
    """The staged form leaves the projection and the whole slot (data rows,
    zeroed tail, untouched rows) bit-identical to norm + RoPE followed by
    KVSlot.pack of the same rows."""
    torch = torch_mod
    from taomate_hd_amd import fused_qkv_qk_norm_rope_, fused_qkv_qk_norm_rope_stage_
    from taomate_hd_amd.slots import KVSlot

    qkv, qw, kw, cache, pos = _case(tokens, heads, head_dim, rotary, seed=tokens + count, npos=tokens)
    args = (bf16.to_torch(qw, dev), bf16.to_torch(kw, dev), bf16.to_torch(cache, dev).reshape(cache.shape[0], rotary),
            torch.tensor(pos, device=dev), 1e-6)
    slots = []
    for _ in range(2):
        s = KVSlot(torch, heads=heads, head_dim=head_dim, capacity=dst + count + 130, device=dev)
        g = torch.Generator(device=dev).manual_seed(5)
        s.k.copy_(torch.randn(s.k.shape, generator=g, device=dev).to(torch.bfloat16))  # stale contents
        s.vt.copy_(torch.randn(s.vt.shape, generator=g, device=dev).to(torch.bfloat16))
        slots.append(s)
    a = bf16.to_torch(qkv, dev)
    b = a.clone()
    width = heads * head_dim
    fused_qkv_qk_norm_rope_(a, *args)
    view = lambda t, i: t[:, i * width : (i + 1) * width].view(tokens, heads, head_dim)  # noqa: E731
    slots[0].pack(view(a, 1), view(a, 2), row0=row0, count=count, dst=dst)
    out = fused_qkv_qk_norm_rope_stage_(b, *args, slots[1], row0=row0, count=count, dst=dst)
    torch.cuda.synchronize()
    assert out is b and slots[1].tokens == slots[0].tokens == dst + count
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(slots[0].k.view(torch.int16), slots[1].k.view(torch.int16))
    assert torch.equal(slots[0].vt.view(torch.int16), slots[1].vt.view(torch.int16))
    want = orope.qkv_norm_rope(qkv, qw, kw, cache, pos, 1e-6, heads)
    assert np.array_equal(bf16.from_torch(b).view(np.uint32), want.view(np.uint32))
    with pytest.raises(ValueError, match="outside the"):
        fused_qkv_qk_norm_rope_stage_(b, *args, slots[1], row0=tokens - 1, count=2)
