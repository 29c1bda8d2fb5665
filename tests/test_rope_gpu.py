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
    [(37, 5, 128, 128, 1e-6), (64, 3, 128, 64, 1e-5), (20, 4, 64, 64, 1e-6), (9, 2, 64, 32, 1e-6), (5, 3, 128, 0, 1e-6)],
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
