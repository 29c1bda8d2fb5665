"""Seeded random sweeps of the bit-exact row kernels against the oracle:
RMSNorm / AdaLN modulate / residual gate / gate-add (random row counts,
widths up to 8,192, table rows, indices, eps) and Q/K RMSNorm + RoPE in the
merged QKV projection (random tokens, heads, head dims, rotary spans,
position tables, eps)."""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import adaln as oada
from oracle import bf16
from oracle import rope as orope

pytestmark = pytest.mark.gpu

# a wider sweep: TMHD_SWEEP_CASES=<cases> TMHD_SWEEP_SEED=<seed offset>
_N = os.environ.get("TMHD_SWEEP_CASES")
_OFF = int(os.environ.get("TMHD_SWEEP_SEED", "0"))
ROW_CASES = [777 + _OFF + c for c in range(int(_N or 20))]
ROPE_CASES = [4040 + _OFF + c for c in range(int(_N or 16))]


def _bf(rng, shape, std=1.0, mean=0.0):
    return bf16.round_f32((mean + std * rng.standard_normal(shape)).astype(np.float32))


@pytest.mark.parametrize("seed", ROW_CASES)
def test_random_row_ops_bit_exact(torch_mod, dev, seed):
    torch = torch_mod
    from taomate_hd_amd import (fused_gate_add, fused_modulate, fused_residual_gate_rms_norm_modulate,
                                fused_rms_norm, fused_rms_norm_modulate)

    rng = np.random.default_rng(seed)
    rows, cols, trows = int(rng.integers(1, 200)), 8 * int(rng.integers(1, 1025)), int(rng.integers(1, 5))
    eps = float(rng.choice([1e-6, 1e-5]))
    x = _bf(rng, (rows, cols), float(rng.choice([0.01, 1.0, 30.0])))
    br = _bf(rng, (rows, cols))
    w = _bf(rng, (cols,), 0.1, 1.0)
    proj = _bf(rng, (trows, 6 * cols), 0.3)
    tables = [proj[:, i * cols : (i + 1) * cols] for i in range(6)]
    idx = rng.integers(0, trows, rows)
    td = lambda a: bf16.to_torch(np.ascontiguousarray(a), dev)
    tproj = td(proj)
    view = lambda i: tproj[:, i * cols : (i + 1) * cols]
    ti = torch.tensor(idx, device=dev)
    tx, tb = td(x), td(br)
    eq = lambda got, want: np.array_equal(bf16.from_torch(got).reshape(want.shape).view(np.uint32), want.view(np.uint32))

    assert eq(fused_rms_norm(tx, td(w), eps), oada.rms_norm(x, w, eps))
    assert eq(fused_rms_norm_modulate(tx, td(w), view(1), view(0), ti, eps),
              oada.rms_norm_modulate(x, w, tables[1], tables[0], idx, eps))
    hidden, out = fused_residual_gate_rms_norm_modulate(tx, tb, view(2), td(w), view(4), view(3), ti, eps)
    h_want, o_want = oada.residual_gate_rms_norm_modulate(x, br, tables[2], w, tables[4], tables[3], idx, eps)
    assert eq(hidden, h_want) and eq(out, o_want)
    assert eq(fused_modulate(tx, view(3), view(4), ti), oada.modulate(x, tables[4], tables[3], idx))
    assert eq(fused_gate_add(tx, view(5), tb, ti), oada.gate_add(x, tables[5], br, idx))
    torch.cuda.synchronize()


@pytest.mark.parametrize("seed", ROPE_CASES)
def test_random_qkv_norm_rope_bit_exact(torch_mod, dev, seed):
    torch = torch_mod
    from taomate_hd_amd import fused_qkv_qk_norm_rope_

    rng = np.random.default_rng(seed)
    tokens, heads, head_dim = int(rng.integers(1, 100)), int(rng.integers(1, 9)), int(rng.choice([64, 128]))
    rotary = 8 * int(rng.integers(0, head_dim // 8 + 1))
    npos, eps = int(rng.integers(1, 50)), float(rng.choice([1e-6, 1e-5]))
    qkv = _bf(rng, (tokens, 3 * heads * head_dim), float(rng.choice([0.05, 3.0, 40.0])))
    qw = _bf(rng, (head_dim,), 0.2, 1.0)
    kw = _bf(rng, (head_dim,), 0.2, 1.0)
    ang = rng.uniform(-7, 7, (npos, rotary // 2))
    cache = bf16.round_f32(np.concatenate([np.cos(ang), np.sin(ang)], -1).astype(np.float32))
    pos = rng.integers(0, npos, tokens)
    t = bf16.to_torch(qkv, dev)
    v_before = t[:, 2 * heads * head_dim :].clone()
    fused_qkv_qk_norm_rope_(t, bf16.to_torch(qw, dev), bf16.to_torch(kw, dev),
                            bf16.to_torch(cache, dev).reshape(npos, rotary), torch.tensor(pos, device=dev), eps)
    torch.cuda.synchronize()
    want = orope.qkv_norm_rope(qkv, qw, kw, cache, pos, eps, heads)
    assert np.array_equal(bf16.from_torch(t).view(np.uint32), want.view(np.uint32))
    assert torch.equal(t[:, 2 * heads * head_dim :], v_before)  # V is left alone
