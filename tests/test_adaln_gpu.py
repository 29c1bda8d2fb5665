"""RMSNorm / AdaLN-modulate / residual-gate row ops: the HIP kernels (through
the Python drop-ins and the C ABI) against the oracle, bit for bit."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import adaln as oada
from oracle import bf16

pytestmark = pytest.mark.gpu


def _bf(rng, shape, std=1.0, mean=0.0):
    return bf16.round_f32((mean + std * rng.standard_normal(shape)).astype(np.float32))


def _tables(rng, trows, cols):
    # six chunks of one AdaLN projection [trows, 6 * cols], as the DiT block splits them
    proj = _bf(rng, (trows, 6 * cols), 0.3)
    return proj, [proj[:, i * cols : (i + 1) * cols] for i in range(6)]


@pytest.mark.parametrize("rows,cols", [(37, 5376), (5, 64), (13, 1024), (6, 8192), (64, 2056)])
def test_row_ops_bit_exact(torch_mod, dev, rows, cols):
    torch = torch_mod
    from taomate_hd_amd import (fused_gate_add, fused_modulate, fused_residual_gate_rms_norm_modulate,
                                fused_rms_norm, fused_rms_norm_modulate)

    rng = np.random.default_rng(rows + cols)
    x = _bf(rng, (rows, cols), 2.0)
    x[0] *= 300.0  # a large row and a tiny row
    x[-1] *= 1e-3
    x = bf16.round_f32(x)
    br = _bf(rng, (rows, cols))
    w = _bf(rng, (cols,), 0.1, 1.0)
    trows = 3
    proj, (shift_a, scale_a, gate_a, shift_m, scale_m, gate_m) = _tables(rng, trows, cols)
    idx = rng.integers(0, trows, rows)
    td = lambda a: bf16.to_torch(np.ascontiguousarray(a), dev)
    tproj = td(proj)
    view = lambda i: tproj[:, i * cols : (i + 1) * cols]  # strided table views, read without a copy
    ti = torch.tensor(idx, device=dev)
    tx = td(x).reshape(1, rows, cols)  # [batch, rows, cols] as the block passes it
    tb = td(br).reshape(1, rows, cols)
    eq = lambda got, want: np.array_equal(bf16.from_torch(got).reshape(want.shape).view(np.uint32), want.view(np.uint32))

    out = fused_rms_norm(tx, td(w), 1e-6)
    assert tuple(out.shape) == (1, rows, cols)
    assert eq(out, oada.rms_norm(x, w, 1e-6))
    out = fused_rms_norm_modulate(tx, td(w), view(1), view(0), ti, 1e-6)
    assert eq(out, oada.rms_norm_modulate(x, w, scale_a, shift_a, idx, 1e-6))
    hidden, out = fused_residual_gate_rms_norm_modulate(tx, tb, view(2), td(w), view(4), view(3), ti, 1e-5)
    h_want, o_want = oada.residual_gate_rms_norm_modulate(x, br, gate_a, w, scale_m, shift_m, idx, 1e-5)
    assert eq(hidden, h_want) and eq(out, o_want)
    out = fused_modulate(tx, view(3), view(4), ti)
    assert eq(out, oada.modulate(x, scale_m, shift_m, idx))
    out = fused_gate_add(tx, view(5), tb, ti)
    assert eq(out, oada.gate_add(x, gate_m, br, idx))
    torch.cuda.synchronize()


def test_row_ops_index_clamp_and_checks(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import fused_modulate, fused_rms_norm_modulate

    rng = np.random.default_rng(1)
    rows, cols = 6, 512
    x = _bf(rng, (rows, cols))
    scale, shift = _bf(rng, (2, cols), 0.3), _bf(rng, (2, cols), 0.3)
    idx = np.array([-5, 0, 1, 2, 99, 1])
    td = lambda a: bf16.to_torch(np.ascontiguousarray(a), dev)
    out = fused_modulate(td(x), td(shift), td(scale), torch.tensor(idx, device=dev))
    want = oada.modulate(x, scale, shift, np.clip(idx, 0, 1))
    assert np.array_equal(bf16.from_torch(out).view(np.uint32), want.view(np.uint32))
    with pytest.raises(ValueError, match="indices do not cover every row"):
        fused_rms_norm_modulate(td(x), td(np.ones(cols, np.float32)), td(scale), td(shift),
                                torch.tensor(idx[:3], device=dev), 1e-6)
    with pytest.raises(ValueError, match="on the GPU"):  # host indices never reach a kernel
        fused_modulate(td(x), td(shift), td(scale), torch.tensor(idx))
    with pytest.raises(ValueError, match="multiple of 8"):
        fused_modulate(td(x[:, :12]), td(shift[:, :12]), td(scale[:, :12]), torch.tensor(idx, device=dev))
    torch.cuda.synchronize()


@pytest.mark.parametrize("rows,half", [(33, 14336), (7, 64), (130, 1032)])
def test_swiglu_within_one_bf16_ulp(torch_mod, dev, rows, half):
    # tolerance: the reference's sigmoid is its compiler's, so the gate is one
    # bf16 ulp everywhere and bit-identity on at least 99.9% of the elements
    torch = torch_mod
    from taomate_hd_amd import fused_swiglu

    rng = np.random.default_rng(rows + half)
    x = _bf(rng, (rows, 2 * half), 3.0)
    out = fused_swiglu(bf16.to_torch(x, dev).reshape(1, rows, 2 * half))
    torch.cuda.synchronize()
    assert tuple(out.shape) == (1, rows, half)
    got = bf16.from_torch(out).reshape(rows, half)
    want = oada.swiglu(x)
    gi, wi = got.view(np.int32).astype(np.int64), want.view(np.int32).astype(np.int64)
    ulps = np.abs((gi >> 16) - (wi >> 16))
    assert ulps.max() <= 1
    assert np.mean(ulps == 0) >= 0.999


def test_swiglu_every_bf16_gate(torch_mod, dev):
    """All 65,536 bf16 gate patterns against five up values: bit-identical to
    the oracle (sigmoid in float64) wherever the gate is above -87.5; below it
    the exact silu(gate) is under 1e-36 in magnitude and the kernel's output
    may be a signed zero in place of the product; NaN gates give NaN."""
    torch = torch_mod
    from taomate_hd_amd import fused_swiglu

    gates = np.arange(65536, dtype=np.uint32) << 16
    g = np.tile(gates.view(np.float32), 5)
    u = np.repeat(np.array([1.0, 1.5, -3.75, 0.0107, 100.0], dtype=np.float32), 65536)
    u = bf16.round_f32(u)
    x = np.concatenate([g.reshape(-1, 1024), u.reshape(-1, 1024)], 1)  # rows [gate 1024 | up 1024]
    out = fused_swiglu(bf16.to_torch(x, dev).reshape(1, -1, 2048))
    torch.cuda.synchronize()
    got = bf16.from_torch(out).reshape(-1)
    with np.errstate(over="ignore", invalid="ignore"):
        want = oada.swiglu(x).reshape(-1)
    nan_g = np.isnan(g)
    assert np.all(np.isnan(got[nan_g]))
    live = ~nan_g & ~(g <= -87.5)
    assert np.array_equal(got[live].view(np.uint32), want[live].view(np.uint32))
    deep = ~nan_g & (g <= -87.5) & np.isfinite(g)
    bound = 1e-36 * np.maximum(1.0, np.abs(u[deep]))
    assert np.all(np.abs(got[deep]) <= bound) and np.all(np.abs(want[deep]) <= bound)
