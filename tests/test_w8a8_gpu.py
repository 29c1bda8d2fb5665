"""The W8A8 projection module (workspace, dispatch, torch ops) on the GPU."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16
from oracle import adaln as oada
from oracle import quant as oq
from tests.helpers import randn_bf16, to_dev

pytestmark = pytest.mark.gpu


def _expected(x, w, bias=None):
    qx, sx = oq.token_quant(x)
    qw, sw = oq.weight_quant(w)
    acc = oq.int_gemm(qx, qw)
    return oq.scaled_mm_epilogue(acc, sx, sw, bias)


def test_cutlass_w8a8_linear_paths_bit_exact(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import W8A8Workspace, cutlass_w8a8_linear, linear, quantize_cutlass_w8a8_weight

    x = randn_bf16((3, 50, 512), 70)  # [..., K] activations, flattened to 150 rows
    x[..., 11] *= 20.0
    x = bf16.round_f32(x)
    w = randn_bf16((384, 512), 71, std=0.02)
    bias = randn_bf16((384,), 72, std=0.02)
    qw, sw = quantize_cutlass_w8a8_weight(torch, to_dev(w, dev))
    want = _expected(x.reshape(-1, 512), w).reshape(3, 50, 384)
    xd = to_dev(x, dev)
    out = cutlass_w8a8_linear(torch, xd, qw, sw, bias=None)
    torch.cuda.synchronize()
    assert np.array_equal(bf16.from_torch(out), want)
    ws = W8A8Workspace(torch)
    for rows in (150, 40, 150):  # grow, shrink (reuse), reuse
        xr = xd.reshape(-1, 512)[:rows]
        o2 = cutlass_w8a8_linear(torch, xr, qw, sw, bias=to_dev(bias, dev), workspace=ws)
        torch.cuda.synchronize()
        assert np.array_equal(bf16.from_torch(o2), _expected(x.reshape(-1, 512)[:rows], w, bias))
    # dispatch rule of _linear: with a scale -> W8A8, without -> F.linear
    o3 = linear(torch, xd, qw, None, cutlass_w8a8_weight_scale=sw)
    torch.cuda.synchronize()
    assert np.array_equal(bf16.from_torch(o3), want)
    wd = to_dev(w, dev)
    o4 = linear(torch, xd, wd, None)
    assert o4.dtype == torch.bfloat16 and tuple(o4.shape) == (3, 50, 384)


def test_registered_torch_ops(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import register_torch_ops

    ops = register_torch_ops()
    x = randn_bf16((64, 256), 80)
    w = randn_bf16((128, 256), 81, std=0.02)
    xd = to_dev(x, dev)
    q = torch.empty((64, 256), dtype=torch.int8, device=dev)
    s = torch.empty((64, 1), dtype=torch.float32, device=dev)
    ops.dynamic_scaled_int8_quant(q, xd, s, None)
    from taomate_hd_amd import quantize_weight

    qw, sw = quantize_weight(to_dev(w, dev))
    out = torch.empty((64, 128), dtype=torch.bfloat16, device=dev)
    ops.cutlass_scaled_mm(out, q, qw.t(), s, sw.t(), None)
    torch.cuda.synchronize()
    assert np.array_equal(bf16.from_torch(out), _expected(x, w))


def test_w8a8_projection_full_size_sampled_rows(torch_mod, dev):
    """The 768p projection at full size (12,252 x 5,120 -> 13,824, bf16 bias)
    on the projection workload's distribution (X ~ N(0, 1) with 1% of the
    channels, 51, scaled by 20; W ~ N(0, 0.02)): the whole GEMM runs (whole
    tiles, and the 32-tile last round as 64 x 128 sub-tiles); 24 rows, spread
    over the row tiles (row 11,276 lies in the last round's tiles), are
    checked bit for bit against the oracle (token quantization is per row, so
    sampled rows stand alone)."""
    torch = torch_mod
    from taomate_hd_amd import cutlass_w8a8_linear, quantize_cutlass_w8a8_weight

    m, k, n = 12252, 5120, 13824
    gen = torch.Generator(device=dev).manual_seed(3)
    xd = torch.randn(m, k, generator=gen, device=dev)
    outliers = torch.randperm(k, generator=torch.Generator().manual_seed(6))[: k // 100]
    assert outliers.numel() == 51
    xd[:, outliers.to(dev)] *= 20.0
    xd = xd.to(torch.bfloat16)
    wd = (0.02 * torch.randn(n, k, generator=gen, device=dev)).to(torch.bfloat16)
    bd = (0.02 * torch.randn(n, generator=gen, device=dev)).to(torch.bfloat16)
    qw, sw = quantize_cutlass_w8a8_weight(torch, wd)
    out = cutlass_w8a8_linear(torch, xd, qw, sw, bias=bd)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, m - 1], np.arange(12, m, 512)]))[:24]
    x = bf16.from_torch(xd[torch.tensor(rows, device=dev)].contiguous())
    want = _expected(x, bf16.from_torch(wd), bf16.from_torch(bd))
    got = bf16.from_torch(out[torch.tensor(rows, device=dev)].contiguous())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("m,k,f,with_bias", [(300, 1024, 384, False), (130, 256, 128, False), (3 * 256 + 40, 2048, 1024, False),
                                             (300, 1024, 384, True), (130, 256, 128, True),
                                             (200, 576, 256, True), (70, 320, 128, False)])
def test_fused_fc1_swiglu_equals_two_step(torch_mod, dev, m, k, f, with_bias):
    """FC1 with the SwiGLU epilogue (interleaved gate / up rows) against the
    two-step path (the W8A8 projection, then fused_swiglu), bit for bit; the
    first and last shapes of the first five run the k-split merge, the middle
    one does not; the last two have k an odd multiple of 64, which the fused
    kernel does not take (its projection runs on the 64-byte-block GEMM)."""
    torch = torch_mod
    from taomate_hd_amd import (W8A8Workspace, cutlass_w8a8_linear, cutlass_w8a8_linear_swiglu, fused_swiglu,
                                interleave_swiglu_rows, quantize_cutlass_w8a8_swiglu_weight,
                                quantize_cutlass_w8a8_weight)

    x = to_dev(randn_bf16((m, k), 80 + m), dev)
    w = to_dev(randn_bf16((2 * f, k), 81 + m, std=0.03), dev)
    bias = to_dev(randn_bf16((2 * f,), 82 + m, std=0.5), dev) if with_bias else None
    qw, sw = quantize_cutlass_w8a8_weight(torch, w)
    two_step = fused_swiglu(cutlass_w8a8_linear(torch, x, qw, sw, bias=bias))
    qwi, swi = quantize_cutlass_w8a8_swiglu_weight(torch, w)
    bias_i = None if bias is None else interleave_swiglu_rows(bias)
    fused = cutlass_w8a8_linear_swiglu(torch, x, qwi, swi, bias=bias_i, workspace=W8A8Workspace(torch) if with_bias else None)
    torch.cuda.synchronize()
    assert tuple(fused.shape) == (m, f)
    assert torch.equal(fused.view(torch.int16), two_step.view(torch.int16))
    # the oracle's rounding chain for the projection, then SwiGLU within one bf16 ulp
    proj = _expected(bf16.from_torch(x), bf16.from_torch(w), None if bias is None else bf16.from_torch(bias))
    want = oada.swiglu(proj)
    got = bf16.from_torch(fused)
    ulps = np.abs((got.view(np.int32).astype(np.int64) >> 16) - (want.view(np.int32).astype(np.int64) >> 16))
    assert ulps.max() <= 1 and np.mean(ulps == 0) >= 0.999
