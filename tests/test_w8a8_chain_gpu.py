"""The W8A8 enablement chain on the GPU (the drop-in for
src/taomate_hd/inference/w8a8.py:148-336 and its call sites
model/layers.py:355-358, model/weight_loading.py:154-158,
inference/acceleration.py:230-245): streamed row-chunked loading gives the
bits of whole-matrix quantization, and the projections it enables, called the
way the reference's ``_linear`` calls them (distributed/linear.py:54-68), are
bit-exact against the oracle."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16
from oracle import quant as oq
from tests.helpers import randn_bf16, to_dev

pytestmark = pytest.mark.gpu


def _expected(x, w):
    qx, sx = oq.token_quant(x)
    qw, sw = oq.weight_quant(w)
    return oq.scaled_mm_epilogue(oq.int_gemm(qx, qw), sx, sw, None)


@pytest.mark.parametrize("max_bytes", [1, 3 * 256 * 2, 7 * 256 * 2 + 5, 1 << 23])
def test_stream_load_in_row_chunks_equals_whole_matrix(torch_mod, dev, max_bytes):
    """Chunks of 1, 3, 7 and all rows (the last one ragged) from a host-side
    bf16 source, as the safetensors loader hands it over."""
    torch = torch_mod
    from taomate_hd_amd import (load_cutlass_w8a8_stream_weight_, prepare_cutlass_w8a8_stream_load_slot_,
                                quantize_cutlass_w8a8_weight)

    w = randn_bf16((100, 256), 90, std=0.02)
    w[5] *= 1e-9  # a row whose scale hits the 1e-12 floor
    w[17] = 0.0
    w = bf16.round_f32(w)
    src = bf16.to_torch(w, "cpu")
    m = torch.nn.Module()
    m.weight = torch.nn.Parameter(torch.empty(100, 256, dtype=torch.bfloat16, device=dev), requires_grad=False)
    m.bias = None
    prepare_cutlass_w8a8_stream_load_slot_(torch, m, name="blocks.2.mlp.fc1")
    m.weight.data.fill_(99)  # stale storage: every byte must be written
    m._cutlass_w8a8_weight_scale.fill_(-1.0)
    load_cutlass_w8a8_stream_weight_(torch, m, src, name="blocks.2.mlp.fc1", maximum_temporary_bytes=max_bytes)
    whole_q, whole_s = quantize_cutlass_w8a8_weight(torch, src.to(dev))
    torch.cuda.synchronize()
    assert m._cutlass_w8a8_stream_load_pending is False and m._cutlass_w8a8_stream_loaded is True
    assert torch.equal(m.weight, whole_q)
    assert torch.equal(m._cutlass_w8a8_weight_scale.view(torch.int32), whole_s.view(torch.int32))
    qo, so = oq.weight_quant(w)
    assert np.array_equal(m.weight.cpu().numpy(), qo)
    assert np.array_equal(m._cutlass_w8a8_weight_scale.cpu().numpy().reshape(-1), so.reshape(-1))


def test_enabled_projections_bit_exact_through_the_linear_dispatch(torch_mod, dev):
    """Blocks 2..4 of an 8-block tree: the QKV projections streamed in at load
    time, the FC1 projections converted after loading; then the shared
    workspace.  Each enabled projection, called with the module attributes the
    reference's ``_linear`` reads, equals the oracle bit for bit; the boundary
    blocks keep their bf16 weights."""
    torch = torch_mod
    from taomate_hd_amd import (cutlass_w8a8_linear, enable_h3_cutlass_w8a8_workspace_,
                                load_cutlass_w8a8_stream_weight_, prepare_cutlass_w8a8_stream_load_slot_,
                                quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_)

    hidden, ffn, blocks = 256, 192, 8

    def proj(out_f, in_f):
        m = torch.nn.Module()
        m.weight = torch.nn.Parameter(torch.empty(out_f, in_f, dtype=torch.bfloat16, device=dev), requires_grad=False)
        m.bias = None
        return m

    t = torch.nn.Module()
    t.blocks = torch.nn.ModuleList()
    for _ in range(blocks):
        b = torch.nn.Module()
        b.attn, b.mlp = torch.nn.Module(), torch.nn.Module()
        b.attn.qkv_proj, b.attn.out_proj = proj(3 * hidden, hidden), proj(hidden, hidden)
        b.mlp.fc1, b.mlp.fc2 = proj(2 * ffn, hidden), proj(hidden, ffn)
        t.blocks.append(b)
    sources = {}
    for i, (name, m) in enumerate(sorted((n, m) for n, m in t.named_modules() if hasattr(m, "weight"))):
        sources[name] = randn_bf16(tuple(m.weight.shape), 200 + i, std=0.03)
    streamed = [f"blocks.{i}.attn.qkv_proj" for i in (2, 3, 4)]
    modules = dict(t.named_modules())
    for name in streamed:  # the model constructor's step (layers.py:355-358)
        prepare_cutlass_w8a8_stream_load_slot_(torch, modules[name], name=name)
    for name, w in sources.items():  # the loader (weight_loading.py:154-166)
        m = modules[name]
        if getattr(m, "_cutlass_w8a8_stream_load_pending", None) is True:
            load_cutlass_w8a8_stream_weight_(torch, m, bf16.to_torch(w, "cpu"), name=name, maximum_temporary_bytes=4096)
        else:
            m.weight.data.copy_(bf16.to_torch(w, dev))
    receipt = quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, t, policy="interior_fc1_qkv_v1")
    assert receipt["stream_load_linear_count"] == 3 and receipt["linear_count"] == 6
    enable_h3_cutlass_w8a8_workspace_(torch, t)

    x = randn_bf16((2, 75, hidden), 300)
    x[..., 9] *= 20.0
    x = bf16.round_f32(x)
    xd = to_dev(x, dev)
    for name in receipt["quantized_linear_names"]:
        m = modules[name]
        assert m.weight.dtype == torch.int8
        out = cutlass_w8a8_linear(
            torch, xd, m.weight, m._cutlass_w8a8_weight_scale, bias=None,
            workspace=m._cutlass_w8a8_workspace, weight_t=m._cutlass_w8a8_weight_t,
            weight_scale_t=m._cutlass_w8a8_weight_scale_t,
        )
        torch.cuda.synchronize()
        want = _expected(x.reshape(-1, hidden), sources[name]).reshape(2, 75, -1)
        assert np.array_equal(bf16.from_torch(out).view(np.uint32), want.view(np.uint32)), name
    for name in receipt["bf16_protected_linear_names"]:
        assert modules[name].weight.dtype == torch.bfloat16
        assert np.array_equal(bf16.from_torch(modules[name].weight), sources[name])
