"""Host logic of the W8A8 enablement chain (the drop-in for
src/taomate_hd/inference/w8a8.py:76-336) on a stub module tree shaped like the
DiT's blocks, without a GPU: selection, flags, validation errors and receipts.
The GPU half (the quantization itself) is in test_w8a8_chain_gpu.py."""

from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")
nn = torch.nn

# keys of the reference's two receipts (w8a8.py:164-172, 310-336)
QUANTIZE_RECEIPT_KEYS = {
    "schema", "format", "scope", "policy", "projection_set", "quantized_projection_suffixes",
    "activation_scale", "weight_scale", "kernel", "eligible_linear_count", "linear_count",
    "stream_load_linear_count", "bf16_protected_linear_count", "quantized_linear_names",
    "bf16_protected_linear_names", "bf16_boundary_block_indices", "source_weight_bytes",
    "quantized_weight_bytes", "eligible_source_weight_bytes", "eligible_weight_fraction",
    "bf16_projection_suffixes", "lora_branch", "base_teacher_adapter_bypass",
    "base_teacher_base_precision", "runtime_state",
}
WORKSPACE_RECEIPT_KEYS = {
    "schema", "linear_count", "workspace_count_per_rank", "allocation_policy",
    "activation_quantization", "weight_quantization", "arithmetic_order_changed",
}


class _Proj(nn.Module):
    def __init__(self, out_f: int, in_f: int, bias: bool = False, dtype=torch.bfloat16) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.zeros(out_f, in_f, dtype=dtype), requires_grad=False)
        self.bias = nn.Parameter(torch.zeros(out_f, dtype=dtype)) if bias else None


class _Lora(nn.Module):
    """A LoRA wrapper: the projection it adapts is ``base``."""

    def __init__(self, base: nn.Module) -> None:
        super().__init__()
        self.base = base
        self.lora_a = nn.Parameter(torch.zeros(2, base.weight.shape[1]))


class _Block(nn.Module):
    def __init__(self, hidden: int, ffn: int, lora_qkv: bool = False) -> None:
        super().__init__()
        self.attn = nn.Module()
        qkv = _Proj(3 * hidden, hidden)
        self.attn.qkv_proj = _Lora(qkv) if lora_qkv else qkv
        self.attn.out_proj = _Proj(hidden, hidden)
        self.mlp = nn.Module()
        self.mlp.fc1 = _Proj(2 * ffn, hidden)
        self.mlp.fc2 = _Proj(hidden, ffn)


def _tree(blocks: int = 8, hidden: int = 64, ffn: int = 96) -> nn.Module:
    t = nn.Module()
    t.blocks = nn.ModuleList([_Block(hidden, ffn, lora_qkv=(i == 3)) for i in range(blocks)])
    return t


def _mark_loaded(module: nn.Module) -> None:
    """What a finished streamed load leaves behind (flags only: no GPU here)."""
    module._cutlass_w8a8_stream_load_pending = False
    module._cutlass_w8a8_stream_loaded = True


def test_require_returns_the_hip_op_namespace():
    from taomate_hd_amd import require_vllm_cutlass_w8a8

    backend = require_vllm_cutlass_w8a8()
    assert callable(backend.scaled_int8_quant) and callable(backend.cutlass_scaled_mm)
    assert require_vllm_cutlass_w8a8() is backend  # cached like the reference's


def test_prepare_stream_load_slot_replaces_weight_and_sets_flags():
    from taomate_hd_amd import prepare_cutlass_w8a8_stream_load_slot_

    m = _Proj(48, 64)
    prepare_cutlass_w8a8_stream_load_slot_(torch, m, name="blocks.2.mlp.fc1")
    assert m.weight.dtype == torch.int8 and tuple(m.weight.shape) == (48, 64) and not m.weight.requires_grad
    assert m._cutlass_w8a8_weight_scale.dtype == torch.float32 and tuple(m._cutlass_w8a8_weight_scale.shape) == (48, 1)
    assert "_cutlass_w8a8_weight_scale" not in m.state_dict()  # not persistent
    assert m._cutlass_w8a8_stream_load_pending is True and m._cutlass_w8a8_stream_loaded is False
    assert m._cutlass_w8a8_source_weight_bytes == 48 * 64 * 2
    with pytest.raises(RuntimeError, match="already owns CUTLASS W8A8 storage"):
        prepare_cutlass_w8a8_stream_load_slot_(torch, m, name="x")
    pre = _Proj(8, 64, dtype=torch.int8)  # an INT8 weight the constructor allocated
    prepare_cutlass_w8a8_stream_load_slot_(torch, pre, name="pre")
    assert pre._cutlass_w8a8_stream_load_pending is True
    with pytest.raises(TypeError, match="uninitialized BF16 or INT8"):
        prepare_cutlass_w8a8_stream_load_slot_(torch, _Proj(8, 64, dtype=torch.float32), name="f32")
    with pytest.raises(RuntimeError, match="bias-free"):
        prepare_cutlass_w8a8_stream_load_slot_(torch, _Proj(8, 64, bias=True), name="b")


def test_stream_load_validation_before_any_work():
    from taomate_hd_amd import load_cutlass_w8a8_stream_weight_, prepare_cutlass_w8a8_stream_load_slot_

    src = torch.zeros(48, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no pending CUTLASS W8A8 stream load"):
        load_cutlass_w8a8_stream_weight_(torch, _Proj(48, 64), src, name="n")
    m = _Proj(48, 64)
    prepare_cutlass_w8a8_stream_load_slot_(torch, m, name="n")
    with pytest.raises(TypeError, match="dtype differs"):
        load_cutlass_w8a8_stream_weight_(torch, m, src.float(), name="n")
    with pytest.raises(ValueError, match="shape differs"):
        load_cutlass_w8a8_stream_weight_(torch, m, src[:40], name="n")
    with pytest.raises(ValueError, match="maximum_temporary_bytes"):
        load_cutlass_w8a8_stream_weight_(torch, m, src, name="n", maximum_temporary_bytes=0)
    # storage on the CPU: there is no CPU path, so the load refuses it loudly
    with pytest.raises(ValueError, match="GPU tensor"):
        load_cutlass_w8a8_stream_weight_(torch, m, src, name="n")
    assert m._cutlass_w8a8_stream_load_pending is True  # nothing was marked loaded


def test_quantize_policy_over_streamed_projections_and_receipt():
    from taomate_hd_amd import (enable_h3_cutlass_w8a8_workspace_, prepare_cutlass_w8a8_stream_load_slot_,
                                quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_)

    t = _tree()
    interior = [f"blocks.{i}.{p}" for i in (2, 3, 4) for p in ("attn.qkv_proj", "mlp.fc1")]
    modules = dict(t.named_modules())
    for name in interior:
        m = getattr(modules[name], "base", modules[name])
        prepare_cutlass_w8a8_stream_load_slot_(torch, m, name=name)
    with pytest.raises(RuntimeError, match="blocks.2.attn.qkv_proj has incomplete CUTLASS W8A8 storage"):
        quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, t, policy="interior_fc1_qkv_v1")
    for name in interior:
        _mark_loaded(getattr(modules[name], "base", modules[name]))
    with pytest.raises(ValueError, match="unsupported H3 CUTLASS W8A8 policy"):
        quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, t, policy="other")
    r = quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, t, policy="interior_fc1_qkv_v1")
    assert set(r) == QUANTIZE_RECEIPT_KEYS
    assert r["quantized_linear_names"] == interior  # blocks 0, 1 and 5, 6, 7 stay bf16
    assert r["bf16_boundary_block_indices"] == [0, 1, 5, 6, 7]
    assert r["eligible_linear_count"] == 24 and r["linear_count"] == 6 and r["stream_load_linear_count"] == 6
    assert r["bf16_protected_linear_count"] == 18
    qkv, fc1, fc2 = 192 * 64 * 2, 192 * 64 * 2, 64 * 96 * 2
    assert r["source_weight_bytes"] == 3 * (qkv + fc1)
    assert r["quantized_weight_bytes"] == 3 * (qkv + fc1) // 2
    assert r["eligible_source_weight_bytes"] == 8 * (qkv + fc1 + fc2)
    assert r["eligible_weight_fraction"] == pytest.approx(3 * (qkv + fc1) / (8 * (qkv + fc1 + fc2)))
    assert modules["blocks.0.attn.qkv_proj"].weight.dtype == torch.bfloat16
    assert modules["blocks.4.mlp.fc2"].weight.dtype == torch.bfloat16

    w = enable_h3_cutlass_w8a8_workspace_(torch, t)
    assert set(w) == WORKSPACE_RECEIPT_KEYS and w["linear_count"] == 6
    attached = {id(getattr(modules[n], "base", modules[n])._cutlass_w8a8_workspace) for n in interior}
    assert len(attached) == 1  # one workspace per model
    m = modules["blocks.3.attn.qkv_proj"].base  # behind the LoRA wrapper
    assert m._cutlass_w8a8_weight_t.data_ptr() == m.weight.data_ptr() and m._cutlass_w8a8_weight_t.stride() == (1, 64)
    assert tuple(m._cutlass_w8a8_weight_scale_t.shape) == (1, 192)
    assert not hasattr(modules["blocks.0.mlp.fc1"], "_cutlass_w8a8_workspace")


def test_quantize_policy_validation_and_candidate_types():
    from taomate_hd_amd import enable_h3_cutlass_w8a8_workspace_, quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_

    with pytest.raises(RuntimeError, match="requires quantized H3 linears"):
        enable_h3_cutlass_w8a8_workspace_(torch, _tree())
    t = _tree()
    t.blocks[2].mlp.fc1.bias = nn.Parameter(torch.zeros(192, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="blocks.2.mlp.fc1 expected a bias-free H3 projection"):
        quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, t, policy="interior_fc1_qkv_v1")
    t = _tree()
    t.blocks[4].attn.qkv_proj.weight = nn.Parameter(torch.zeros(192, 64), requires_grad=False)
    with pytest.raises(TypeError, match="blocks.4.attn.qkv_proj expected BF16 weight"):
        quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, t, policy="interior_fc1_qkv_v1")
    # candidates restricted to given classes: none of these is one
    with pytest.raises(ValueError, match="requires projection candidates"):
        quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, _tree(), policy="interior_fc1_qkv_v1",
                                                            linear_types=(nn.Linear,))
    # a module without a 2-D weight is no candidate
    t = _tree(blocks=7)  # interior blocks 2 and 3
    t.blocks[2].mlp.fc1 = nn.Identity()
    from taomate_hd_amd import prepare_cutlass_w8a8_stream_load_slot_

    modules = dict(t.named_modules())
    for name in ("blocks.2.attn.qkv_proj", "blocks.3.attn.qkv_proj", "blocks.3.mlp.fc1"):
        m = getattr(modules[name], "base", modules[name])
        prepare_cutlass_w8a8_stream_load_slot_(torch, m, name=name)
        _mark_loaded(m)
    r = quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, t, policy="interior_fc1_qkv_v1")
    assert r["eligible_linear_count"] == 20
    assert r["quantized_linear_names"] == ["blocks.2.attn.qkv_proj", "blocks.3.attn.qkv_proj", "blocks.3.mlp.fc1"]
