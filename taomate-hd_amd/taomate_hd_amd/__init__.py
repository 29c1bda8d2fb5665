"""taomate_hd_amd: MI355X (gfx950) streaming KV-cache attention for TaoMate-HD.

A drop-in for the reference's per-layer streaming attention hook
(src/taomate_hd/streaming/attention_hook.py), its clean audio-video KV cache
(streaming/cache.py), the session around them (streaming/session.py,
capability.py, policy.py) and the selective W8A8 projection ops
(inference/w8a8.py, distributed/linear.py ``_linear``), plus the DiT block's
fused row ops around each attention call (Q/K norm + RoPE, RMSNorm / AdaLN /
residual gate; inference/fused_kernels.py) and the dense packed attention of
non-streamed forwards (model/layers.py ``_packed_sdpa``).  All compute runs in
the hand-written HIP kernels of libtmhd.so; nothing falls back to the CPU.
"""

from . import _native, condition
from .attention import QKQuantWorkspace, segment_attention
from .capability import (
    STREAM_HOOK_ABI,
    native_stream_attention_hook,
    native_stream_attention_metadata,
    set_native_stream_attention_hook,
    set_official_attention_hook,
    streaming_capability,
)
from .hook import H3StreamingAttentionHook, HookMode, StreamingAttentionHook
from .kvcache import (
    AVKV,
    AUDIO_TOKEN_TAG,
    MAIN_LAYER_NAMES,
    VIDEO_TOKEN_TAG,
    CleanAVKVCache,
    HeadMajorRingKVCache,
    KVContract,
    kv_contract_from_model,
)
from .adaln import (
    fused_gate_add,
    fused_modulate,
    fused_residual_gate_rms_norm_modulate,
    fused_rms_norm,
    fused_rms_norm_modulate,
    fused_swiglu,
)
from .packed import packed_sdpa
from .rope import fused_apply_rope, fused_qk_norm_rope, fused_qkv_qk_norm_rope_, fused_qkv_qk_norm_rope_stage_
from .quant import (
    cutlass_scaled_mm,
    cutlass_scaled_mm_out,
    dynamic_scaled_int8_quant,
    int8_mm_i32,
    quantize_weight,
    quantize_weight_into,
    scaled_int8_quant,
)
from .session import H3StreamingSession, StreamingInferencePolicy, StreamingSession, apply_cross_chunk_cache_policy
from .slots import KVSlot, SlotPool, SlotView, vt_position
from .w8a8 import (
    CutlassW8A8Workspace,
    W8A8Workspace,
    cutlass_w8a8_linear,
    cutlass_w8a8_linear_swiglu,
    enable_h3_cutlass_w8a8_workspace_,
    interleave_swiglu_rows,
    linear,
    load_cutlass_w8a8_stream_weight_,
    prepare_cutlass_w8a8_stream_load_slot_,
    quantize_cutlass_w8a8_swiglu_weight,
    quantize_cutlass_w8a8_weight,
    quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_,
    register_torch_ops,
    require_vllm_cutlass_w8a8,
    resolve_h3_cutlass_w8a8_policy,
)

__all__ = [
    "fused_apply_rope",
    "fused_gate_add",
    "fused_modulate",
    "fused_qk_norm_rope",
    "fused_residual_gate_rms_norm_modulate",
    "fused_rms_norm",
    "fused_rms_norm_modulate",
    "fused_swiglu",
    "packed_sdpa",
    "fused_qkv_qk_norm_rope_",
    "fused_qkv_qk_norm_rope_stage_",
    "_native",
    "AVKV",
    "AUDIO_TOKEN_TAG",
    "CleanAVKVCache",
    "CutlassW8A8Workspace",
    "H3StreamingAttentionHook",
    "H3StreamingSession",
    "HeadMajorRingKVCache",
    "HookMode",
    "KVContract",
    "KVSlot",
    "MAIN_LAYER_NAMES",
    "QKQuantWorkspace",
    "STREAM_HOOK_ABI",
    "SlotPool",
    "SlotView",
    "StreamingAttentionHook",
    "StreamingInferencePolicy",
    "StreamingSession",
    "VIDEO_TOKEN_TAG",
    "W8A8Workspace",
    "apply_cross_chunk_cache_policy",
    "cutlass_scaled_mm",
    "cutlass_scaled_mm_out",
    "cutlass_w8a8_linear",
    "cutlass_w8a8_linear_swiglu",
    "interleave_swiglu_rows",
    "dynamic_scaled_int8_quant",
    "enable_h3_cutlass_w8a8_workspace_",
    "int8_mm_i32",
    "kv_contract_from_model",
    "linear",
    "load_cutlass_w8a8_stream_weight_",
    "native_stream_attention_hook",
    "native_stream_attention_metadata",
    "quantize_cutlass_w8a8_swiglu_weight",
    "prepare_cutlass_w8a8_stream_load_slot_",
    "quantize_cutlass_w8a8_weight",
    "quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_",
    "quantize_weight",
    "quantize_weight_into",
    "register_torch_ops",
    "require_vllm_cutlass_w8a8",
    "resolve_h3_cutlass_w8a8_policy",
    "scaled_int8_quant",
    "segment_attention",
    "set_native_stream_attention_hook",
    "set_official_attention_hook",
    "streaming_capability",
    "vt_position",
]

__version__ = "0.1.0"
