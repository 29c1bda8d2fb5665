"""CPU tests of the C ABI (load, exports, struct layout) and the host logic
(hook/session validation and state machine, W8A8 policy, slot layout)."""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "tmhd.h"


def _declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char \*)\s*(tmhd_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    from taomate_hd_amd import _native

    lib = _native.load()
    declared = _declared_symbols()
    assert len(declared) == 32
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.EXPORTED_SYMBOLS)
    assert _native.version().startswith("tmhd ") and "gfx950" in _native.version()


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_ctypes_structs_match_c_header(tmp_path):
    from taomate_hd_amd import _native

    src = tmp_path / "layout.c"
    fields = {
        "tmhd_kv_segment": [f[0] for f in _native.KVSegment._fields_],
        "tmhd_attn_args": [f[0] for f in _native.AttnArgs._fields_],
        "tmhd_qk_quant": [f[0] for f in _native.QKQuant._fields_],
    }
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "tmhd.h"', "int main(void) {"]
    for struct, names in fields.items():
        lines.append(f'printf("{struct} %zu\\n", sizeof({struct}));')
        for n in names:
            lines.append(f'printf("{struct}.{n} %zu\\n", offsetof({struct}, {n}));')
    lines += ["return 0;", "}"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{REPO / 'include'}", str(src), "-o", str(exe)], check=True)
    out = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines())
    for struct, cls in (("tmhd_kv_segment", _native.KVSegment), ("tmhd_attn_args", _native.AttnArgs), ("tmhd_qk_quant", _native.QKQuant)):
        assert int(out[struct]) == ctypes.sizeof(cls), struct
        for name in fields[struct]:
            assert int(out[f"{struct}.{name}"]) == getattr(cls, name).offset, (struct, name)


def test_invalid_arguments_are_rejected_without_a_gpu():
    from taomate_hd_amd import _native

    lib = _native.load()
    args = _native.AttnArgs()
    args.head_dim = 96
    args.heads = 1
    args.n_segments = 1
    with pytest.raises(ValueError, match="head_dim"):
        _native.check(lib.tmhd_attn_fwd_bf16(args, None), "attn")
    with pytest.raises(ValueError, match="multiple of 64"):
        _native.check(lib.tmhd_gemm_i8_i32(None, None, None, 4, 4, 100, 100, 100, 4, None), "gemm")
    # the SwiGLU GEMM exists only in the kernel with 128-byte k blocks
    with pytest.raises(ValueError, match="multiple of 128"):
        _native.check(lib.tmhd_gemm_w8a8_swiglu_ws(None, None, None, None, None, None, 4, 256, 192, 192, 192, 128,
                                                   None, 0, None), "swiglu gemm")
    with pytest.raises(ValueError, match="cols"):
        _native.check(lib.tmhd_token_quant_i8(None, None, None, 4, 12, 12, None), "quant")
    # a V^T row stride of 2^23 tokens or more is refused (the kernels form row
    # offsets with 24-bit multiplies); lq = 0 launches nothing when it is accepted
    for stride, ok in (((1 << 23) - 64, True), (1 << 23, False)):
        a = _native.AttnArgs()
        a.q = a.o = a.seg[0].k = a.seg[0].vt = 1 << 20
        a.heads, a.head_dim, a.scale, a.n_segments, a.lq = 1, 128, 0.125, 1, 0
        a.seg[0].tokens, a.seg[0].vt_row_stride = 64, stride
        a.seg[0].k_head_stride = a.seg[0].vt_head_stride = 128 * stride
        if ok:
            _native.check(lib.tmhd_attn_fwd_bf16(a, None), "attn")
        else:
            with pytest.raises(ValueError, match="not a slot"):
                _native.check(lib.tmhd_attn_fwd_bf16(a, None), "attn")


def test_vt_position_is_the_mfma_lane_order():
    from taomate_hd_amd import vt_position

    assert [vt_position(t) for t in range(16)] == [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]
    assert all(vt_position(vt_position(t)) == t for t in range(4096))
    # lane group g of 16-key step s reads stored columns 16s + 8g .. +7, which must hold
    # keys 16s + 4g + {0..3} and 16s + 8 + 4g + {0..3} (the S^T accumulator rows of that lane)
    inverse = {vt_position(t): t for t in range(64)}
    for s in range(4):
        for g in range(2):
            keys = [inverse[16 * s + 8 * g + e] for e in range(8)]
            assert keys == [16 * s + 4 * g + e for e in range(4)] + [16 * s + 8 + 4 * g + e for e in range(4)]


def test_live_documents_resolution():
    import torch

    from taomate_hd_amd.hook import _live_documents_from_mask_or_hint

    bounds = (0, 3, 3, 8, 10)
    mask = torch.tensor([False, True, False, False, False, True, False, False, False, False])
    assert _live_documents_from_mask_or_hint(boundaries=bounds, commit_mask=mask, live_documents_hint=None) == (0, 2)
    assert _live_documents_from_mask_or_hint(boundaries=bounds, commit_mask=mask, live_documents_hint=(0, 2)) == (0, 2)
    with pytest.raises(TypeError):
        _live_documents_from_mask_or_hint(boundaries=bounds, commit_mask=mask, live_documents_hint=[0])
    with pytest.raises(ValueError, match="invalid"):
        _live_documents_from_mask_or_hint(boundaries=bounds, commit_mask=mask, live_documents_hint=(5,))
    with pytest.raises(ValueError, match="sorted"):
        _live_documents_from_mask_or_hint(boundaries=bounds, commit_mask=mask, live_documents_hint=(2, 0))
    with pytest.raises(ValueError, match="empty"):
        _live_documents_from_mask_or_hint(boundaries=bounds, commit_mask=mask, live_documents_hint=(1,))


def _hook_and_inputs():
    import torch

    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingAttentionHook

    cache = HeadMajorRingKVCache(KVContract(layer_names=("blocks.0.attn",), local_heads=2, head_dim=64))
    hook = StreamingAttentionHook(cache)
    q = torch.zeros(8, 2, 64, dtype=torch.bfloat16)
    kw = dict(
        attention=type("A", (), {"softmax_scale": 0.125})(), layer_name="blocks.0.attn", query=q, key=q, value=q,
        token_tags=torch.zeros(8, dtype=torch.long), commit_mask=torch.ones(8, dtype=torch.bool),
        cu_seqlens=None, cu_seqlens_host=(0, 8), max_seqlen=8,
    )
    return cache, hook, kw


def test_hook_validation_and_state_machine():
    import torch

    from taomate_hd_amd import HookMode

    cache, hook, kw = _hook_and_inputs()
    with pytest.raises(RuntimeError, match="outside a streaming step"):
        hook(**kw)
    with pytest.raises(ValueError, match="differs from clean history"):
        hook.activate(mode=HookMode.NOISY, block_index=1)
    with pytest.raises(ValueError, match="fused progress-denoise"):
        hook.activate(mode=HookMode.NOISY, block_index=0, fused_current_recent_blocks=2)
    with pytest.raises(ValueError, match="denoise step index"):
        hook.activate(mode=HookMode.CLEAN_COMMIT, block_index=0, denoise_step_index=0)
    hook.activate(mode=HookMode.NOISY, block_index=0)
    with pytest.raises(RuntimeError, match="already active"):
        hook.activate(mode=HookMode.NOISY, block_index=0)
    with pytest.raises(ValueError, match="non-main"):
        hook(**{**kw, "layer_name": "blocks.9.attn"})
    with pytest.raises(ValueError, match=r"\[tokens, 2, 64\]"):
        hook(**{**kw, "query": torch.zeros(8, 3, 64, dtype=torch.bfloat16)})
    with pytest.raises(ValueError, match="CUDA bfloat16"):
        hook(**kw)  # CPU tensors: the HIP path has no CPU fallback
    hook.deactivate()
    with pytest.raises(ValueError):
        type(hook)(cache, attention_backend="flash")


def test_session_state_machine_without_gpu():
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingSession, native_stream_attention_hook

    class Plan:
        phases = ("p0", "p1")

    cache = HeadMajorRingKVCache(KVContract(layer_names=("blocks.0.attn",), local_heads=2, head_dim=64))
    with pytest.raises(TypeError):
        StreamingSession(object())
    session = StreamingSession(Plan(), cache=cache)
    with pytest.raises(RuntimeError, match="context manager"):
        with session.noisy_step(0):
            pass
    with session:
        assert native_stream_attention_hook() is session.hook
        with pytest.raises(RuntimeError, match="already installed"):
            StreamingSession(Plan(), cache=cache).__enter__()
        with pytest.raises(RuntimeError, match="at least one noisy"):
            with session.clean_commit(0):
                pass
        with pytest.raises(ValueError, match="in order"):
            with session.noisy_step(1):
                pass
        with pytest.raises(ValueError, match="unknown streaming block"):
            session.phase(7)
        with session.noisy_step(0) as phase:
            assert phase == "p0" and session.hook.mode.value == "noisy"
        assert session.hook.mode.value == "idle"
        with pytest.raises(ValueError, match="adjacent"):
            with session.fused_clean_commit_denoise(0, 2):
                pass
    assert native_stream_attention_hook() is None


def test_cache_ledger_errors_without_gpu():
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract

    cache = HeadMajorRingKVCache(KVContract(layer_names=("blocks.0.attn",), local_heads=2, head_dim=64))
    with pytest.raises(ValueError, match="order mismatch"):
        cache.begin_clean_commit(1)
    with pytest.raises(RuntimeError, match="no clean commit"):
        cache.commit()
    cache.begin_clean_commit(0)
    with pytest.raises(RuntimeError, match="already active"):
        cache.begin_clean_commit(0)
    with pytest.raises(RuntimeError, match="during a clean commit"):
        cache.retain_sink_and_recent_commits(2)
    with pytest.raises(RuntimeError, match="missing attention layers"):
        cache.commit()
    cache.rollback()
    assert not cache.clean_commit_active and cache.committed_blocks == 0
    with pytest.raises(ValueError, match="non-negative"):
        cache.retain_sink_and_recent_commits(-1)
    with pytest.raises(KeyError):
        cache.history("blocks.3.attn")
    assert cache.history("blocks.0.attn") is None and cache.history_views("blocks.0.attn") == ()


def test_w8a8_policy_hand_derived():
    from taomate_hd_amd import resolve_h3_cutlass_w8a8_policy

    names = [f"blocks.{i}.{s}" for i in range(50) for s in ("attn.qkv_proj", "attn.out_proj", "mlp.fc1", "mlp.fc2")]
    sel = resolve_h3_cutlass_w8a8_policy(names, policy="interior_fc1_qkv_v1")
    assert sel["bf16_boundary_block_indices"] == [0, 1, 47, 48, 49]
    assert len(sel["quantized_linear_names"]) == 45 * 2
    assert "blocks.2.attn.qkv_proj" in sel["quantized_linear_names"]
    assert "blocks.46.mlp.fc1" in sel["quantized_linear_names"]
    assert "blocks.47.mlp.fc1" in sel["bf16_protected_linear_names"]
    assert all(not n.endswith("fc2") for n in sel["quantized_linear_names"])
    with pytest.raises(ValueError):
        resolve_h3_cutlass_w8a8_policy(names, policy="other")


def test_build_recipe_targets_gfx950_without_packed_fp32():
    import importlib.util

    spec = importlib.util.spec_from_file_location("tmhd_build", REPO / "taomate-hd_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert "--offload-arch=gfx950" in mod.HIPCC_FLAGS
    assert "-packed-fp32-ops" in mod.HIPCC_FLAGS


def test_packed_sdpa_boundary_validation_without_gpu():
    import torch
    from taomate_hd_amd import packed_sdpa

    q = torch.zeros((10, 2, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="cumulative lengths are invalid"):
        packed_sdpa(q, q, q, cu_seqlens=torch.tensor([0, 4, 9]), cu_seqlens_host=None, max_seqlen=5, scale=0.1)
    with pytest.raises(ValueError, match="cumulative lengths are invalid"):
        packed_sdpa(q, q, q, cu_seqlens=None, cu_seqlens_host=(0, 6, 4, 10), max_seqlen=6, scale=0.1)
    with pytest.raises(ValueError, match="no live segment"):
        packed_sdpa(q[:0], q[:0], q[:0], cu_seqlens=None, cu_seqlens_host=(0, 0, 0), max_seqlen=0, scale=0.1)
    with pytest.raises(ValueError, match="GPU tensor"):  # valid boundaries: the HIP path is required
        packed_sdpa(q, q, q, cu_seqlens=None, cu_seqlens_host=(0, 4, 10), max_seqlen=6, scale=0.1)


def test_swiglu_row_interleave_layout_without_gpu():
    # gate rows [0, F) then up rows [F, 2F) -> per 256-row tile t: gate 128t.., then up 128t..
    import torch
    from taomate_hd_amd import interleave_swiglu_rows

    f = 384
    rows = torch.arange(2 * f)
    got = interleave_swiglu_rows(rows.view(2 * f, 1)).view(-1).tolist()
    want = []
    for t in range(f // 128):
        want += list(range(128 * t, 128 * t + 128)) + list(range(f + 128 * t, f + 128 * t + 128))
    assert got == want
    assert interleave_swiglu_rows(rows).tolist() == want  # 1-D (bias, scale vectors) too
    with pytest.raises(ValueError, match="multiple of 256"):
        interleave_swiglu_rows(torch.arange(2 * 200))


def test_staged_norm_rope_validation_without_gpu():
    import torch
    from taomate_hd_amd import (HeadMajorRingKVCache, KVContract, StreamingAttentionHook,
                                fused_qkv_qk_norm_rope_stage_)
    from taomate_hd_amd.hook import HookMode

    qkv = torch.zeros((8, 3 * 2 * 64), dtype=torch.bfloat16)
    w = torch.ones(64, dtype=torch.bfloat16)
    table = torch.zeros((8, 32), dtype=torch.bfloat16)
    pos = torch.arange(8)
    with pytest.raises(ValueError, match="three complete projections"):
        fused_qkv_qk_norm_rope_stage_(qkv[:, :-64].contiguous(), w, w, table, pos, 1e-6, None)
    with pytest.raises(ValueError, match="must be on the GPU"):  # checked before the slot is touched
        fused_qkv_qk_norm_rope_stage_(qkv, w, w, table, pos, 1e-6, None)
    hook = StreamingAttentionHook(HeadMajorRingKVCache(KVContract(layer_names=("blocks.0.attn",), local_heads=2,
                                                                  head_dim=64)))
    hook.activate(mode=HookMode.NOISY, block_index=0)
    with pytest.raises(ValueError, match="non-main attention layer"):
        hook.preprocess_qkv_("blocks.9.attn", qkv, w, w, table, pos, 1e-6, row0=0, count=8)
    hook.deactivate()
    assert hook._prestaged == {}


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys

    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300, cwd=str(REPO))
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_condition_cache_queries_and_compact_writer_without_gpu():
    import torch

    from taomate_hd_amd import condition

    cached_fn, compact_fn = condition.resolve()
    assert cached_fn is condition.condition_attention_cached  # no reference runtime here
    assert compact_fn is condition.compact_condition_attention_output
    q = torch.zeros((10, 2, 4), dtype=torch.bfloat16)
    assert not cached_fn("blocks.0.attn", 0) and compact_fn("blocks.0.attn", q) is None
    state = condition.ConditionLayerState("blocks.0", cached_documents=(1,))
    with condition.condition_layer(state):
        assert cached_fn("blocks.0.attn", 1) and not cached_fn("blocks.0.attn", 0)
        assert not cached_fn("blocks.1.attn", 1)
        assert compact_fn("blocks.0.attn", q) is None  # no compact order
    assert not cached_fn("blocks.0.attn", 1)
    with pytest.raises(ValueError, match="sorted"):
        condition.ConditionLayerState("blocks.0", compact_rows=[3, 2])
    state = condition.ConditionLayerState("blocks.0.attn", cached_documents=(0,), compact_rows=[2, 3, 5, 7, 8, 9])
    with condition.condition_layer(state):
        assert compact_fn("blocks.1.attn", q) is None
        assert not state.attention_output_compact
        writer = compact_fn("blocks.0.attn", q)
        assert state.attention_output_compact  # the caller learns the output is compact
        assert tuple(writer.output.shape) == (6, 2, 4) and not bool(writer.output.any())
        value = torch.arange(1, 3, dtype=torch.bfloat16).view(2, 1, 1).expand(2, 2, 4)
        writer.write_rows(0, "media", 1, torch.tensor([2, 4]), value)  # global rows 3, 5
        doc = torch.arange(10, 13, dtype=torch.bfloat16).view(3, 1, 1).expand(3, 2, 4)
        writer.write_document(7, 10, doc)  # global rows 7..9, all kept
        assert writer.output[:, 0, 0].tolist() == [0, 1, 2, 10, 11, 12]
        with pytest.raises(ValueError, match="compact row set"):
            writer.write_rows(0, "condition", 0, torch.tensor([0, 1]), value)  # rows 0, 1 not kept


def test_session_forwards_condition_cache_queries_without_gpu():
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingSession, condition

    class Plan:
        phases = ("p0",)

    def cached(layer, doc):
        return False

    def compact(layer, query):
        return None

    cache = HeadMajorRingKVCache(KVContract(layer_names=("blocks.0.attn",), local_heads=2, head_dim=64))
    session = StreamingSession(Plan(), cache=cache, condition_attention_cached=cached,
                               compact_condition_attention_output=compact)
    assert session.hook._condition_attention_cached is cached and session.hook._compact_output is compact
    default = StreamingSession(Plan(), cache=cache)
    assert default.hook._condition_attention_cached is condition.condition_attention_cached


def test_w8a8_workspace_storage_without_gpu():
    import torch

    from taomate_hd_amd import W8A8Workspace

    ws = W8A8Workspace(torch, max_bytes=1 << 20)
    x = torch.zeros((100, 256))
    q, s = ws.activations(x)
    assert q.dtype == torch.int8 and tuple(q.shape) == (100, 256)
    assert s.dtype == torch.float32 and tuple(s.shape) == (100, 1)
    assert (s.data_ptr() - q.data_ptr()) % 256 == 0 and s.data_ptr() >= q.data_ptr() + q.numel()
    q2, _ = ws.activations(torch.zeros((10, 512)))  # smaller: same arena
    assert q2.data_ptr() == q.data_ptr()
    a = ws.output(x, 384)
    b = ws.output(x, 128)
    assert a.dtype == torch.bfloat16 and tuple(a.shape) == (100, 384) and a.data_ptr() != b.data_ptr()
    assert ws.output(x[:7], 384).data_ptr() == a.data_ptr()  # same width: reused
    assert ws.nbytes == (100 * 256 + 4 * 100) + 2 * 100 * (384 + 128)
    with pytest.raises(MemoryError, match="bound"):
        ws.output(torch.zeros((4096, 1)), 4096)
    ws.release()
    assert ws.nbytes == 0


def test_slot_pool_keeps_at_most_max_free_slots_without_gpu():
    import torch

    from taomate_hd_amd import SlotPool

    pool = SlotPool(torch, heads=1, head_dim=64, device="cpu", max_free=2)
    slots = [pool.acquire(n) for n in (64, 128, 192, 256)]
    for s in slots:
        pool.release(s)
    assert len(pool._free) == 2 and sorted(s.capacity for s in pool._free) == [192, 256]
    assert pool.free_bytes == sum(s.nbytes for s in pool._free)
    assert pool.acquire(100) is slots[2]  # smallest free slot that fits
    # a slot goes back out only on the stream it was released on
    pool.release(slots[2])
    slots[2].released_on = 12345  # as if released on another stream
    other = pool.acquire(100)
    assert other is not slots[2] and other.capacity == 256  # the other free slot, released here


def test_row_lists_are_range_checked_before_the_int32_cast_without_gpu():
    import torch

    from taomate_hd_amd.attention import _row_list

    with pytest.raises(ValueError, match=r"in \[0, 10\)"):
        _row_list(torch, torch.tensor([0, 2 ** 32 + 3], dtype=torch.int64), "cpu", 10, "rows", False)
    with pytest.raises(ValueError, match="int32 or int64"):
        _row_list(torch, torch.tensor([0.0, 1.0]), "cpu", 10, "rows", False)
    rows = _row_list(torch, torch.tensor([3, 9], dtype=torch.int64), "cpu", 10, "rows", False)
    assert rows.dtype == torch.int32 and rows.tolist() == [3, 9]


def test_vt_columns_match_vt_position():
    import torch

    from taomate_hd_amd.slots import vt_columns, vt_position

    for n in (0, 1, 15, 16, 17, 63, 64, 65, 1000):
        assert vt_columns(torch, n, "cpu").tolist() == [vt_position(t) for t in range(n)], n


def test_ulysses_receive_layouts_refuse_non_bf16_buffers_without_gpu():
    """The receive kernels address their buffers as bf16 elements: a 1-byte
    ``out`` would be written past its end, a 4-byte one scrambled, so every
    buffer's dtype is checked before the library is called."""
    import torch

    from taomate_hd_amd.ulysses import attention_receive_layout, qkv_receive_layout

    received = torch.zeros((2, 3, 4, 2, 8), dtype=torch.bfloat16)
    for dtype in (torch.int8, torch.uint8, torch.float32, torch.float16):
        with pytest.raises(ValueError, match="out must be a bf16"):
            qkv_receive_layout(received, out=torch.empty((8, 48), dtype=dtype))
        with pytest.raises(ValueError, match="received QKV must be a contiguous bf16"):
            qkv_receive_layout(received.to(dtype))
    value = torch.zeros((2, 4, 3, 8), dtype=torch.bfloat16)
    for dtype in (torch.int8, torch.float32):
        with pytest.raises(ValueError, match="out must be a bf16"):
            attention_receive_layout(value, num_heads=6, out=torch.empty((4, 6, 8), dtype=dtype))
        with pytest.raises(ValueError, match="received attention output must be a contiguous bf16"):
            attention_receive_layout(value.to(dtype), num_heads=6)
    # correct dtypes reach the device check (no CPU path)
    with pytest.raises(ValueError, match="GPU tensor"):
        qkv_receive_layout(received, out=torch.empty((8, 48), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="GPU tensor"):
        attention_receive_layout(value, num_heads=6)


def test_condition_resolve_binds_the_reference_runtime_module_when_importable(monkeypatch):
    """Inside the reference runtime ``taomate_hd.model.condition_cache`` is
    importable and the hook must consult it (the reference hook imports it,
    attention_hook.py:322-324, 445-465); a stub module of that name stands in
    for it here.  Injected queries still win over it, and without it the
    package's own scope is used."""
    import sys
    import types

    from taomate_hd_amd import condition

    asked = []

    def cached(layer_name, document_index):
        asked.append(("cached", layer_name, document_index))
        return document_index == 1

    def compact(layer_name, query):
        asked.append(("compact", layer_name))
        return None

    root, model, module = (types.ModuleType(n) for n in ("taomate_hd", "taomate_hd.model",
                                                          "taomate_hd.model.condition_cache"))
    root.model, model.condition_cache = model, module
    module.condition_attention_cached, module.compact_condition_attention_output = cached, compact
    for name, mod in (("taomate_hd", root), ("taomate_hd.model", model), ("taomate_hd.model.condition_cache", module)):
        monkeypatch.setitem(sys.modules, name, mod)
    assert condition.resolve() == (cached, compact)
    cache, hook, _ = _hook_and_inputs()
    assert hook._condition_attention_cached is cached and hook._compact_output is compact
    assert hook._condition_attention_cached("blocks.0.attn", 1) and asked == [("cached", "blocks.0.attn", 1)]

    def mine(layer_name, document_index):
        return False

    injected = type(hook)(cache, condition_attention_cached=mine)
    assert injected._condition_attention_cached is mine and injected._compact_output is compact

    monkeypatch.delitem(sys.modules, "taomate_hd.model.condition_cache")
    monkeypatch.setitem(sys.modules, "taomate_hd.model.condition_cache", None)  # not importable
    assert condition.resolve() == (condition.condition_attention_cached, condition.compact_condition_attention_output)
