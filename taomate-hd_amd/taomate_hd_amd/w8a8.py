"""Selective W8A8 projection: drop-in for src/taomate_hd/inference/w8a8.py and
the ``_linear`` dispatch of src/taomate_hd/distributed/linear.py:43-68.

* ``W8A8Workspace`` plays the role of ``CutlassW8A8Workspace`` (w8a8.py:12-73):
  per-stream storage for the quantized activations (one arena) and the bf16
  outputs (one buffer per output width), then ``dynamic_scaled_int8_quant`` +
  ``cutlass_scaled_mm`` into them.
* ``cutlass_w8a8_linear`` (w8a8.py:117-145) also accepts a bf16 bias, applied
  in the GEMM epilogue (the reference raises for a bias).
* ``resolve_h3_cutlass_w8a8_policy`` restates the interior QKV/FC1 selection
  (w8a8.py:89-114); ``quantize_cutlass_w8a8_weight`` the weight quantizer
  (w8a8.py:175-179, run as a HIP kernel).
* ``linear`` is the ``_linear`` dispatch rule: a module that carries a W8A8
  weight scale takes the INT8 path, otherwise ``F.linear``.
* ``register_torch_ops`` exposes the two ops as ``torch.ops.tmhd.*`` with the
  ``torch.ops._C`` signatures the reference's workspace resolves by name.
* The load-time chain the reference runtime calls to switch W8A8 on
  (w8a8.py:76-86, 148-336): ``require_vllm_cutlass_w8a8`` (here: the HIP
  library loads and exports the INT8 entry points),
  ``prepare_cutlass_w8a8_stream_load_slot_`` /
  ``load_cutlass_w8a8_stream_weight_`` (row-chunked quantization of a
  streamed bf16 weight straight into its int8 storage),
  ``quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_`` (post-load
  conversion of the selected projections, with the reference's receipt keys)
  and ``enable_h3_cutlass_w8a8_workspace_``.  Names, keywords, module
  attributes, errors and receipt keys are the reference's, so this module can
  stand in for ``taomate_hd.inference.w8a8`` at every call site.
"""

from __future__ import annotations

from functools import lru_cache
from typing import Any

from . import _native, quant

INTERIOR_FC1_QKV_CUTLASS_W8A8_POLICY = "interior_fc1_qkv_v1"
H3_CUTLASS_W8A8_POLICIES = (INTERIOR_FC1_QKV_CUTLASS_W8A8_POLICY,)
_STREAM_LOAD_TEMPORARY_BYTES = 8 * 1024 * 1024
_PROJECTION_SUFFIXES = (".attn.qkv_proj", ".mlp.fc1", ".mlp.fc2")
# the entry points the W8A8 path calls: token quant, weight quant, GEMM
_W8A8_ENTRY_POINTS = ("tmhd_token_quant_i8", "tmhd_weight_quant_i8", "tmhd_gemm_w8a8_ws")


def _stream_of(torch: Any, tensor: Any) -> tuple[str, int | None, int]:
    """(device type, index, stream handle) of the stream work on ``tensor`` is queued on."""
    device = tensor.device
    handle = int(torch.cuda.current_stream(device=device).cuda_stream) if device.type == "cuda" else 0
    return (device.type, device.index, handle)


class _StreamStorage:
    """Device memory of one stream: a byte arena holding the quantized
    activations (int8 rows, then their fp32 scales at a 256-byte aligned
    offset), and one bf16 output buffer per output width."""

    def __init__(self) -> None:
        self.arena: Any | None = None
        self.outputs: dict[int, Any] = {}

    def nbytes(self) -> int:
        total = 0 if self.arena is None else int(self.arena.numel())
        return total + sum(int(t.numel()) * 2 for t in self.outputs.values())


class W8A8Workspace:
    """Projection storage reused per stream (the role of the reference's
    ``CutlassW8A8Workspace``, w8a8.py:12-73).

    Work on one stream is ordered, so every call on a stream shares one
    arena for its quantized activations: the next call's quantization is
    queued behind the previous call's GEMM.  A call's bf16 output lives in a
    buffer kept per output width and stays valid until the next call on the
    same stream with the same output width.  Storage grows to the largest
    call seen; ``max_bytes`` (optional) bounds the total per workspace,
    ``nbytes`` reports it and ``release`` returns it to the allocator.
    """

    def __init__(self, torch: Any, *, max_bytes: int | None = None) -> None:
        self._torch = torch
        self._max_bytes = None if max_bytes is None else int(max_bytes)
        self._streams: dict[tuple[Any, ...], _StreamStorage] = {}

    @property
    def nbytes(self) -> int:
        return sum(s.nbytes() for s in self._streams.values())

    def release(self) -> None:
        self._streams.clear()

    def _storage(self, inputs: Any) -> _StreamStorage:
        return self._streams.setdefault(_stream_of(self._torch, inputs), _StreamStorage())

    def _reserve(self, grow_by: int) -> None:
        if self._max_bytes is not None and self.nbytes + grow_by > self._max_bytes:
            raise MemoryError(f"W8A8 workspace would exceed its {self._max_bytes}-byte bound")

    def activations(self, inputs: Any) -> tuple[Any, Any]:
        """int8 ``[rows, width]`` and fp32 ``[rows, 1]`` views for the quantized ``inputs``."""
        torch = self._torch
        rows, width = int(inputs.shape[0]), int(inputs.shape[1])
        scale_at = (rows * width + 255) // 256 * 256
        need = scale_at + 4 * rows
        store = self._storage(inputs)
        if store.arena is None or int(store.arena.numel()) < need:
            self._reserve(need - (0 if store.arena is None else int(store.arena.numel())))
            store.arena = None  # let the allocator reuse the old block
            store.arena = torch.empty(need, dtype=torch.uint8, device=inputs.device)
        quantized = store.arena[: rows * width].view(torch.int8).view(rows, width)
        scales = store.arena[scale_at:need].view(torch.float32).view(rows, 1)
        return quantized, scales

    def output(self, inputs: Any, width: int) -> Any:
        """The bf16 ``[rows, width]`` output buffer of a call."""
        torch = self._torch
        rows, width = int(inputs.shape[0]), int(width)
        store = self._storage(inputs)
        buf = store.outputs.get(width)
        if buf is None or int(buf.shape[0]) < rows:
            self._reserve(2 * width * (rows - (0 if buf is None else int(buf.shape[0]))))
            store.outputs.pop(width, None)
            buf = torch.empty((rows, width), dtype=torch.bfloat16, device=inputs.device)
            store.outputs[width] = buf
        return buf[:rows]

    def linear(self, inputs: Any, weight_t: Any, weight_scale: Any, bias: Any | None = None) -> Any:
        quantized, activation_scale = self.activations(inputs)
        output = self.output(inputs, int(weight_t.shape[1]))
        quant.dynamic_scaled_int8_quant(quantized, inputs, activation_scale, None)
        quant.cutlass_scaled_mm_out(output, quantized, weight_t, activation_scale, weight_scale, bias)
        return output


# the reference's class name
CutlassW8A8Workspace = W8A8Workspace


def resolve_h3_cutlass_w8a8_policy(linear_names: list[str], *, policy: str) -> dict[str, Any]:
    """Select the interior QKV/FC1 projections for W8A8 (w8a8.py:89-114)."""
    if policy not in H3_CUTLASS_W8A8_POLICIES:
        raise ValueError("unsupported H3 CUTLASS W8A8 policy")
    projection_names = [name for name in linear_names if name.endswith((".attn.qkv_proj", ".mlp.fc1", ".mlp.fc2"))]
    if not projection_names:
        raise ValueError("H3 CUTLASS W8A8 policy requires projection candidates")
    block_indices = sorted({int(name.split(".", 2)[1]) for name in projection_names})
    boundary_blocks = (*block_indices[:2], *block_indices[-3:])
    eligible_suffixes = (".attn.qkv_proj", ".mlp.fc1")
    quantized_names = [
        name
        for name in projection_names
        if name.endswith(eligible_suffixes) and int(name.split(".", 2)[1]) not in boundary_blocks
    ]
    quantized_set = set(quantized_names)
    return {
        "policy": policy,
        "quantized_linear_names": quantized_names,
        "bf16_protected_linear_names": [name for name in projection_names if name not in quantized_set],
        "bf16_boundary_block_indices": list(boundary_blocks),
    }


def quantize_cutlass_w8a8_weight(torch: Any, weight: Any) -> tuple[Any, Any]:
    """Exact W8 conversion (w8a8.py:175-179): returns (q [N, K] int8, scale [N, 1] fp32)."""
    del torch
    return quant.quantize_weight(weight)


# the reference's private name for the same conversion (w8a8.py:175)
_quantize_cutlass_w8a8_weight = quantize_cutlass_w8a8_weight


@lru_cache(maxsize=1)
def require_vllm_cutlass_w8a8() -> Any:
    """The INT8 backend of an enabled W8A8 run (w8a8.py:76-86).

    The reference imports vLLM's CUDA custom ops here; on MI355X the ops are
    this package's HIP kernels, so the check is that libtmhd.so loads and
    exports the quant and GEMM entry points.  Returns the op namespace
    (``scaled_int8_quant``, ``cutlass_scaled_mm``, with vLLM's signatures);
    raises RuntimeError otherwise, as the reference does.  A failure is not
    cached, so a later call after building the library succeeds."""
    try:
        lib = _native.load()
    except (OSError, RuntimeError) as exc:
        raise RuntimeError("CUTLASS W8A8 requires libtmhd.so with its HIP INT8 operations") from exc
    for name in _W8A8_ENTRY_POINTS:
        if not hasattr(lib, name):
            raise RuntimeError(f"libtmhd.so is missing {name}")
    for name in ("scaled_int8_quant", "cutlass_scaled_mm"):
        if not callable(getattr(quant, name, None)):
            raise RuntimeError(f"HIP INT8 operations are missing {name}")
    return quant


def _is_projection(module: Any, linear_types: tuple[type, ...] | None) -> bool:
    """A candidate projection: an instance of ``linear_types`` when given (the
    reference passes its Column/RowParallelLinear, w8a8.py:250-260), else any
    module holding a 2-D ``weight`` tensor, which selects the same modules of
    the DiT (its qkv_proj / fc1 / fc2 are those linears or LoRA wrappers whose
    ``base`` is one)."""
    if linear_types is not None:
        return isinstance(module, linear_types)
    weight = getattr(module, "weight", None)
    return weight is not None and getattr(weight, "ndim", 0) == 2


def enable_h3_cutlass_w8a8_workspace_(torch: Any, transformer: Any) -> dict[str, Any]:
    """Attach one stream-keyed workspace to every W8A8 linear of the blocks
    (w8a8.py:148-172); the dispatch then quantizes into and writes through it."""
    require_vllm_cutlass_w8a8()
    selected = [
        (name, module)
        for name, module in transformer.named_modules()
        if name.startswith("blocks.") and getattr(module, "_cutlass_w8a8_weight_scale", None) is not None
    ]
    if not selected:
        raise RuntimeError("CUTLASS W8A8 workspace requires quantized H3 linears")
    workspace = W8A8Workspace(torch)
    for _, module in selected:
        module._cutlass_w8a8_workspace = workspace
        module._cutlass_w8a8_weight_t = module.weight.t()
        module._cutlass_w8a8_weight_scale_t = module._cutlass_w8a8_weight_scale.t()
    return {
        "schema": "taomate_hd.inference.cutlass_w8a8_workspace.v1",
        "linear_count": len(selected),
        "workspace_count_per_rank": 1,
        "allocation_policy": "grow_only_per_stream_activation_arena_and_output_width",
        "activation_quantization": "unchanged_dynamic_per_token_symmetric",
        "weight_quantization": "unchanged_static_per_output_channel_symmetric",
        "arithmetic_order_changed": False,
    }


def prepare_cutlass_w8a8_stream_load_slot_(torch: Any, module: Any, *, name: str) -> None:
    """Give a not yet loaded bf16 projection its final int8 weight and fp32
    scale storage, so that loading writes int8 rows and never holds the whole
    bf16 matrix on the device (w8a8.py:182-204)."""
    weight = module.weight
    if weight.dtype not in {torch.bfloat16, torch.int8}:
        raise TypeError(f"{name} expected an uninitialized BF16 or INT8 weight")
    if getattr(module, "bias", None) is not None:
        raise RuntimeError(f"{name} expected a bias-free H3 projection")
    if getattr(module, "_cutlass_w8a8_weight_scale", None) is not None:
        raise RuntimeError(f"{name} already owns CUTLASS W8A8 storage")
    if weight.dtype == torch.int8:
        if weight.requires_grad:
            raise RuntimeError(f"{name} preallocated INT8 weight requires gradients")
    else:
        storage = torch.empty(tuple(weight.shape), dtype=torch.int8, device=weight.device)
        module.weight = torch.nn.Parameter(storage, requires_grad=False)
    rows = int(weight.shape[0])
    module.register_buffer(
        "_cutlass_w8a8_weight_scale",
        torch.empty((rows, 1), dtype=torch.float32, device=weight.device),
        persistent=False,
    )
    module._cutlass_w8a8_stream_load_pending = True
    module._cutlass_w8a8_stream_loaded = False
    module._cutlass_w8a8_source_weight_bytes = int(weight.numel()) * 2


def load_cutlass_w8a8_stream_weight_(
    torch: Any,
    module: Any,
    source_weight: Any,
    *,
    name: str,
    maximum_temporary_bytes: int = _STREAM_LOAD_TEMPORARY_BYTES,
) -> None:
    """Quantize a bf16 source weight into a prepared projection, a range of
    output rows at a time (w8a8.py:207-242).

    Each output row has its own scale, so row ranges quantize to exactly the
    bits of the whole matrix.  A range is at most ``maximum_temporary_bytes``
    of bf16 (at least one row); it is moved to the device and quantized by the
    HIP weight kernel straight into the rows and scales of the prepared
    storage, with no int8 temporary in between."""
    if getattr(module, "_cutlass_w8a8_stream_load_pending", None) is not True:
        raise RuntimeError(f"{name} has no pending CUTLASS W8A8 stream load")
    if module.weight.dtype != torch.int8 or source_weight.dtype != torch.bfloat16:
        raise TypeError(f"{name} streamed CUTLASS W8A8 dtype differs")
    if tuple(module.weight.shape) != tuple(source_weight.shape):
        raise ValueError(f"{name} streamed CUTLASS W8A8 shape differs")
    if source_weight.ndim != 2:
        raise ValueError(f"{name} streamed CUTLASS W8A8 weight must be 2D")
    if maximum_temporary_bytes <= 0:
        raise ValueError("maximum_temporary_bytes must be positive")
    device = module.weight.device
    _native.require_device_tensor(torch, module.weight, f"{name} weight")
    rows, row_bytes = int(source_weight.shape[0]), int(source_weight.shape[1]) * 2
    chunk = max(1, int(maximum_temporary_bytes) // max(1, row_bytes))
    scales = module._cutlass_w8a8_weight_scale
    for start in range(0, rows, chunk):
        stop = min(rows, start + chunk)
        piece = source_weight[start:stop].to(device=device, dtype=torch.bfloat16)
        quant.quantize_weight_into(module.weight.data[start:stop], scales[start:stop], piece)
    module._cutlass_w8a8_stream_load_pending = False
    module._cutlass_w8a8_stream_loaded = True


def quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(
    torch: Any, transformer: Any, *, policy: str, linear_types: tuple[type, ...] | None = None
) -> dict[str, Any]:
    """Switch the policy's interior QKV / FC1 projections to W8A8 after loading
    (w8a8.py:245-336): streamed projections are checked complete, the others
    are quantized from their bf16 weight on the GPU.  Returns the reference's
    receipt.  ``linear_types`` restricts the candidates to those classes (the
    reference's Column/RowParallelLinear); by default any block projection
    holding a 2-D weight is a candidate."""
    require_vllm_cutlass_w8a8()
    candidates: list[tuple[str, Any]] = []
    for name, module in transformer.named_modules():
        if not name.startswith("blocks.") or not name.endswith(_PROJECTION_SUFFIXES):
            continue
        base = getattr(module, "base", module)
        if _is_projection(base, linear_types):
            candidates.append((name, base))
    selection = resolve_h3_cutlass_w8a8_policy([name for name, _ in candidates], policy=policy)
    chosen = set(selection["quantized_linear_names"])
    selected = [(name, module) for name, module in candidates if name in chosen]
    if not selected:
        raise RuntimeError("H3 CUTLASS W8A8 policy selected no linears")
    # every selected projection is checked before any is converted
    streamed: set[str] = set()
    for name, module in selected:
        if getattr(module, "_cutlass_w8a8_weight_scale", None) is not None:
            complete = (
                module.weight.dtype == torch.int8
                and getattr(module, "_cutlass_w8a8_stream_load_pending", None) is False
                and getattr(module, "_cutlass_w8a8_stream_loaded", None) is True
            )
            if not complete:
                raise RuntimeError(f"{name} has incomplete CUTLASS W8A8 storage")
            streamed.add(name)
        elif module.weight.dtype != torch.bfloat16:
            raise TypeError(f"{name} expected BF16 weight before W8A8 conversion")
        if getattr(module, "bias", None) is not None:
            raise RuntimeError(f"{name} expected a bias-free H3 projection")

    def source_bytes_of(module: Any) -> int:
        default = int(module.weight.numel()) * int(module.weight.element_size())
        return int(getattr(module, "_cutlass_w8a8_source_weight_bytes", default))

    eligible_bytes = sum(source_bytes_of(module) for _, module in candidates)
    source_bytes = quantized_bytes = 0
    converted: list[str] = []
    for name, module in selected:
        if name in streamed:
            source_bytes += source_bytes_of(module)
        else:
            weight = module.weight.detach()
            source_bytes += int(weight.numel()) * int(weight.element_size())
            q, scale = quantize_cutlass_w8a8_weight(torch, weight)
            module.weight = torch.nn.Parameter(q, requires_grad=False)
            module.register_buffer("_cutlass_w8a8_weight_scale", scale, persistent=False)
        quantized_bytes += int(module.weight.numel()) * int(module.weight.element_size())
        converted.append(name)
    return {
        "schema": "taomate_hd.inference.cutlass_w8a8.v1",
        "format": "int8_w8a8",
        "scope": "frozen_main_dit_base_weights_only",
        "policy": policy,
        "projection_set": "interior_qkv_and_fc1",
        "quantized_projection_suffixes": ["attn.qkv_proj", "mlp.fc1"],
        "activation_scale": "dynamic_per_token_symmetric",
        "weight_scale": "static_per_output_channel_symmetric",
        "kernel": "tmhd_gemm_w8a8_gfx950",
        "eligible_linear_count": len(candidates),
        "linear_count": len(converted),
        "stream_load_linear_count": len(streamed),
        "bf16_protected_linear_count": len(selection["bf16_protected_linear_names"]),
        "quantized_linear_names": converted,
        "bf16_protected_linear_names": selection["bf16_protected_linear_names"],
        "bf16_boundary_block_indices": selection["bf16_boundary_block_indices"],
        "source_weight_bytes": source_bytes,
        "quantized_weight_bytes": quantized_bytes,
        "eligible_source_weight_bytes": eligible_bytes,
        "eligible_weight_fraction": source_bytes / eligible_bytes,
        "bf16_projection_suffixes": ["attn.out_proj", "mlp.fc2"],
        "lora_branch": {"storage": "fp32_online_unmodified", "compute": "bf16"},
        "base_teacher_adapter_bypass": "lora_only",
        "base_teacher_base_precision": "int8_w8a8",
        "runtime_state": "transient_not_checkpoint_reconstructible",
    }


def cutlass_w8a8_linear(
    torch: Any,
    inputs: Any,
    weight: Any,
    weight_scale: Any,
    *,
    bias: Any | None,
    workspace: W8A8Workspace | None = None,
    weight_t: Any | None = None,
    weight_scale_t: Any | None = None,
) -> Any:
    """Dynamic per-token A8 x per-channel W8 GEMM (w8a8.py:117-145), bf16 out."""
    shape = (*inputs.shape[:-1], int(weight.shape[0]))
    flattened = inputs.reshape(-1, int(inputs.shape[-1])).contiguous()
    w_t = weight.t() if weight_t is None else weight_t
    s_t = weight_scale.t() if weight_scale_t is None else weight_scale_t
    if workspace is not None:
        return workspace.linear(flattened, w_t, s_t, bias).reshape(shape)
    quantized, activation_scale, _ = quant.scaled_int8_quant(flattened)
    output = quant.cutlass_scaled_mm(quantized, w_t, activation_scale, s_t, torch.bfloat16, bias)
    return output.reshape(shape)


def interleave_swiglu_rows(t: Any) -> Any:
    """Rows of a fused gate / up tensor ``[2F, ...]`` (gate rows first, as the
    MLP's merged FC1 stores them, model/layers.py:497-511) reordered in blocks
    of 128: gate rows 128t.. then up rows 128t.., so that one 256-row GEMM tile
    holds both halves of 128 output columns.  F must be a multiple of 128."""
    n = int(t.shape[0])
    if n % 256:
        raise ValueError("gate / up rows must be a multiple of 256 (F a multiple of 128)")
    return t.reshape(2, n // 256, 128, *t.shape[1:]).transpose(0, 1).reshape(t.shape).contiguous()


def quantize_cutlass_w8a8_swiglu_weight(torch: Any, weight: Any) -> tuple[Any, Any]:
    """Per-channel INT8 FC1 weight (gate rows, then up rows) for
    ``cutlass_w8a8_linear_swiglu``: quantized as ``quantize_cutlass_w8a8_weight``
    (per row, so the row order does not change the values), then interleaved."""
    qw, sw = quantize_cutlass_w8a8_weight(torch, weight)
    return interleave_swiglu_rows(qw), interleave_swiglu_rows(sw)


def cutlass_w8a8_linear_swiglu(torch: Any, inputs: Any, weight: Any, weight_scale: Any, *,
                               bias: Any | None = None, workspace: W8A8Workspace | None = None) -> Any:
    """``fused_swiglu(cutlass_w8a8_linear(inputs, W1))`` of the MLP
    (model/layers.py:525-534) in one GEMM whose epilogue applies SwiGLU, so
    the [M, 2F] projection is never written.  ``weight`` / ``weight_scale``
    come from ``quantize_cutlass_w8a8_swiglu_weight``; returns ``[..., F]``,
    bit-identical to the two-step form."""
    shape = (*inputs.shape[:-1], int(weight.shape[0]) // 2)
    flattened = inputs.reshape(-1, int(inputs.shape[-1])).contiguous()
    if workspace is not None:
        quantized, activation_scale = workspace.activations(flattened)
        quant.dynamic_scaled_int8_quant(quantized, flattened, activation_scale, None)
    else:
        quantized, activation_scale, _ = quant.scaled_int8_quant(flattened)
    out = quant.cutlass_scaled_mm_swiglu(quantized, weight.t(), activation_scale, weight_scale.t(), bias)
    return out.reshape(shape)


def linear(
    torch: Any,
    inputs: Any,
    weight: Any,
    bias: Any | None,
    *,
    cutlass_w8a8_weight_scale: Any | None = None,
    cutlass_w8a8_workspace: W8A8Workspace | None = None,
    cutlass_w8a8_weight_t: Any | None = None,
    cutlass_w8a8_weight_scale_t: Any | None = None,
) -> Any:
    """The ``_linear`` dispatch (distributed/linear.py:43-68) without its dead FP8 branch."""
    if cutlass_w8a8_weight_scale is not None:
        return cutlass_w8a8_linear(
            torch,
            inputs,
            weight,
            cutlass_w8a8_weight_scale,
            bias=bias,
            workspace=cutlass_w8a8_workspace,
            weight_t=cutlass_w8a8_weight_t,
            weight_scale_t=cutlass_w8a8_weight_scale_t,
        )
    return torch.nn.functional.linear(inputs, weight, bias)


_REGISTERED = False


def register_torch_ops() -> Any:
    """Register ``torch.ops.tmhd.dynamic_scaled_int8_quant`` and
    ``torch.ops.tmhd.cutlass_scaled_mm`` (out-variants with the argument order
    of ``torch.ops._C`` used at w8a8.py:71-72); returns ``torch.ops.tmhd``."""
    global _REGISTERED
    import torch

    if not _REGISTERED:
        lib = torch.library.Library("tmhd", "DEF")
        lib.define("dynamic_scaled_int8_quant(Tensor(a!) out, Tensor x, Tensor(b!) scale, Tensor? azp) -> ()")
        lib.define(
            "cutlass_scaled_mm(Tensor(a!) out, Tensor a, Tensor b, Tensor a_scales, Tensor b_scales, Tensor? bias) -> ()"
        )
        lib.impl("dynamic_scaled_int8_quant", quant.dynamic_scaled_int8_quant, "CUDA")
        lib.impl("cutlass_scaled_mm", quant.cutlass_scaled_mm_out, "CUDA")
        register_torch_ops._lib = lib  # keep the registration alive
        _REGISTERED = True
    return torch.ops.tmhd
