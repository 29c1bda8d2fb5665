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
"""

from __future__ import annotations

from typing import Any

from . import quant

INTERIOR_FC1_QKV_CUTLASS_W8A8_POLICY = "interior_fc1_qkv_v1"
H3_CUTLASS_W8A8_POLICIES = (INTERIOR_FC1_QKV_CUTLASS_W8A8_POLICY,)


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
