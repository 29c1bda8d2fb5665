"""Row-wise RMSNorm / AdaLN-modulate / residual-gate / SwiGLU ops of the DiT block.

Drop-ins for the reference's SOL fused kernels around every attention call
(src/taomate_hd/inference/fused_kernels.py:643-671, 706-796): same signatures, checks
and error messages, bf16 in and out, run by the gfx950 row kernels behind
``tmhd_rms_norm`` / ``tmhd_rms_norm_modulate`` /
``tmhd_residual_gate_rms_norm_modulate`` / ``tmhd_modulate`` /
``tmhd_gate_add`` on the current stream.  The bf16 rounding chain is the
reference's; the order of the sum of squares and a correctly rounded inverse
square root are fixed where the reference leaves them to its compiler
(stated in include/tmhd.h).  Tables (scale / shift / gate) are read through
their row stride, without the reference's contiguous copies.
"""

from __future__ import annotations

from typing import Any

from . import _native


def _rows(torch: Any, value: Any, name: str) -> Any:
    """[rows, cols] view of ``value`` with unit column stride and aligned rows."""
    _native.require_device_tensor(torch, value, name)
    if value.dtype != torch.bfloat16:
        raise ValueError(f"SOL {name} must be bfloat16")
    flat = value.reshape(-1, value.shape[-1])
    if flat.stride(-1) != 1 or flat.stride(0) % 8 or flat.data_ptr() % 16:
        flat = flat.contiguous()
    return flat


def _table(torch: Any, table: Any, name: str, cols: int, device: Any) -> Any:
    _native.require_same_gpu(torch, device, **{name: table})
    if table.dtype != torch.bfloat16 or table.ndim != 2 or int(table.shape[-1]) != cols:
        raise ValueError(f"SOL {name} table must be bf16 [table_rows, {cols}]")
    if table.stride(-1) != 1 or table.stride(0) % 8 or table.data_ptr() % 16:
        table = table.contiguous()
    return table


def _weight(torch: Any, weight: Any, cols: int, device: Any) -> Any:
    _native.require_same_gpu(torch, device, weight=weight)
    if weight.dtype != torch.bfloat16 or int(weight.numel()) != cols:
        raise ValueError("SOL RMSNorm weight must be bf16 with one value per column")
    return weight.reshape(-1).contiguous()


def _index(torch: Any, indices: Any, rows: int, message: str | None, device: Any) -> Any:
    if not torch.is_tensor(indices) or indices.device != device:
        raise ValueError("SOL table indices must be a tensor on the GPU of the rows")
    index = indices.reshape(-1).to(dtype=torch.int64).contiguous()
    if message is not None and int(index.numel()) != rows:
        raise ValueError(message)
    if int(index.numel()) < rows:
        raise ValueError("SOL table indices do not cover every row")
    return index


def _run(status: int, what: str) -> None:
    _native.check(status, what)


def fused_rms_norm(value: Any, weight: Any, eps: float) -> Any:
    """``bf16(value * rsqrt(mean(value^2) + eps) * weight)`` per row (fused_kernels.py:312-321, 706-721)."""
    import torch

    shape = value.shape
    flat = _rows(torch, value, "value")
    rows, cols = int(flat.shape[0]), int(flat.shape[1])
    w = _weight(torch, weight, cols, flat.device)
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=flat.device)
    _run(_native.load().tmhd_rms_norm(_native.ptr(flat), flat.stride(0), _native.ptr(out), out.stride(0),
                                      _native.ptr(w), rows, cols, float(eps), _native.stream_ptr(torch, flat.device)),
         "tmhd_rms_norm")
    return out.reshape(shape)


def fused_rms_norm_modulate(value: Any, weight: Any, scale: Any, shift: Any, indices: Any, eps: float) -> Any:
    """RMSNorm then AdaLN modulation with table row ``indices[row]`` (fused_kernels.py:323-348, 723-755)."""
    import torch

    shape = value.shape
    flat = _rows(torch, value, "value")
    rows, cols = int(flat.shape[0]), int(flat.shape[1])
    index = _index(torch, indices, rows, "SOL RMSNorm/AdaLN indices do not cover every row", flat.device)
    w = _weight(torch, weight, cols, flat.device)
    scale, shift = _table(torch, scale, "scale", cols, flat.device), _table(torch, shift, "shift", cols, flat.device)
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=flat.device)
    _run(_native.load().tmhd_rms_norm_modulate(
        _native.ptr(flat), flat.stride(0), _native.ptr(out), out.stride(0), _native.ptr(w), _native.ptr(scale),
        scale.stride(0), _native.ptr(shift), shift.stride(0), _native.ptr(index), min(int(scale.shape[0]), int(shift.shape[0])),
        rows, cols, float(eps), _native.stream_ptr(torch, flat.device)), "tmhd_rms_norm_modulate")
    return out.reshape(shape)


def fused_residual_gate_rms_norm_modulate(residual: Any, branch: Any, gate: Any, weight: Any, scale: Any, shift: Any,
                                          indices: Any, eps: float) -> tuple[Any, Any]:
    """``hidden = residual + gate * branch`` (bf16 rounded), then RMSNorm + AdaLN
    modulation of ``hidden``; returns ``(hidden, output)`` (fused_kernels.py:350-383, 757-796)."""
    import torch

    shape = residual.shape
    res = _rows(torch, residual, "residual")
    rows, cols = int(res.shape[0]), int(res.shape[1])
    br = _rows(torch, branch.reshape(-1, cols), "branch")
    _native.require_same_gpu(torch, res.device, branch=br)
    if int(br.shape[0]) != rows:
        raise ValueError("SOL residual and branch rows differ")
    index = _index(torch, indices, rows, "SOL residual/AdaLN indices do not cover every row", res.device)
    w = _weight(torch, weight, cols, res.device)
    gate, scale, shift = (_table(torch, t, n, cols, res.device) for t, n in ((gate, "gate"), (scale, "scale"), (shift, "shift")))
    hidden = torch.empty((rows, cols), dtype=torch.bfloat16, device=res.device)
    out = torch.empty_like(hidden)
    _run(_native.load().tmhd_residual_gate_rms_norm_modulate(
        _native.ptr(res), res.stride(0), _native.ptr(br), br.stride(0), _native.ptr(gate), gate.stride(0),
        _native.ptr(w), _native.ptr(scale), scale.stride(0), _native.ptr(shift), shift.stride(0), _native.ptr(index),
        min(int(gate.shape[0]), int(scale.shape[0]), int(shift.shape[0])), _native.ptr(hidden), hidden.stride(0), _native.ptr(out), out.stride(0), rows, cols, float(eps),
        _native.stream_ptr(torch, res.device)), "tmhd_residual_gate_rms_norm_modulate")
    return hidden.reshape(shape), out.reshape(shape)


def fused_modulate(value: Any, shift: Any, scale: Any, indices: Any) -> Any:
    """AdaLN modulation ``bf16(bf16(value * bf16(1 + scale[t])) + shift[t])`` (fused_kernels.py:221-237, 643-656)."""
    import torch

    shape = value.shape
    flat = _rows(torch, value, "value")
    rows, cols = int(flat.shape[0]), int(flat.shape[1])
    index = _index(torch, indices, rows, None, flat.device)
    scale, shift = _table(torch, scale, "scale", cols, flat.device), _table(torch, shift, "shift", cols, flat.device)
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=flat.device)
    _run(_native.load().tmhd_modulate(
        _native.ptr(flat), flat.stride(0), _native.ptr(out), out.stride(0), _native.ptr(scale), scale.stride(0),
        _native.ptr(shift), shift.stride(0), _native.ptr(index), min(int(scale.shape[0]), int(shift.shape[0])), rows,
        cols, _native.stream_ptr(torch, flat.device)), "tmhd_modulate")
    return out.reshape(shape)


def fused_gate_add(residual: Any, gate: Any, branch: Any, indices: Any) -> Any:
    """``bf16(residual + bf16(gate[t] * branch))`` (fused_kernels.py:239-255, 658-671)."""
    import torch

    shape = residual.shape
    res = _rows(torch, residual, "residual")
    rows, cols = int(res.shape[0]), int(res.shape[1])
    br = _rows(torch, branch.reshape(-1, cols), "branch")
    _native.require_same_gpu(torch, res.device, branch=br)
    if int(br.shape[0]) != rows:
        raise ValueError("SOL residual and branch rows differ")
    index = _index(torch, indices, rows, None, res.device)
    gate = _table(torch, gate, "gate", cols, res.device)
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=res.device)
    _run(_native.load().tmhd_gate_add(
        _native.ptr(res), res.stride(0), _native.ptr(gate), gate.stride(0), _native.ptr(br), br.stride(0),
        _native.ptr(index), int(gate.shape[0]), _native.ptr(out), out.stride(0), rows, cols,
        _native.stream_ptr(torch, res.device)), "tmhd_gate_add")
    return out.reshape(shape)


def fused_swiglu(value: Any) -> Any:
    """``bf16(bf16(gate * sigmoid(gate)) * up)`` over the two halves of the last
    axis (fused_kernels.py:299-310, 694-704); within one bf16 ulp of the
    reference (its sigmoid is its compiler's)."""
    import torch

    shape = value.shape
    half = int(shape[-1]) // 2
    flat = _rows(torch, value, "value")
    rows = int(flat.shape[0])
    out = torch.empty((rows, half), dtype=torch.bfloat16, device=flat.device)
    _run(_native.load().tmhd_swiglu(_native.ptr(flat), flat.stride(0), _native.ptr(out), out.stride(0), rows, half,
                                    _native.stream_ptr(torch, flat.device)), "tmhd_swiglu")
    return out.reshape(*shape[:-1], half)
