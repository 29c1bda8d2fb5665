"""INT8 quant / scaled-mm operators with the signatures of the vLLM ops the
reference calls (src/taomate_hd/inference/w8a8.py:23-32, 71-72, 140-144).

* ``scaled_int8_quant(x)``                     -> (q int8 [M, K], scale fp32 [M, 1], None)
* ``dynamic_scaled_int8_quant(out, x, scale, azp=None)``  out-variant
* ``cutlass_scaled_mm(a, b, scale_a, scale_b, out_dtype=torch.bfloat16, bias=None)``
* ``cutlass_scaled_mm_out(out, a, b, scale_a, scale_b, bias=None)``  (the
  ``torch.ops._C.cutlass_scaled_mm`` argument order used at w8a8.py:72)

``b`` is the ``[K, N]`` transposed view of the row-major ``[N, K]`` INT8 weight
(``weight.t()``), ``scale_b`` the ``[1, N]`` view of the per-channel scale.
Every op runs a gfx950 HIP kernel from libtmhd.so.
"""

from __future__ import annotations

from typing import Any

from . import _native


def _torch():
    import torch

    return torch


def _check_rows(torch: Any, x: Any, name: str) -> None:
    _native.require_device_tensor(torch, x, name)
    if x.ndim != 2 or x.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D row-major GPU tensor")


def dynamic_scaled_int8_quant(out: Any, x: Any, scale: Any, azp: Any | None = None) -> None:
    """Per-token dynamic symmetric INT8 quantization into ``out`` / ``scale``.

    scale[m] = amax_m / 127, out[m, k] = sat_int8(rint(x[m, k] * (127 / amax_m)));
    a zero row gives scale 0 and zeros.  Only the symmetric form (azp None) is
    implemented, the form the reference uses (w8a8.py:71).
    """
    torch = _torch()
    if azp is not None:
        raise NotImplementedError("asymmetric (azp) INT8 quantization is not implemented")
    _check_rows(torch, x, "x")
    _native.require_same_gpu(torch, x.device, out=out, scale=scale)
    if x.dtype != torch.bfloat16:
        raise ValueError("x must be bf16")
    rows, cols = int(x.shape[0]), int(x.shape[1])
    if out.dtype != torch.int8 or tuple(out.shape) != (rows, cols) or not out.is_contiguous():
        raise ValueError("out must be a contiguous int8 tensor shaped like x")
    if scale.dtype != torch.float32 or scale.numel() != rows or not scale.is_contiguous():
        raise ValueError("scale must be a contiguous fp32 tensor with one entry per row")
    status = _native.load().tmhd_token_quant_i8(
        _native.ptr(out), _native.ptr(scale), _native.ptr(x), rows, cols, x.stride(0),
        _native.stream_ptr(torch, x.device),
    )
    _native.check(status, "tmhd_token_quant_i8")


def scaled_int8_quant(x: Any, scale: Any | None = None, azp: Any | None = None, symmetric: bool = True):
    """Allocating form: returns ``(q, scale [M, 1], None)`` (w8a8.py:141)."""
    torch = _torch()
    if scale is not None or azp is not None or not symmetric:
        raise NotImplementedError("only dynamic symmetric per-token quantization is implemented")
    x2 = x.reshape(-1, int(x.shape[-1]))
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    out = torch.empty(x2.shape, dtype=torch.int8, device=x.device)
    s = torch.empty((x2.shape[0], 1), dtype=torch.float32, device=x.device)
    dynamic_scaled_int8_quant(out, x2, s)
    return out.view(*x.shape), s, None


def quantize_weight(weight: Any) -> tuple[Any, Any]:
    """Static per-output-channel INT8 weight quantization (w8a8.py:175-179).

    scale = max(amax_row / 127, 1e-12), q = clamp(rint(w / scale), -127, 127);
    returns (q int8 [N, K] contiguous, scale fp32 [N, 1]).
    """
    torch = _torch()
    _check_rows(torch, weight, "weight")
    n, k = int(weight.shape[0]), int(weight.shape[1])
    q = torch.empty((n, k), dtype=torch.int8, device=weight.device)
    s = torch.empty((n, 1), dtype=torch.float32, device=weight.device)
    quantize_weight_into(q, s, weight)
    return q, s


def quantize_weight_into(q: Any, scale: Any, weight: Any) -> None:
    """``quantize_weight`` writing into caller storage: ``q`` a contiguous int8
    ``[N, K]`` tensor (for instance rows ``start:stop`` of a prepared weight),
    ``scale`` N contiguous fp32 values.  Rows are independent, so quantizing a
    matrix in row ranges gives the bits of quantizing it whole."""
    torch = _torch()
    _check_rows(torch, weight, "weight")
    _native.require_same_gpu(torch, weight.device, q=q, scale=scale)
    if weight.dtype != torch.bfloat16:
        raise ValueError("weight must be bf16")
    w = weight.contiguous()
    n, k = int(w.shape[0]), int(w.shape[1])
    if q.dtype != torch.int8 or tuple(q.shape) != (n, k) or not q.is_contiguous():
        raise ValueError("q must be a contiguous int8 tensor shaped like weight")
    if scale.dtype != torch.float32 or scale.numel() != n or not scale.is_contiguous():
        raise ValueError("scale must be a contiguous fp32 tensor with one entry per weight row")
    status = _native.load().tmhd_weight_quant_i8(
        _native.ptr(q), _native.ptr(scale), _native.ptr(w), n, k, _native.stream_ptr(torch, w.device)
    )
    _native.check(status, "tmhd_weight_quant_i8")


def _gemm_operands(torch: Any, a: Any, b: Any) -> tuple[int, int, int, int, int]:
    _native.require_device_tensor(torch, a, "a")
    _native.require_device_tensor(torch, b, "b")
    if a.dtype != torch.int8 or b.dtype != torch.int8:
        raise ValueError("a and b must be int8")
    if a.ndim != 2 or b.ndim != 2 or a.stride(1) != 1:
        raise ValueError("a must be a row-major [M, K] int8 matrix")
    if b.stride(0) != 1:
        raise ValueError("b must be the [K, N] column-major view (weight.t()) of a row-major [N, K] weight")
    m, k = int(a.shape[0]), int(a.shape[1])
    if int(b.shape[0]) != k:
        raise ValueError(f"inner dimensions differ: a {tuple(a.shape)}, b {tuple(b.shape)}")
    n = int(b.shape[1])
    return m, n, k, a.stride(0), b.stride(1)


_SPLIT_WS: dict[tuple[str, int], Any] = {}


def _split_workspace(torch: Any, device: Any, m: int, n: int, k: int) -> tuple[int | None, int]:
    """Grow-only scratch for the K split of the GEMM's last round (int32
    partial tiles), one per (device, stream): calls on one stream are
    ordered, so they share it."""
    need = int(_native.load().tmhd_gemm_split_workspace_bytes(m, n, k))
    if need <= 0:
        return None, 0
    key = (str(device), _native.stream_ptr(torch, device))
    ws = _SPLIT_WS.get(key)
    if ws is None or int(ws.numel()) < need:
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        _SPLIT_WS[key] = ws
    return _native.ptr(ws), int(ws.numel())


def cutlass_scaled_mm_out(out: Any, a: Any, b: Any, scale_a: Any, scale_b: Any, bias: Any | None = None) -> None:
    """out = bf16(float(a @ b) * scale_b[n] * scale_a[m] (+ bias[n])), int32 accumulate."""
    torch = _torch()
    m, n, k, lda, ldb = _gemm_operands(torch, a, b)
    _native.require_same_gpu(torch, a.device, b=b, out=out, scale_a=scale_a, scale_b=scale_b, bias=bias)
    if out.dtype != torch.bfloat16:
        raise NotImplementedError("only bf16 output is implemented")
    if tuple(out.shape) != (m, n) or out.stride(1) != 1:
        raise ValueError("out must be a row-major [M, N] bf16 tensor")
    sa = scale_a.reshape(-1)
    sb = scale_b.reshape(-1)
    if sa.dtype != torch.float32 or sb.dtype != torch.float32 or sa.numel() != m or sb.numel() != n:
        raise ValueError("scale_a must hold M and scale_b N fp32 values (per-token / per-channel)")
    sa = sa.contiguous()
    sb = sb.contiguous()
    bias_ptr = None
    if bias is not None:
        if bias.dtype != torch.bfloat16 or bias.numel() != n:
            raise ValueError("bias must be a bf16 vector of N values")
        bias = bias.contiguous()
        bias_ptr = _native.ptr(bias)
    ws, ws_bytes = _split_workspace(torch, a.device, m, n, k)
    status = _native.load().tmhd_gemm_w8a8_ws(
        _native.ptr(out), _native.ptr(a), _native.ptr(b), _native.ptr(sa), _native.ptr(sb), bias_ptr,
        m, n, k, lda, ldb, out.stride(0), ws, ws_bytes, _native.stream_ptr(torch, a.device),
    )
    _native.check(status, "tmhd_gemm_w8a8_ws")


def cutlass_scaled_mm(a: Any, b: Any, scale_a: Any, scale_b: Any, out_dtype: Any = None, bias: Any | None = None):
    """Allocating form used at w8a8.py:142-144."""
    torch = _torch()
    if out_dtype is not None and out_dtype != torch.bfloat16:
        raise NotImplementedError("only bf16 output is implemented")
    out = torch.empty((int(a.shape[0]), int(b.shape[1])), dtype=torch.bfloat16, device=a.device)
    cutlass_scaled_mm_out(out, a, b, scale_a, scale_b, bias)
    return out


def int8_mm_i32(a: Any, b: Any) -> Any:
    """Raw int32 accumulators of ``a @ b`` (same GEMM kernel, no epilogue)."""
    torch = _torch()
    m, n, k, lda, ldb = _gemm_operands(torch, a, b)
    _native.require_same_gpu(torch, a.device, b=b)
    out = torch.empty((m, n), dtype=torch.int32, device=a.device)
    ws, ws_bytes = _split_workspace(torch, a.device, m, n, k)
    status = _native.load().tmhd_gemm_i8_i32_ws(
        _native.ptr(out), _native.ptr(a), _native.ptr(b), m, n, k, lda, ldb, n, ws, ws_bytes,
        _native.stream_ptr(torch, a.device)
    )
    _native.check(status, "tmhd_gemm_i8_i32_ws")
    return out


def cutlass_scaled_mm_swiglu(a: Any, b: Any, scale_a: Any, scale_b: Any, bias: Any | None = None) -> Any:
    """SwiGLU of the scaled INT8 GEMM without materialising it: ``b`` is the
    [K, 2F] column-major view of gate / up weight rows interleaved in blocks
    of 128 (``interleave_swiglu_rows``), ``scale_b`` (and ``bias``) in the same
    order; returns ``[M, F]`` bf16 = fused_swiglu(cutlass_scaled_mm(...)) of
    the de-interleaved weight, bit for bit."""
    torch = _torch()
    m, n, k, lda, ldb = _gemm_operands(torch, a, b)
    _native.require_same_gpu(torch, a.device, b=b, scale_a=scale_a, scale_b=scale_b, bias=bias)
    sa = scale_a.reshape(-1)
    sb = scale_b.reshape(-1)
    if sa.dtype != torch.float32 or sb.dtype != torch.float32 or sa.numel() != m or sb.numel() != n:
        raise ValueError("scale_a must hold M and scale_b N fp32 values (per-token / per-channel)")
    sa, sb = sa.contiguous(), sb.contiguous()
    bias_ptr = None
    if bias is not None:
        if bias.dtype != torch.bfloat16 or bias.numel() != n:
            raise ValueError("bias must be a bf16 vector of N values")
        bias = bias.contiguous()
        bias_ptr = _native.ptr(bias)
    if k % 128 == 64 and n % 256 == 0:
        # the fused kernel takes k in 128-byte blocks; for an odd multiple of 64
        # the projection runs on the GEMM that takes it, then its interleaved
        # 128-column gate / up blocks are paired by fused_swiglu: the same
        # projection values and the same SwiGLU, so the same bits
        from .adaln import fused_swiglu

        proj = torch.empty((m, n), dtype=torch.bfloat16, device=a.device)
        cutlass_scaled_mm_out(proj, a, b, sa, sb, bias)
        return fused_swiglu(proj.view(m, n // 256, 2, 128).transpose(1, 2).reshape(m, n))
    out = torch.empty((m, n // 2), dtype=torch.bfloat16, device=a.device)
    ws, ws_bytes = _split_workspace(torch, a.device, m, n, k)
    status = _native.load().tmhd_gemm_w8a8_swiglu_ws(
        _native.ptr(out), _native.ptr(a), _native.ptr(b), _native.ptr(sa), _native.ptr(sb), bias_ptr,
        m, n, k, lda, ldb, out.stride(0), ws, ws_bytes, _native.stream_ptr(torch, a.device),
    )
    _native.check(status, "tmhd_gemm_w8a8_swiglu_ws")
    return out
