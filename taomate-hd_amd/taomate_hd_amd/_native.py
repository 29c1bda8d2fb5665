"""ctypes binding of libtmhd.so (the C ABI declared in include/tmhd.h).

The library is the only compute path of this package: every operator raises
if it is not built or no GPU is present.  There is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path
from typing import Any

LIB_PATH = Path(__file__).with_name("libtmhd.so")
MAX_SEGMENTS = 16
KV_TILE = 64
QUANT_BLOCK = 128
QUERY_TILE = 256

TMHD_OK = 0
TMHD_ERR_INVALID = 1
TMHD_ERR_UNSUPPORTED = 2
TMHD_ERR_HIP = 3


class KVSegment(ctypes.Structure):
    _fields_ = [
        ("k", c_void_p),
        ("vt", c_void_p),
        ("k_head_stride", c_int64),
        ("vt_head_stride", c_int64),
        ("vt_row_stride", c_int32),
        ("tokens", c_int32),
    ]


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_void_p),
        ("q_token_stride", c_int64),
        ("q_head_stride", c_int64),
        ("q_rows", c_void_p),
        ("q_row0", c_int32),
        ("lq", c_int32),
        ("o", c_void_p),
        ("o_token_stride", c_int64),
        ("o_head_stride", c_int64),
        ("o_rows", c_void_p),
        ("o_row0", c_int32),
        ("heads", c_int32),
        ("head_dim", c_int32),
        ("scale", c_float),
        ("n_segments", c_int32),
        ("seg", KVSegment * MAX_SEGMENTS),
        ("split_workspace", c_void_p),
        ("split_workspace_bytes", c_int64),
    ]


class QKQuant(ctypes.Structure):
    _fields_ = [
        ("q_i8", c_void_p),
        ("q_scale", c_void_p),
        ("q_head_stride", c_int64),
        ("q_scale_head_stride", c_int32),
        ("reserved0", c_int32),
        ("k_i8", c_void_p * MAX_SEGMENTS),
        ("k_scale", c_void_p * MAX_SEGMENTS),
        ("k_head_stride", c_int64 * MAX_SEGMENTS),
        ("k_scale_head_stride", c_int32 * MAX_SEGMENTS),
        ("k_mean", c_void_p),
        ("mean_workspace", c_void_p),
        ("k_sum", c_void_p * MAX_SEGMENTS),
    ]


_SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "tmhd_version": (c_char_p, []),
    "tmhd_last_error": (c_char_p, []),
    "tmhd_attn_split_workspace_bytes": (c_int64, [c_int32]),
    "tmhd_attn_fwd_bf16": (c_int, [POINTER(AttnArgs), c_void_p]),
    "tmhd_attn_fwd_bf16_noalloc": (c_int, [POINTER(AttnArgs), c_void_p]),
    "tmhd_attn_fwd_i8qk": (c_int, [POINTER(AttnArgs), POINTER(QKQuant), c_void_p]),
    "tmhd_qk_smooth_quant": (c_int, [POINTER(AttnArgs), POINTER(QKQuant), c_void_p]),
    "tmhd_kv_pack": (
        c_int,
        [
            c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_int32,
            c_void_p, c_void_p, c_int64, c_int64, c_int32, c_int32, c_int32,
            c_int32, c_int32, c_void_p,
        ],
    ),
    "tmhd_rms_norm": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int32, c_float, c_void_p]),
    "tmhd_rms_norm_modulate": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
         c_int64, c_int32, c_float, c_void_p],
    ),
    "tmhd_residual_gate_rms_norm_modulate": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
         c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int32, c_float, c_void_p],
    ),
    "tmhd_modulate": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64,
         c_int32, c_void_p],
    ),
    "tmhd_gate_add": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64,
         c_int32, c_void_p],
    ),
    "tmhd_swiglu": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int32, c_void_p]),
    "tmhd_selfcheck_rounding": (c_int, [c_void_p, c_void_p]),
    "tmhd_apply_rope": (
        c_int,
        [c_void_p, c_int32, c_int32, c_int32, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
         c_int32, c_void_p],
    ),
    "tmhd_qk_norm_rope": (
        c_int,
        [
            c_void_p, c_int32, c_int32, c_int32, c_int64, c_void_p, c_int64, c_void_p,
            c_void_p, c_int64, c_void_p, c_int64, c_int32, c_float, c_void_p,
        ],
    ),
    "tmhd_qkv_norm_rope": (
        c_int,
        [
            c_void_p, c_int32, c_int32, c_int32, c_int64, c_void_p, c_void_p,
            c_void_p, c_int64, c_int64, c_int32, c_void_p, c_float, c_void_p,
        ],
    ),
    "tmhd_qkv_norm_rope_stage": (
        c_int,
        [
            c_void_p, c_int32, c_int32, c_int32, c_int64, c_void_p, c_void_p,
            c_void_p, c_int64, c_int64, c_int32, c_void_p, c_float,
            c_int32, c_int32, c_void_p, c_void_p, c_int64, c_int64, c_int32, c_int32, c_int32, c_void_p,
        ],
    ),
    "tmhd_ulysses_qkv_send": (
        c_int, [c_void_p, c_int64, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p],
    ),
    "tmhd_ulysses_qkv_norm_rope_send": (
        c_int,
        [
            c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
            c_int32, c_void_p, c_float, c_int32, c_int32, c_void_p, c_void_p,
        ],
    ),
    "tmhd_ulysses_qkv_receive": (
        c_int, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_int64, c_void_p],
    ),
    "tmhd_ulysses_attention_receive": (
        c_int, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_int64, c_int64, c_void_p],
    ),
    "tmhd_k_fixed_sum": (c_int, [c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "tmhd_token_quant_i8": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int64, c_void_p]),
    "tmhd_weight_quant_i8": (c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "tmhd_gemm_w8a8": (
        c_int,
        [
            c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
            c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_void_p,
        ],
    ),
    "tmhd_gemm_i8_i32": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_void_p],
    ),
    "tmhd_gemm_split_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32]),
    "tmhd_gemm_w8a8_ws": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int64,
         c_int64, c_void_p, c_int64, c_void_p],
    ),
    "tmhd_gemm_w8a8_swiglu_ws": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int64,
         c_int64, c_void_p, c_int64, c_void_p],
    ),
    "tmhd_gemm_i8_i32_ws": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int64, c_int64, c_void_p, c_int64,
         c_void_p],
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load libtmhd.so (once) and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"libtmhd.so is not built ({LIB_PATH}); run taomate-hd_amd/build.py "
                    "(hipcc --offload-arch=gfx950) before using the HIP operators"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def version() -> str:
    return load().tmhd_version().decode()


def check(status: int, what: str) -> None:
    """Turn a tmhd_status into the exception type the reference raises."""
    if status == TMHD_OK:
        return
    message = load().tmhd_last_error().decode() or what
    if status in (TMHD_ERR_INVALID, TMHD_ERR_UNSUPPORTED):
        raise ValueError(message)
    raise RuntimeError(message)


def require_device_tensor(torch: Any, tensor: Any, name: str) -> None:
    if not torch.is_tensor(tensor) or not tensor.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the HIP kernels have no CPU path)")


def require_same_gpu(torch: Any, device: Any, **tensors: Any) -> None:
    """Every given tensor (None skipped) lives on ``device``, a GPU."""
    for name, tensor in tensors.items():
        if tensor is None:
            continue
        require_device_tensor(torch, tensor, name)
        if tensor.device != device:
            raise ValueError(f"{name} must be on {device} (found {tensor.device})")


def stream_ptr(torch: Any, device: Any) -> int:
    return int(torch.cuda.current_stream(device=device).cuda_stream)


def ptr(tensor: Any) -> int:
    return int(tensor.data_ptr())
