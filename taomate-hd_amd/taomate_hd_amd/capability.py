"""Hook installation ABI (src/taomate_hd/streaming/capability.py:1-51 and the
hook registry / metadata context of src/taomate_hd/model/layers.py:53-82).

A model integration reads ``native_stream_attention_hook()`` and
``native_stream_attention_metadata_value()`` at its attention call site, as
``MiniMaxH3Attention.forward`` does (layers.py:446-466).
"""

from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import asdict, dataclass
from typing import Any, Iterator

STREAM_HOOK_ABI = 3

_NATIVE_STREAM_HOOK: Any | None = None
_OFFICIAL_ATTENTION_HOOK: Any | None = None
_NATIVE_STREAM_METADATA: ContextVar[tuple[Any, Any] | None] = ContextVar("tmhd_stream_metadata", default=None)
_NATIVE_STREAM_LIVE_DOCUMENTS_HINT: ContextVar[tuple[int, ...] | None] = ContextVar(
    "tmhd_stream_live_documents_hint", default=None
)
_NATIVE_STREAM_MLP_VIDEO_STRIDE: ContextVar[int] = ContextVar("tmhd_stream_mlp_video_stride", default=1)


@dataclass(frozen=True)
class StreamingCapability:
    backend: str
    hook_abi: int
    hook_setter: str
    layer_count: int | None

    def to_dict(self) -> dict[str, object]:
        return asdict(self)


def set_native_stream_attention_hook(hook: Any | None) -> None:
    """Install (or clear) the one streaming hook (layers.py:53-59)."""
    global _NATIVE_STREAM_HOOK
    if hook is not None and not callable(hook):
        raise TypeError("native H3 streaming hook must be callable")
    if hook is not None and _NATIVE_STREAM_HOOK is not None:
        raise RuntimeError("a native H3 streaming hook is already installed")
    _NATIVE_STREAM_HOOK = hook


def native_stream_attention_hook() -> Any | None:
    return _NATIVE_STREAM_HOOK


@contextmanager
def native_stream_attention_metadata(
    token_tags: Any,
    commit_mask: Any,
    *,
    live_documents_hint: tuple[int, ...] | None = None,
    mlp_video_stride: int = 1,
) -> Iterator[None]:
    """Bind (token_tags, commit_mask) for the hook call sites (layers.py:62-82)."""
    if mlp_video_stride < 1:
        raise ValueError("native stream MLP video stride must be positive")
    if _NATIVE_STREAM_METADATA.get() is not None:
        raise RuntimeError("native H3 streaming attention metadata is nested")
    token = _NATIVE_STREAM_METADATA.set((token_tags, commit_mask))
    live_documents_token = _NATIVE_STREAM_LIVE_DOCUMENTS_HINT.set(live_documents_hint)
    stride_token = _NATIVE_STREAM_MLP_VIDEO_STRIDE.set(int(mlp_video_stride))
    try:
        yield
    finally:
        _NATIVE_STREAM_MLP_VIDEO_STRIDE.reset(stride_token)
        _NATIVE_STREAM_LIVE_DOCUMENTS_HINT.reset(live_documents_token)
        _NATIVE_STREAM_METADATA.reset(token)


def native_stream_attention_metadata_value() -> tuple[Any, Any] | None:
    return _NATIVE_STREAM_METADATA.get()


def native_stream_live_documents_hint() -> tuple[int, ...] | None:
    return _NATIVE_STREAM_LIVE_DOCUMENTS_HINT.get()


def streaming_capability(*, model: Any | None = None) -> StreamingCapability:
    """capability.py:23-31."""
    return StreamingCapability(
        backend="taomate_hd_amd_gfx950",
        hook_abi=STREAM_HOOK_ABI,
        hook_setter=f"{set_native_stream_attention_hook.__module__}.{set_native_stream_attention_hook.__name__}",
        layer_count=None if model is None else len(model.blocks),
    )


def set_official_attention_hook(hook: Any | None) -> None:
    """capability.py:34-39."""
    global _OFFICIAL_ATTENTION_HOOK
    set_native_stream_attention_hook(hook)
    _OFFICIAL_ATTENTION_HOOK = hook


def official_attention_hook_mode() -> str | None:
    """capability.py:42-47."""
    hook = _OFFICIAL_ATTENTION_HOOK
    if hook is None:
        return None
    mode = getattr(hook, "mode", None)
    return None if mode is None else str(getattr(mode, "value", mode))


def official_attention_denoise_step_index() -> int | None:
    """capability.py:50-51."""
    return getattr(_OFFICIAL_ATTENTION_HOOK, "_denoise_step_index", None)
