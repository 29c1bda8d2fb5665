"""taomate_hd_amd: MI355X (gfx950) streaming KV-cache attention for TaoMate-HD.

A drop-in for the reference's per-layer streaming attention hook
(src/taomate_hd/streaming/attention_hook.py), its clean audio-video KV cache
(streaming/cache.py), the session around them (streaming/session.py) and the
selective W8A8 projection ops (inference/w8a8.py).  All compute runs in the
hand-written HIP kernels of libtmhd.so; nothing falls back to the CPU.
"""

from . import _native
from .attention import QKQuantWorkspace, segment_attention
from .slots import KVSlot, SlotPool, SlotView, vt_position

__all__ = [
    "_native",
    "QKQuantWorkspace",
    "segment_attention",
    "KVSlot",
    "SlotPool",
    "SlotView",
    "vt_position",
]

__version__ = "0.1.0"
