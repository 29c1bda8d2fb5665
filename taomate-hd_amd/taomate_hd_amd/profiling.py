"""Event-based per-component timing of kernel launches.

The counterpart of the reference's CUDA-event ``InferenceComponentTimer``
(src/taomate_hd/inference/acceleration.py:67-182): events are recorded on the
current stream around each launch, so a summary after synchronisation gives
the device time of each component ("pack", "qk_quant", "attention", ...).
Ranges also appear as roctx markers when ``torch.cuda.nvtx`` is available
(it maps to roctx on ROCm), like the reference's NVTX ranges
(src/taomate_hd/inference/profiling.py:7-22).
"""

from __future__ import annotations

from collections import defaultdict
from contextlib import contextmanager
from typing import Any, Iterator


class ComponentTimer:
    def __init__(self, torch: Any, *, markers: bool = False) -> None:
        self._torch = torch
        self._events: dict[str, list[tuple[Any, Any]]] = defaultdict(list)
        self._markers = markers

    @contextmanager
    def region(self, name: str) -> Iterator[None]:
        torch = self._torch
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        if self._markers:
            torch.cuda.nvtx.range_push(name)
        start.record()
        try:
            yield
        finally:
            end.record()
            if self._markers:
                torch.cuda.nvtx.range_pop()
            self._events[name].append((start, end))

    def reset(self) -> None:
        self._events.clear()

    def summary(self) -> dict[str, dict[str, float]]:
        """Per component: launches, total and mean device milliseconds (synchronises)."""
        self._torch.cuda.synchronize()
        out = {}
        for name, pairs in self._events.items():
            total = sum(s.elapsed_time(e) for s, e in pairs)
            out[name] = {"calls": len(pairs), "total_ms": total, "mean_ms": total / max(len(pairs), 1)}
        return out


@contextmanager
def maybe_region(timer: ComponentTimer | None, name: str) -> Iterator[None]:
    if timer is None:
        yield
    else:
        with timer.region(name):
            yield
