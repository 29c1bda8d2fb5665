"""Streaming session: the transactional state machine around the hook
(drop-in for src/taomate_hd/streaming/session.py:15-184) plus the fixed cache
policy (src/taomate_hd/streaming/policy.py:7-16).

``plan`` is any object with a ``phases`` sequence (the reference passes its
``StreamPlan``, streaming/geometry.py); phases are handed back untouched.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import asdict, dataclass
from typing import Any, Iterator

from .capability import set_official_attention_hook, streaming_capability
from .hook import HookMode, StreamingAttentionHook
from .kvcache import HeadMajorRingKVCache, KVContract, kv_contract_from_model


@dataclass(frozen=True)
class StreamingInferencePolicy:
    """policy.py:7-16."""

    max_prefix_blocks: int = 2
    cross_chunk_kv_recent_blocks: int = 2

    @property
    def recent_prefix_blocks(self) -> int:
        return min(self.max_prefix_blocks, self.cross_chunk_kv_recent_blocks)

    def to_dict(self) -> dict[str, object]:
        return asdict(self)


def apply_cross_chunk_cache_policy(cache: HeadMajorRingKVCache, policy: StreamingInferencePolicy | None = None) -> None:
    """After each commit: keep the sink plus the recent blocks (streaming/runtime.py:898-900)."""
    cache.retain_sink_and_recent_commits((policy or StreamingInferencePolicy()).recent_prefix_blocks)


class StreamingSession:
    """State machine around real transformer forwards (session.py:15-184).

    Noisy forwards only read committed history.  A clean sigma=0 forward
    stages all layers' K/V and commits the block atomically; any exception
    rolls the staged block back.
    """

    def __init__(
        self,
        plan: Any,
        *,
        model: Any | None = None,
        contract: KVContract | None = None,
        cache: HeadMajorRingKVCache | None = None,
        attention_backend: str = "sdpa",
        fused_history_use_sink: bool = False,
        fused_history_recent_blocks: int | None = None,
    ) -> None:
        if not hasattr(plan, "phases"):
            raise TypeError("plan must be a StreamPlan")
        self.plan = plan
        if cache is not None and contract is not None and cache.contract != contract:
            raise ValueError("injected clean cache and KV contract differ")
        resolved_contract = contract
        if resolved_contract is None and cache is None and model is not None:
            resolved_contract = kv_contract_from_model(model)
        self.cache = cache or HeadMajorRingKVCache(resolved_contract)
        self._block_index_base = self.cache.committed_blocks
        self.hook = StreamingAttentionHook(self.cache, attention_backend=attention_backend)
        self.capability = streaming_capability(model=model)
        self._installed = False
        self._noisy_blocks: set[int] = set()
        self._fused_history_use_sink = bool(fused_history_use_sink)
        self._fused_history_recent_blocks = fused_history_recent_blocks

    def __enter__(self) -> "StreamingSession":
        if self._installed:
            raise RuntimeError("H3 streaming session is already installed")
        set_official_attention_hook(self.hook)
        self._installed = True
        return self

    def __exit__(self, exc_type: Any, exc: Any, traceback: Any) -> None:
        if self.cache.clean_commit_active:
            self.cache.rollback()
        self.hook.deactivate()
        if self._installed:
            set_official_attention_hook(None)
            self._installed = False

    def phase(self, block_index: int) -> Any:
        if isinstance(block_index, bool) or not isinstance(block_index, int):
            raise TypeError("block_index must be an integer")
        try:
            return self.plan.phases[block_index]
        except IndexError as exc:
            raise ValueError(f"unknown streaming block {block_index}") from exc

    def _require_installed(self, block_index: int) -> Any:
        if not self._installed:
            raise RuntimeError("use H3StreamingSession as a context manager")
        phase = self.phase(block_index)
        if self._block_index_base + block_index != self.cache.committed_blocks:
            raise ValueError("streaming blocks must be processed and committed in order")
        return phase

    @contextmanager
    def noisy_step(self, block_index: int, *, denoise_step_index: int | None = None) -> Iterator[Any]:
        """Wrap exactly one noisy transformer forward (session.py:85-109)."""
        phase = self._require_installed(block_index)
        global_block_index = self._block_index_base + block_index
        self.hook.activate(mode=HookMode.NOISY, block_index=global_block_index, denoise_step_index=denoise_step_index)
        try:
            yield phase
        finally:
            self.hook.deactivate()
        self._noisy_blocks.add(global_block_index)

    @contextmanager
    def fused_clean_commit_denoise(
        self, previous_block_index: int, current_block_index: int, *, denoise_step_index: int = 0
    ) -> Iterator[tuple[Any, Any]]:
        """Commit clean block N while running noisy step zero of N+1 (session.py:111-150)."""
        previous_phase = self._require_installed(previous_block_index)
        if current_block_index != previous_block_index + 1:
            raise ValueError("fused direct H3 blocks must be adjacent")
        current_phase = self.phase(current_block_index)
        previous_global = self._block_index_base + previous_block_index
        current_global = self._block_index_base + current_block_index
        if previous_global not in self._noisy_blocks:
            raise RuntimeError("fused direct commit requires the previous denoise output")
        self.cache.begin_clean_commit(previous_global)
        self.hook.activate(
            mode=HookMode.FUSED_PROGRESS_DENOISE,
            block_index=previous_global,
            fused_current_use_sink=self._fused_history_use_sink,
            fused_current_recent_blocks=self._fused_history_recent_blocks,
            denoise_step_index=denoise_step_index,
        )
        try:
            yield (previous_phase, current_phase)
        except BaseException:
            self.cache.rollback()
            raise
        else:
            try:
                self.cache.commit()
            except BaseException:
                self.cache.rollback()
                raise
            self._noisy_blocks.remove(previous_global)
            self._noisy_blocks.add(current_global)
        finally:
            self.hook.deactivate()

    @contextmanager
    def clean_commit(self, block_index: int) -> Iterator[Any]:
        """Wrap the clean sigma=0 forward and commit on success (session.py:152-181)."""
        phase = self._require_installed(block_index)
        global_block_index = self._block_index_base + block_index
        if global_block_index not in self._noisy_blocks:
            raise RuntimeError("a clean commit requires at least one noisy denoise forward")
        self.cache.begin_clean_commit(global_block_index)
        self.hook.activate(mode=HookMode.CLEAN_COMMIT, block_index=global_block_index)
        try:
            yield phase
        except BaseException:
            self.cache.rollback()
            raise
        else:
            try:
                self.cache.commit()
            except BaseException:
                self.cache.rollback()
                raise
            else:
                self._noisy_blocks.remove(global_block_index)
        finally:
            self.hook.deactivate()

    def close(self) -> None:
        self.__exit__(None, None, None)


# the reference's class name
H3StreamingSession = StreamingSession
