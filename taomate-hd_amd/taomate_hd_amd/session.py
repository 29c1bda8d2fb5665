"""Streaming session: the transactional state machine around the hook
(drop-in for ``H3StreamingSession``, src/taomate_hd/streaming/session.py:15-184)
plus the fixed continuation policy (src/taomate_hd/streaming/policy.py:7-16).

The reference writes each step kind (noisy, fused commit + denoise, clean
commit) as its own context manager.  Here a step is a ``_Step`` record: the
hook mode and activation keywords, the block whose staged K/V is committed
on success (if any), the block that must already have a noisy forward, and
the edits to the set of denoised blocks on success.  One runner executes any
step: it opens the commit, activates the hook, and on leaving either commits
(rolling back if the commit itself fails) or rolls back and re-raises; the
hook is deactivated on every path.  The contract kept from the reference is
the public surface: method names, keywords, the order of the checks, their
messages and exception types, and commit-or-rollback.

``plan`` is any object with a ``phases`` sequence (the reference passes its
``StreamPlan``, streaming/geometry.py); phases are handed back untouched.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import asdict, dataclass, field
from typing import Any, Callable, Iterator

from .capability import set_official_attention_hook, streaming_capability
from .hook import HookMode, StreamingAttentionHook
from .kvcache import HeadMajorRingKVCache, KVContract, kv_contract_from_model


@dataclass(frozen=True)
class StreamingInferencePolicy:
    """How many recent blocks a continuation keeps (policy.py:7-16)."""

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


@dataclass(frozen=True)
class _Step:
    """One transformer forward of the session, described by its effects."""

    mode: HookMode
    hook_block: int  # global block the hook is activated for
    yielded: Any  # what the context manager hands to the caller
    commit: int | None = None  # global block committed on success
    denoised_gone: tuple[int, ...] = ()  # removed from the denoised set on success
    denoised_new: tuple[int, ...] = ()  # added to the denoised set on success
    activate: dict[str, Any] = field(default_factory=dict)


class StreamingSession:
    """State machine around real transformer forwards.

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
        condition_attention_cached: Callable[[str, int], bool] | None = None,
        compact_condition_attention_output: Callable[[str, Any], Any] | None = None,
    ) -> None:
        if not hasattr(plan, "phases"):
            raise TypeError("plan must be a StreamPlan")
        if cache is not None and contract is not None and cache.contract != contract:
            raise ValueError("injected clean cache and KV contract differ")
        if cache is None:
            if contract is None and model is not None:
                contract = kv_contract_from_model(model)
            cache = HeadMajorRingKVCache(contract)
        self.plan = plan
        self.cache = cache
        # local block i of the plan is global block base + i of the cache
        self._base = cache.committed_blocks
        # the condition-cache queries default to the runtime's own (condition.resolve)
        self.hook = StreamingAttentionHook(
            cache,
            attention_backend=attention_backend,
            condition_attention_cached=condition_attention_cached,
            compact_condition_attention_output=compact_condition_attention_output,
        )
        self.capability = streaming_capability(model=model)
        self._fused_history = {
            "fused_current_use_sink": bool(fused_history_use_sink),
            "fused_current_recent_blocks": fused_history_recent_blocks,
        }
        self._installed = False
        self._denoised: set[int] = set()  # global blocks with a finished noisy forward

    # ---- installation
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
        if not self._installed:
            return
        set_official_attention_hook(None)
        self._installed = False

    def close(self) -> None:
        self.__exit__(None, None, None)

    # ---- checks shared by the steps
    def phase(self, block_index: int) -> Any:
        if isinstance(block_index, bool) or not isinstance(block_index, int):
            raise TypeError("block_index must be an integer")
        phases = self.plan.phases
        if not -len(phases) <= block_index < len(phases):
            raise ValueError(f"unknown streaming block {block_index}")
        return phases[block_index]

    def _next_block(self, block_index: int) -> tuple[Any, int]:
        """(phase, global index) of the block the cache expects next."""
        if not self._installed:
            raise RuntimeError("use H3StreamingSession as a context manager")
        phase = self.phase(block_index)
        if self._base + block_index != self.cache.committed_blocks:
            raise ValueError("streaming blocks must be processed and committed in order")
        return phase, self._base + block_index

    # ---- the one step runner
    @contextmanager
    def _run(self, step: _Step) -> Iterator[Any]:
        if step.commit is not None:
            self.cache.begin_clean_commit(step.commit)
        self.hook.activate(mode=step.mode, block_index=step.hook_block, **step.activate)
        try:
            try:
                yield step.yielded
            except BaseException:
                if step.commit is not None:
                    self.cache.rollback()
                raise
            if step.commit is not None:
                try:
                    self.cache.commit()
                except BaseException:
                    self.cache.rollback()
                    raise
            self._denoised.difference_update(step.denoised_gone)
            self._denoised.update(step.denoised_new)
        finally:
            self.hook.deactivate()

    # ---- the steps (session.py:85-181); their checks run on entering the block
    @contextmanager
    def noisy_step(self, block_index: int, *, denoise_step_index: int | None = None) -> Iterator[Any]:
        """One noisy forward of the next block; it only reads committed history."""
        phase, block = self._next_block(block_index)
        with self._run(_Step(HookMode.NOISY, block, phase, denoised_new=(block,),
                             activate={"denoise_step_index": denoise_step_index})) as phase:
            yield phase

    @contextmanager
    def fused_clean_commit_denoise(
        self, previous_block_index: int, current_block_index: int, *, denoise_step_index: int = 0
    ) -> Iterator[tuple[Any, Any]]:
        """Commit clean block N while running noisy step zero of block N + 1."""
        previous_phase, previous = self._next_block(previous_block_index)
        if current_block_index != previous_block_index + 1:
            raise ValueError("fused direct H3 blocks must be adjacent")
        current_phase = self.phase(current_block_index)
        if previous not in self._denoised:
            raise RuntimeError("fused direct commit requires the previous denoise output")
        with self._run(_Step(
            HookMode.FUSED_PROGRESS_DENOISE, previous, (previous_phase, current_phase), commit=previous,
            denoised_gone=(previous,), denoised_new=(previous + 1,),
            activate={**self._fused_history, "denoise_step_index": denoise_step_index},
        )) as phases:
            yield phases

    @contextmanager
    def clean_commit(self, block_index: int) -> Iterator[Any]:
        """The clean sigma=0 forward of a denoised block, committed on success."""
        phase, block = self._next_block(block_index)
        if block not in self._denoised:
            raise RuntimeError("a clean commit requires at least one noisy denoise forward")
        with self._run(_Step(HookMode.CLEAN_COMMIT, block, phase, commit=block, denoised_gone=(block,))) as phase:
            yield phase


# the reference's class name
H3StreamingSession = StreamingSession
