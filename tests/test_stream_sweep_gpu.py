"""Seeded random streams through the hook and the in-place cache against the
oracle's restatement of the reference hook and cache: random head counts and
head dims, one or two layers, 3-5 blocks, 1-3 documents per call (empty ones
among them) with the live document at a random place, interleaved commit
masks with video / audio tags, noisy steps, commits through clean-commit or
fused progress-denoise steps (random sink / recent views), 0-2 recent
blocks retained after each commit with the sink video-only or whole, random
condition-cache decisions (cached documents, compact output rows), both
backends."""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import attention as oatt
from oracle import bf16
from oracle import stream as ost
from tests.helpers import err_stats, key_offset, randn_bf16, to_dev

pytestmark = pytest.mark.gpu

# a wider sweep: TMHD_SWEEP_CASES=<streams> TMHD_SWEEP_SEED=<another base>
N_STREAMS = int(os.environ.get("TMHD_SWEEP_CASES", "8"))
SEED0 = int(os.environ.get("TMHD_SWEEP_SEED", "31000"))


def _layout(rng: np.random.Generator):
    """(tags, commit mask, document bounds, live document) of one call: one
    live document between 0-2 others, its media rows interleaved with
    condition rows."""
    ndoc = int(rng.integers(1, 4))
    live = int(rng.integers(0, ndoc))
    tags, mask, bounds = [], [], [0]
    for d in range(ndoc):
        if d == live:
            n = int(rng.integers(20, 260))
            m = rng.random(n) < rng.uniform(0.3, 0.9)
            m[rng.choice(n, 2, replace=False)] = True  # at least two media rows
            t = np.where(rng.random(n) < 0.8, 0, 2)  # media: video 0 / audio 2
            media = np.nonzero(m)[0]
            t[media[0]], t[media[-1]] = 0, 2  # a commit holds video and audio rows (cache.py contract)
            t[~m] = np.where(rng.random(int((~m).sum())) < 0.5, 1, 0)  # condition: text 1 / cond 0
        else:
            n = int(rng.integers(0, 60))
            m = np.zeros(n, bool)
            t = np.where(rng.random(n) < 0.5, 1, -1)
        tags.append(t.astype(np.int64))
        mask.append(m)
        bounds.append(bounds[-1] + n)
    return np.concatenate(tags), np.concatenate(mask), tuple(bounds), live


STREAMS = [dict(seed=SEED0 + 97 * s, backend=("sdpa", "sage_attn")[s % 2]) for s in range(N_STREAMS)]


@pytest.mark.parametrize("stream", STREAMS, ids=[f"{s['backend']}-{s['seed']}" for s in STREAMS])
def test_random_stream_matches_oracle(torch_mod, dev, stream):
    torch = torch_mod
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingAttentionHook, condition
    from taomate_hd_amd.hook import HookMode

    rng = np.random.default_rng(stream["seed"])
    backend = stream["backend"]
    heads, dim = int(rng.integers(1, 4)), int(rng.choice([64, 128]))
    layers = ("blocks.0.attn", "blocks.1.attn")[: int(rng.integers(1, 3))]
    cache = HeadMajorRingKVCache(KVContract(layer_names=layers, local_heads=heads, head_dim=dim))
    hook = StreamingAttentionHook(cache, attention_backend=backend)
    ocache, exact_cache = ost.CacheOracle(layers), ost.CacheOracle(layers)
    ohook, exact_hook = ost.HookOracle(ocache, backend=backend), ost.HookOracle(exact_cache)

    class Attn:
        softmax_scale = dim ** -0.5

    seed = stream["seed"]

    def decisions(tags, mask, bounds, live_docs):
        """Random condition-cache decisions for one call: cached live documents
        (their condition rows are skipped) and, or not, a compact row order
        that drops those rows and random rows of the other documents."""
        if rng.random() >= 0.35:
            return (), None
        cached = tuple(d for d in live_docs if rng.random() < 0.6)
        if rng.random() < 0.5:
            return cached, None
        keep = np.ones(len(tags), bool)
        for d, (a, b) in enumerate(zip(bounds, bounds[1:])):
            if d in cached:
                keep[a:b] &= mask[a:b]  # its condition rows leave the compact order
            elif d not in live_docs:
                keep[a:b] &= rng.random(b - a) < 0.7  # rows of other documents may be dropped
        return cached, [int(r) for r in np.nonzero(keep)[0]]

    def step(mode, block, tags, mask, bounds, hint=None, **kw):
        nonlocal seed
        total = len(tags)
        live_docs = hint if hint is not None else tuple(
            d for d, (a, b) in enumerate(zip(bounds, bounds[1:])) if mask[a:b].any())
        hook.activate(mode=HookMode(mode), block_index=block, **kw)
        for o in (ohook, exact_hook):
            o.activate(mode, block, kw.get("fused_current_use_sink"), kw.get("fused_current_recent_blocks"))
        for layer in layers:
            seed += 10
            q = randn_bf16((total, heads, dim), seed)
            k = randn_bf16((total, heads, dim), seed + 1, offset=key_offset(heads, dim, seed + 2))
            v = randn_bf16((total, heads, dim), seed + 3)
            cached, kept = decisions(tags, mask, bounds, live_docs)
            state = condition.ConditionLayerState(layer, cached_documents=cached, compact_rows=kept)
            with condition.condition_layer(state):
                out = hook(
                    attention=Attn(), layer_name=layer, query=to_dev(q, dev), key=to_dev(k, dev),
                    value=to_dev(v, dev), token_tags=torch.tensor(tags, device=dev),
                    commit_mask=torch.tensor(mask, device=dev),
                    cu_seqlens=torch.tensor(bounds, dtype=torch.int32, device=dev), cu_seqlens_host=bounds,
                    max_seqlen=max(b - a for a, b in zip(bounds, bounds[1:])), live_documents_hint=hint,
                )
            torch.cuda.synchronize()
            got = bf16.from_torch(out)
            kwc = {"cached_documents": cached, "compact_rows": kept}
            want = ohook(layer, q, k, v, tags, mask, bounds, dim ** -0.5, live_documents_hint=hint, **kwc)
            exact = exact_hook(layer, q, k, v, tags, mask, bounds, dim ** -0.5, live_documents_hint=hint, **kwc)
            assert got.shape == want.shape and state.attention_output_compact == (kept is not None)
            if backend == "sdpa":
                mx, mean = err_stats(got, want)
                # few-key documents give O(1) outputs whose bf16 rounding alone nears 1e-3
                mean_round = float(np.abs(bf16.round_f32(want.astype(np.float32)) - want).mean())
                assert mx <= 2e-2 and mean <= max(1e-3, 1.5 * mean_round), (block, mode, layer, mx, mean)
            else:
                assert oatt.cosine(got, exact) >= 0.999, (block, mode, layer)
        hook.deactivate()
        ohook.deactivate()
        exact_hook.deactivate()

    for block in range(int(rng.integers(3, 6))):
        tags, mask, bounds, live = _layout(rng)
        step("noisy", block, tags, mask, bounds)
        for c in (cache, ocache, exact_cache):
            c.begin_clean_commit(block)
        if rng.random() < 0.5:
            step("clean_commit", block, tags, mask, bounds)
        else:
            # the block's media committed by a fused step: its document, then the next chunk's
            tags2, mask2, bounds2, live2 = _layout(rng)
            ftags, fmask = np.concatenate([tags, tags2]), np.concatenate([mask, mask2])
            fbounds = (*bounds, *(len(tags) + b for b in bounds2[1:]))
            kw = {}
            if rng.random() < 0.7:
                kw = dict(fused_current_use_sink=bool(rng.integers(0, 2)),
                          fused_current_recent_blocks=int(rng.integers(1, 4)))
            step("fused_progress_denoise", block, ftags, fmask, fbounds,
                 hint=(live, len(bounds) - 1 + live2), **kw)
        for c in (cache, ocache, exact_cache):
            c.commit()
        keep, video_only = int(rng.integers(0, 3)), bool(rng.integers(0, 2))
        for c in (cache, ocache, exact_cache):
            c.retain_sink_and_recent_commits(keep, sink_video_only=video_only)
        assert list(cache.commit_token_counts) == ocache.counts
        assert list(cache.commit_token_tags) == ocache.tags
        for layer in layers:
            pair = cache.history(layer)
            want_k, want_v = ocache.history(layer)
            assert np.array_equal(bf16.from_torch(pair.key), want_k)
            assert np.array_equal(bf16.from_torch(pair.value), want_v)
