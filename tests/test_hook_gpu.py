"""The streaming hook + in-place KV cache on the GPU against the oracle's CPU
restatement of the reference hook and cache, over whole streaming sequences."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as oatt
from oracle import bf16
from oracle import stream as ost
from tests.helpers import err_stats, key_offset, randn_bf16, to_dev

pytestmark = pytest.mark.gpu

BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 1e-3
I8_COSINE = 0.999
LAYERS = ("blocks.0.attn", "blocks.1.attn")
H, D = 2, 128


class _Attn:
    softmax_scale = D ** -0.5


def _check(backend, got, want, exact=None):
    if backend == "sdpa":
        mx, mean = err_stats(got, want)
        assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (mx, mean)
    else:
        ref = want if exact is None else exact
        assert oatt.cosine(got, ref) >= I8_COSINE


def _qkv(t, seed):
    q = randn_bf16((t, H, D), seed)
    k = randn_bf16((t, H, D), seed + 1, offset=key_offset(H, D, seed + 2))
    v = randn_bf16((t, H, D), seed + 3)
    return q, k, v


def _call(torch, dev, hook, oracle_hook, layer, q, k, v, tags, mask, bounds, hint=None):
    out = hook(
        attention=_Attn(), layer_name=layer, query=to_dev(q, dev), key=to_dev(k, dev), value=to_dev(v, dev),
        token_tags=torch.tensor(tags, device=dev), commit_mask=torch.tensor(mask, device=dev),
        cu_seqlens=torch.tensor(bounds, dtype=torch.int32, device=dev), cu_seqlens_host=tuple(bounds),
        max_seqlen=max(b - a for a, b in zip(bounds, bounds[1:])), live_documents_hint=hint,
    )
    torch.cuda.synchronize()
    want = oracle_hook(layer, q, k, v, tags, mask, bounds, D ** -0.5, live_documents_hint=hint)
    return bf16.from_torch(out), want


@pytest.mark.parametrize("backend", ["sdpa", "sage_attn"])
def test_stream_noisy_commit_retain_sequence(torch_mod, dev, backend):
    torch = torch_mod
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingAttentionHook
    from taomate_hd_amd.hook import HookMode

    cache = HeadMajorRingKVCache(KVContract(layer_names=LAYERS, local_heads=H, head_dim=D))
    hook = StreamingAttentionHook(cache, attention_backend=backend)
    ocache = ost.CacheOracle(LAYERS)
    ohook = ost.HookOracle(ocache, backend=backend)
    exact_cache = ost.CacheOracle(LAYERS)
    exact_hook = ost.HookOracle(exact_cache, backend="sdpa")
    # packed layout [text 37, cond 20, audio 14, video 90, pad] -> 161 used, 192 rows
    tags, mask, bounds = ost.packed_layout(37, 20, 14, 90)
    T = len(tags)
    seed = 100
    for block in range(5):
        for mode in ("noisy", "clean_commit"):
            if mode == "clean_commit":
                cache.begin_clean_commit(block)
                ocache.begin_clean_commit(block)
                exact_cache.begin_clean_commit(block)
            hook.activate(mode=HookMode(mode), block_index=block)
            ohook.activate(mode, block)
            exact_hook.activate(mode, block)
            for layer in LAYERS:
                q, k, v = _qkv(T, seed)
                seed += 10
                got, want = _call(torch, dev, hook, ohook, layer, q, k, v, tags, mask, bounds)
                exact = exact_hook(layer, q, k, v, tags, mask, bounds, D ** -0.5)
                _check(backend, got, want, exact)
            hook.deactivate()
            ohook.deactivate()
            exact_hook.deactivate()
            if mode == "clean_commit":
                cache.commit()
                ocache.commit()
                exact_cache.commit()
                cache.retain_sink_and_recent_commits(2)
                ocache.retain_sink_and_recent_commits(2)
                exact_cache.retain_sink_and_recent_commits(2)
        # ledger and stored history are identical to the reference semantics
        assert cache.committed_blocks == ocache.block_index
        assert list(cache.commit_token_counts) == ocache.counts
        assert list(cache.commit_token_tags) == ocache.tags
        for layer in LAYERS:
            pair = cache.history(layer)
            want_k, want_v = ocache.history(layer)
            assert np.array_equal(bf16.from_torch(pair.key), want_k)
            assert np.array_equal(bf16.from_torch(pair.value), want_v)
    assert cache.retained_blocks == 3  # sink + 2 recent
    assert cache.history_video_tokens == ocache.counts[0] + 2 * 90
    if backend == "sage_attn":
        receipt = hook.attention_backend_receipt()
        assert receipt["kernel_calls"] > 0 and receipt["smooth_k"]


@pytest.mark.parametrize("backend", ["sdpa", "sage_attn"])
def test_stream_fused_progress_denoise(torch_mod, dev, backend):
    """Fused progress-denoise steps (staged previous media, recent / sink
    prefix views, the video-only shortened sink) against the oracle; the
    INT8-QK backend also checks the per-slot key-sum memo on those views."""
    torch = torch_mod
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingAttentionHook
    from taomate_hd_amd.hook import HookMode

    cache = HeadMajorRingKVCache(KVContract(layer_names=LAYERS, local_heads=H, head_dim=D))
    hook = StreamingAttentionHook(cache, attention_backend=backend)
    ocache = ost.CacheOracle(LAYERS)
    ohook = ost.HookOracle(ocache, backend=backend)
    exact_cache = ost.CacheOracle(LAYERS)
    exact_hook = ost.HookOracle(exact_cache)
    tags1, mask1, b1 = ost.packed_layout(9, 0, 6, 40, align=8)
    tags2, mask2, b2 = ost.packed_layout(5, 0, 8, 48, align=8)
    # packed pair: previous document (being committed) + current document
    tags = np.concatenate([tags1, tags2])
    mask = np.concatenate([mask1, mask2])
    bounds = (*b1, *(len(tags1) + b for b in b2[1:]))
    seed = 500

    caches = (cache, ocache, exact_cache)

    def run(mode, block, layout, hint=None, **kw):
        nonlocal seed
        t_, m_, b_ = layout
        hook.activate(mode=HookMode(mode), block_index=block, **kw)
        for o in (ohook, exact_hook):
            o.activate(mode, block, kw.get("fused_current_use_sink"), kw.get("fused_current_recent_blocks"))
        for layer in LAYERS:
            q, k, v = _qkv(len(t_), seed)
            seed += 10
            got, want = _call(torch, dev, hook, ohook, layer, q, k, v, t_, m_, b_, hint=hint)
            exact = exact_hook(layer, q, k, v, t_, m_, b_, D ** -0.5, live_documents_hint=hint)
            _check(backend, got, want, exact)
        hook.deactivate()
        ohook.deactivate()
        exact_hook.deactivate()

    for block in range(4):
        # fused variants against the current cache depth (rolled back)
        for recent, sink in ((2, True), (3, True), (1, True), (2, False), (None, None)):
            kw = {} if recent is None else {"fused_current_use_sink": sink, "fused_current_recent_blocks": recent}
            for c in caches:
                c.begin_clean_commit(block)
            run("fused_progress_denoise", block, (tags, mask, bounds), hint=(0, 2), **kw)
            for c in caches:
                c.rollback()
        # then commit this block through a fused step (or a plain clean commit)
        for c in caches:
            c.begin_clean_commit(block)
        if block % 2:
            run("fused_progress_denoise", block, (tags, mask, bounds), fused_current_use_sink=True,
                fused_current_recent_blocks=2)
        else:
            run("clean_commit", block, (tags1, mask1, b1))
        for c in caches:
            c.commit()
            c.retain_sink_and_recent_commits(2)
        assert list(cache.commit_token_tags) == ocache.tags
        for layer in LAYERS:
            pair = cache.history(layer)
            wk, wv = ocache.history(layer)
            assert np.array_equal(bf16.from_torch(pair.key), wk)
            assert np.array_equal(bf16.from_torch(pair.value), wv)
            if block >= 1:
                fk = cache.history_for_fused_current(layer, use_sink=True, recent_blocks=2)
                ok, ov = ocache.history_for_fused_current(layer, use_sink=True, recent_blocks=2)
                assert np.array_equal(bf16.from_torch(fk.key), ok)
                assert np.array_equal(bf16.from_torch(fk.value), ov)


@pytest.mark.parametrize("backend", ["sdpa", "sage_attn"])
def test_noncontiguous_commit_mask_and_empty_documents(torch_mod, dev, backend):
    torch = torch_mod
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingAttentionHook
    from taomate_hd_amd.hook import HookMode

    cache = HeadMajorRingKVCache(KVContract(layer_names=LAYERS[:1], local_heads=H, head_dim=D))
    hook = StreamingAttentionHook(cache, attention_backend=backend)
    ocache = ost.CacheOracle(LAYERS[:1])
    ohook = ost.HookOracle(ocache, backend=backend)
    exact_cache = ost.CacheOracle(LAYERS[:1])
    exact_hook = ost.HookOracle(exact_cache)
    T = 150
    rng = np.random.default_rng(3)
    mask = np.zeros(T, dtype=bool)
    mask[10:140] = rng.random(130) < 0.7  # interleaved condition/media rows
    tags = np.where(rng.random(T) < 0.5, 0, 2).astype(np.int64)
    tags[~mask] = 1
    tags[mask & (np.arange(T) % 7 == 0)] = 2
    tags[mask & (np.arange(T) % 7 == 1)] = 0
    bounds = (0, 0, 140, 140, 150)  # empty documents at both ends of the live one
    for block, mode in ((0, "noisy"), (0, "clean_commit"), (1, "noisy")):
        if mode == "clean_commit":
            for c in (cache, ocache, exact_cache):
                c.begin_clean_commit(block)
        hook.activate(mode=HookMode(mode), block_index=block)
        ohook.activate(mode, block)
        exact_hook.activate(mode, block)
        q, k, v = _qkv(T, 900 + block)
        got, want = _call(torch, dev, hook, ohook, LAYERS[0], q, k, v, tags, mask, bounds)
        exact = exact_hook(LAYERS[0], q, k, v, tags, mask, bounds, D ** -0.5)
        _check(backend, got, want, exact)
        hook.deactivate()
        ohook.deactivate()
        exact_hook.deactivate()
        if mode == "clean_commit":
            for c in (cache, ocache, exact_cache):
                c.commit()
    pair = cache.history(LAYERS[0])
    wk, wv = ocache.history(LAYERS[0])
    assert np.array_equal(bf16.from_torch(pair.key), wk)
    assert np.array_equal(bf16.from_torch(pair.value), wv)


def test_session_rollback_on_error(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingSession

    class Plan:
        phases = ("p0", "p1", "p2")

    cache = HeadMajorRingKVCache(KVContract(layer_names=LAYERS, local_heads=H, head_dim=D))
    tags, mask, bounds = ost.packed_layout(4, 0, 4, 24, align=8)
    T = len(tags)
    with StreamingSession(Plan(), cache=cache) as session:
        with session.noisy_step(0):
            pass
        with pytest.raises(RuntimeError, match="boom"):
            with session.clean_commit(0):
                q, k, v = (to_dev(x, dev) for x in _qkv(T, 5))
                session.hook(attention=_Attn(), layer_name=LAYERS[0], query=q, key=k, value=v,
                             token_tags=torch.tensor(tags, device=dev), commit_mask=torch.tensor(mask, device=dev),
                             cu_seqlens=None, cu_seqlens_host=bounds, max_seqlen=T)
                assert cache.clean_commit_active
                raise RuntimeError("boom")
        assert not cache.clean_commit_active and cache.committed_blocks == 0 and cache.retained_blocks == 0
        # a commit missing a layer is rejected and rolled back
        with pytest.raises(RuntimeError, match="missing attention layers"):
            with session.clean_commit(0):
                q, k, v = (to_dev(x, dev) for x in _qkv(T, 6))
                session.hook(attention=_Attn(), layer_name=LAYERS[0], query=q, key=k, value=v,
                             token_tags=torch.tensor(tags, device=dev), commit_mask=torch.tensor(mask, device=dev),
                             cu_seqlens=None, cu_seqlens_host=bounds, max_seqlen=T)
        assert cache.committed_blocks == 0 and not cache.clean_commit_active


def test_prestaged_chunk_used_without_pack(torch_mod, dev, monkeypatch):
    """preprocess_qkv_ (norm + RoPE that also stages the media rows) followed
    by the hook gives the same output, bit for bit, as norm + RoPE then the
    hook, and the hook packs one segment fewer."""
    torch = torch_mod
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingAttentionHook, fused_qkv_qk_norm_rope_
    from taomate_hd_amd import slots as slots_mod
    from taomate_hd_amd.hook import HookMode

    packs = []
    orig = slots_mod.KVSlot.pack

    def counting_pack(self, *a, **kw):
        packs.append(1)
        return orig(self, *a, **kw)

    monkeypatch.setattr(slots_mod.KVSlot, "pack", counting_pack)
    tags, mask, bounds = ost.packed_layout(37, 20, 14, 90)
    T, width = len(tags), H * D
    media0, media_n = 37 + 20, 14 + 90
    rng = np.random.default_rng(3)
    qkv = bf16.round_f32(rng.standard_normal((T, 3 * width)).astype(np.float32))
    w = bf16.to_torch(bf16.round_f32(1.0 + 0.1 * rng.standard_normal(D).astype(np.float32)), dev)
    ang = rng.uniform(-4, 4, (T, 48))
    cs = bf16.to_torch(bf16.round_f32(np.concatenate([np.cos(ang), np.sin(ang)], -1).astype(np.float32)), dev)
    pos = torch.arange(T, device=dev)
    outs, counts = [], []
    for prestage in (False, True):
        cache = HeadMajorRingKVCache(KVContract(layer_names=LAYERS, local_heads=H, head_dim=D))
        hook = StreamingAttentionHook(cache)
        hook.activate(mode=HookMode.NOISY, block_index=0)
        t = bf16.to_torch(qkv, dev)
        if prestage:
            hook.preprocess_qkv_(LAYERS[0], t, w, w, cs, pos, 1e-6, row0=media0, count=media_n)
        else:
            fused_qkv_qk_norm_rope_(t, w, w, cs, pos, 1e-6)
        del packs[:]
        q, k, v = (t[:, i * width : (i + 1) * width].view(T, H, D) for i in range(3))
        out = hook(attention=_Attn(), layer_name=LAYERS[0], query=q, key=k, value=v,
                   token_tags=torch.tensor(tags, device=dev), commit_mask=torch.tensor(mask, device=dev),
                   cu_seqlens=torch.tensor(bounds, dtype=torch.int32, device=dev), cu_seqlens_host=tuple(bounds),
                   max_seqlen=T)
        torch.cuda.synchronize()
        outs.append(out.clone())
        counts.append(len(packs))
        assert not hook._prestaged  # consumed by the call
        hook.deactivate()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert counts[1] == counts[0] - 1
    # staged but never consumed: recycled by deactivate
    hook.activate(mode=HookMode.NOISY, block_index=0)
    hook.preprocess_qkv_(LAYERS[0], bf16.to_torch(qkv, dev), w, w, cs, pos, 1e-6, row0=media0, count=media_n)
    slot = hook._prestaged[LAYERS[0]][0]
    hook.deactivate()
    assert not hook._prestaged and any(f is slot for f in hook._scratch._free)


@pytest.mark.parametrize("backend", ["sdpa", "sage_attn"])
def test_condition_cache_cached_rows_and_compact_output(torch_mod, dev, backend):
    """The condition cache as the hook sees it (attention_hook.py:322-324,
    445-465): a cached document's condition query rows read zero while its
    media rows still attend over the condition keys; with the compact order
    the hook returns only the kept rows (media rows through write_rows, the
    padding document through write_document).  Noisy, clean-commit and
    noisy-over-history calls through the drop-in session, against the
    oracle with the same decisions."""
    torch = torch_mod
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingSession, condition

    class Plan:
        phases = ("p0", "p1")

    cache = HeadMajorRingKVCache(KVContract(layer_names=LAYERS, local_heads=H, head_dim=D))
    ocache = ost.CacheOracle(LAYERS)
    ohook = ost.HookOracle(ocache, backend=backend)
    exact_cache = ost.CacheOracle(LAYERS)
    exact_hook = ost.HookOracle(exact_cache)
    tags, mask, bounds = ost.packed_layout(37, 20, 14, 90)  # doc 0 live (rows 0..160), doc 1 padding
    T = len(tags)
    condition_rows = set(range(0, 57))
    dropped_padding = set(range(170, 176))
    variants = [
        ((), None),
        ((0,), None),
        ((0,), [r for r in range(T) if r not in condition_rows]),
        ((0,), [r for r in range(T) if r not in condition_rows | dropped_padding]),
        ((), [r for r in range(T) if r not in dropped_padding]),
    ]
    seed = 700

    def step(block, mode, decisions):
        nonlocal seed
        for layer in LAYERS:
            q, k, v = _qkv(T, seed)
            seed += 10
            cached_docs, kept = decisions
            state = condition.ConditionLayerState(layer, cached_documents=cached_docs, compact_rows=kept, seq_len=T)
            with condition.condition_layer(state):
                out = session.hook(
                    attention=_Attn(), layer_name=layer, query=to_dev(q, dev), key=to_dev(k, dev),
                    value=to_dev(v, dev), token_tags=torch.tensor(tags, device=dev),
                    commit_mask=torch.tensor(mask, device=dev), cu_seqlens=None, cu_seqlens_host=tuple(bounds),
                    max_seqlen=T)
            torch.cuda.synchronize()
            kw = {"cached_documents": cached_docs, "compact_rows": kept}
            want = ohook(layer, q, k, v, tags, mask, bounds, D ** -0.5, **kw)
            exact = exact_hook(layer, q, k, v, tags, mask, bounds, D ** -0.5, **kw)
            got = bf16.from_torch(out)
            assert got.shape == want.shape
            if 0 in cached_docs and kept is None:
                assert np.all(got[sorted(condition_rows)] == 0)
            _check(backend, got, want, exact)

    with StreamingSession(Plan(), cache=cache, attention_backend=backend) as session:
        for i, decisions in enumerate(variants):
            with session.noisy_step(0):
                ohook.activate("noisy", 0)
                exact_hook.activate("noisy", 0)
                step(0, "noisy", decisions)
                ohook.deactivate()
                exact_hook.deactivate()
        with session.clean_commit(0):
            for c in (ocache, exact_cache):
                c.begin_clean_commit(0)
            ohook.activate("clean_commit", 0)
            exact_hook.activate("clean_commit", 0)
            step(0, "clean_commit", variants[2])
            ohook.deactivate()
            exact_hook.deactivate()
        for c in (ocache, exact_cache):
            c.commit()
        for decisions in variants[1:4]:
            with session.noisy_step(1):
                ohook.activate("noisy", 1)
                exact_hook.activate("noisy", 1)
                step(1, "noisy", decisions)
                ohook.deactivate()
                exact_hook.deactivate()
    for layer in LAYERS:
        pair = cache.history(layer)
        wk, wv = ocache.history(layer)
        assert np.array_equal(bf16.from_torch(pair.key), wk)
        assert np.array_equal(bf16.from_torch(pair.value), wv)


@pytest.mark.parametrize("backend", ["sdpa", "sage_attn"])
def test_stream_without_retention_beyond_one_launch(torch_mod, dev, backend, monkeypatch):
    """Every committed block kept (the reference's cache has no bound on the
    history it concatenates): after 15 blocks the media queries see more
    segments than one launch takes and the oldest are merged into one
    temporary slot; the outputs still follow the oracle hook call for call."""
    torch = torch_mod
    from taomate_hd_amd import HeadMajorRingKVCache, KVContract, StreamingAttentionHook
    from taomate_hd_amd.hook import HookMode

    from taomate_hd_amd import attention as attn_mod

    merges = []
    coalesce = attn_mod._coalesce_segments
    monkeypatch.setattr(attn_mod, "_coalesce_segments", lambda *a: merges.append(len(a[1])) or coalesce(*a))
    layer = LAYERS[0]
    cache = HeadMajorRingKVCache(KVContract(layer_names=(layer,), local_heads=H, head_dim=D))
    hook = StreamingAttentionHook(cache, attention_backend=backend)
    ocache, exact_cache = ost.CacheOracle((layer,)), ost.CacheOracle((layer,))
    ohook = ost.HookOracle(ocache, backend=backend)
    exact_hook = ost.HookOracle(exact_cache, backend="sdpa")
    tags, mask, bounds = ost.packed_layout(5, 4, 3, 21)
    T = len(tags)
    seed = 4000
    for block in range(20):
        for mode in ("noisy", "clean_commit"):
            if mode == "clean_commit":
                for c in (cache, ocache, exact_cache):
                    c.begin_clean_commit(block)
            hook.activate(mode=HookMode(mode), block_index=block)
            ohook.activate(mode, block)
            exact_hook.activate(mode, block)
            q, k, v = _qkv(T, seed)
            seed += 10
            got, want = _call(torch, dev, hook, ohook, layer, q, k, v, tags, mask, bounds)
            exact = exact_hook(layer, q, k, v, tags, mask, bounds, D ** -0.5)
            _check(backend, got, want if backend == "sdpa" else None, exact)
            hook.deactivate()
            ohook.deactivate()
            exact_hook.deactivate()
            if mode == "clean_commit":
                for c in (cache, ocache, exact_cache):
                    c.commit()
    assert cache.retained_blocks == 20
    assert merges and max(merges) > 20  # the last calls merged segments
