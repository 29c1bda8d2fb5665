"""Pins the CPU oracle before the kernels are compared against it.

The reference ships no tests, fixtures or golden vectors for this path, so
each oracle function is pinned by closed forms, invariants, brute force on
tiny inputs, an independent library routine, or hand-derived cases chosen so
that a plausible mistake (dropped term, wrong sign/index, transposed operand,
wrong rounding mode) fails.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as oatt
from oracle import bf16
from oracle import quant as oq
from oracle import stream as ost


# ---------------------------------------------------------------- bf16
def test_bf16_known_values_and_ties():
    assert bf16.f32_to_bits(np.array([1.0], np.float32))[0] == 0x3F80
    assert bf16.bits_to_f32(np.array([0xC040], np.uint16))[0] == -3.0
    one_half_ulp = np.float32(1.0 + 2.0 ** -8)  # tie between 1 and 1 + 2^-7 -> even (1.0)
    three_half = np.float32(1.0 + 3 * 2.0 ** -8)  # tie between 1+2^-7 (odd) and 1+2^-6 -> 1+2^-6
    got = bf16.round_f32(np.array([one_half_ulp, three_half], np.float32))
    assert got[0] == 1.0 and got[1] == np.float32(1.0 + 2.0 ** -6)
    special = bf16.round_f32(np.array([np.inf, -np.inf, np.nan], np.float32))
    assert np.isinf(special[0]) and special[1] < 0 and np.isnan(special[2])


def test_bf16_roundtrip_all_patterns_and_torch_agreement():
    import torch

    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = bf16.bits_to_f32(bits)
    finite = np.isfinite(vals)
    assert np.array_equal(bf16.f32_to_bits(vals[finite]), bits[finite])
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 1e3
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()  # torch's own RNE conversion
    assert np.array_equal(bf16.round_f32(x), want)


# ---------------------------------------------------------------- quantizers
def test_token_quant_closed_forms():
    rng = np.random.default_rng(1)
    x = bf16.round_f32(rng.standard_normal((64, 300)).astype(np.float32))
    x[5] = 0.0
    q, s = oq.token_quant(x)
    assert q.dtype == np.int8 and s.shape == (64,)
    assert np.all(q[5] == 0) and s[5] == 0.0
    rows = [r for r in range(64) if r != 5]
    amax = np.abs(x[rows]).max(axis=1)
    # the largest magnitude of every row maps to +-127
    idx = np.abs(x[rows]).argmax(axis=1)
    assert np.array_equal(np.abs(q[rows, idx]), np.full(len(rows), 127))
    assert np.all(np.sign(q[rows, idx]) == np.sign(x[rows, idx]))
    # scale = amax / 127 and dequantization error <= scale / 2
    np.testing.assert_allclose(s[rows] * 127, amax, rtol=1e-6)
    err = np.abs(q[rows].astype(np.float64) * s[rows, None] - x[rows])
    assert np.all(err <= s[rows, None] * 0.5 * (1 + 1e-5))


def test_token_quant_ties_round_half_even():
    x = np.array([[127.0, 2.5, -3.5, 0.5, -0.5, 1.5]], np.float32)  # amax 127 -> multiplier 1.0
    q, s = oq.token_quant(x)
    assert q.tolist() == [[127, 2, -4, 0, 0, 2]] and s[0] == 1.0


# Rows whose second value is exactly half the row maximum, so the exact
# quotient is 63.5, a tie.  In float32 the two ways of forming it differ:
#   row A (amax 0.4765625):  x * fl(127 / amax) = 63.499996  but  x / fl(amax / 127) = 63.5
#   row B (amax 2.234375):   x * fl(127 / amax) = 63.5       but  x / fl(amax / 127) = 63.499996
# so the multiply form gives (63, 64) and the divide form (64, 63): each
# quantizer is pinned to its own stated form by these two rows.
FORM_ROWS = np.array([[0.4765625, 0.23828125, -0.23828125], [2.234375, 1.1171875, -1.1171875]], np.float32)


def test_token_quant_multiplies_by_127_over_amax():
    """vLLM's per-token form, stated in include/tmhd.h: rint(x * (127 / amax))."""
    for amax, x in FORM_ROWS[:, :2]:  # the premise: the two forms really differ here
        mul = np.float32(x) * (np.float32(127.0) / np.float32(amax))
        div = np.float32(x) / (np.float32(amax) / np.float32(127.0))
        assert np.rint(mul) != np.rint(div)
    q, s = oq.token_quant(FORM_ROWS)
    assert q.tolist() == [[127, 63, -63], [127, 64, -64]]
    assert s.tolist() == [np.float32(0.4765625) / np.float32(127), np.float32(2.234375) / np.float32(127)]


def test_weight_quant_divides_by_the_scale():
    """The reference's weight form (w8a8.py:177-178): round(W / (amax / 127))."""
    q, s = oq.weight_quant(FORM_ROWS)
    assert q.tolist() == [[127, 64, -64], [127, 63, -63]]


def test_weight_quant_closed_forms():
    rng = np.random.default_rng(2)
    w = bf16.round_f32((rng.standard_normal((32, 256)) * 0.02).astype(np.float32))
    q, s = oq.weight_quant(w)
    idx = np.abs(w).argmax(axis=1)
    assert np.array_equal(np.abs(q[np.arange(32), idx]), np.full(32, 127))
    assert q.min() >= -127 and q.max() <= 127
    err = np.abs(q.astype(np.float64) * s[:, None] - w)
    assert np.all(err <= s[:, None] * 0.5 * (1 + 1e-5))
    # ties to even with scale exactly 1 (row max 127)
    q2, s2 = oq.weight_quant(np.array([[127.0, -127.0, 2.5, 3.5, -0.5]], np.float32))
    assert s2[0] == 1.0 and q2.tolist() == [[127, -127, 2, 4, 0]]
    # the 1e-12 scale floor: amax 1e-10 would give 7.9e-13, floored to 1e-12 -> q = 100, not 127
    tiny = np.array([[1e-10, -5e-11, 0.0]], np.float32)
    q3, s3 = oq.weight_quant(tiny)
    assert s3[0] == np.float32(1e-12)
    assert q3[0, 0] == 100 and q3[0, 1] == -50
    q4, s4 = oq.weight_quant(np.zeros((1, 8), np.float32))
    assert s4[0] == np.float32(1e-12) and np.all(q4 == 0)


def test_int_gemm_brute_force():
    rng = np.random.default_rng(3)
    a = rng.integers(-128, 128, size=(5, 70), dtype=np.int8)
    b = rng.integers(-127, 128, size=(3, 70), dtype=np.int8)
    a[0] = -128
    b[0] = -127
    want = np.zeros((5, 3), np.int64)
    for i in range(5):
        for j in range(3):
            for kk in range(70):
                want[i, j] += int(a[i, kk]) * int(b[j, kk])
    assert np.array_equal(oq.int_gemm(a, b), want.astype(np.int32))
    assert oq.int_gemm(a, b)[0, 0] == 128 * 127 * 70


def test_scaled_mm_epilogue_forms():
    acc = np.array([[3, -7], [2 ** 24 + 1, 100]], dtype=np.int32)
    one = np.ones(2, np.float32)
    got = oq.scaled_mm_epilogue(acc, one, one, None)
    # int -> fp32 conversion rounds 2^24 + 1 to 2^24 before bf16 rounding
    assert got.tolist() == [[3.0, -7.0], [2.0 ** 24, 100.0]]
    a_s = np.array([0.5, 2.0], np.float32)
    b_s = np.array([0.25, 4.0], np.float32)
    got = oq.scaled_mm_epilogue(acc[:1], a_s[:1], b_s, np.array([1.0, -1.0], np.float32))
    assert got.tolist() == [[3 * 0.25 * 0.5 + 1.0, -7 * 4.0 * 0.5 - 1.0]]


def test_smooth_k_mean_and_block_quant():
    k = np.full((300, 2, 4), 1.5, np.float32)
    assert np.all(oq.smooth_k_mean(k) == 1.5)
    k2 = np.zeros((4, 1, 1), np.float32)
    k2[:, 0, 0] = [1, 2, 3, 4]
    assert oq.smooth_k_mean(k2)[0, 0] == 2.5
    rng = np.random.default_rng(4)
    k3 = bf16.round_f32(rng.standard_normal((1000, 3, 8)).astype(np.float32))
    m = oq.smooth_k_mean(k3)
    # order independent and equal to the correctly rounded fp64 mean for this data
    assert np.array_equal(m, oq.smooth_k_mean(k3[rng.permutation(1000)]))
    assert np.array_equal(m, bf16.round_f32(k3.astype(np.float64).mean(axis=0).astype(np.float32)))
    # blocks of 128 rows are independent; an all-zero block quantizes to zeros with scale 0
    x = bf16.round_f32(rng.standard_normal((300, 2, 8)).astype(np.float32))
    x[128:256] = 0.0
    q, s = oq.block_quant(x)
    assert s.shape == (2, 3) and np.all(s[:, 1] == 0) and np.all(q[128:256] == 0)
    x2 = x.copy()
    x2[290] *= 100.0
    q2, s2 = oq.block_quant(x2)
    assert np.array_equal(q2[:128], q[:128]) and np.array_equal(s2[:, 0], s[:, 0])
    qa, sa = oq.token_quant(x[:128, 0, :].reshape(1, -1))  # one block of one head == one "row"
    assert np.array_equal(q[:128, 0, :].reshape(1, -1), qa) and sa[0] == s[0, 0]


# ---------------------------------------------------------------- attention
def _rand(shape, seed):
    return bf16.round_f32(np.random.default_rng(seed).standard_normal(shape).astype(np.float32))


def test_attention_closed_forms():
    q = _rand((7, 2, 16), 10)
    v = _rand((9, 2, 16), 11)
    # a single key returns its value
    np.testing.assert_allclose(oatt.attention_fp64(q, _rand((1, 2, 16), 12), v[:1], 0.3), np.broadcast_to(v[:1], (7, 2, 16)), atol=1e-12)
    # identical keys give the mean of the values
    k_const = np.repeat(_rand((1, 2, 16), 13), 9, axis=0)
    np.testing.assert_allclose(oatt.attention_fp64(q, k_const, v, 0.3), np.broadcast_to(v.mean(0), (7, 2, 16)), atol=1e-12)
    # one dominant logit selects its value row
    k = _rand((9, 2, 16), 14) * 0.01
    k[4] = q[0] * 50.0
    out = oatt.attention_fp64(q[:1], k, v, 1.0)
    np.testing.assert_allclose(out[0], v[4], atol=1e-6)


def test_attention_permutation_and_lse_merge():
    q = _rand((11, 3, 32), 20)
    k = _rand((40, 3, 32), 21)
    v = _rand((40, 3, 32), 22)
    s = 32 ** -0.5
    base = oatt.attention_fp64(q, k, v, s)
    perm = np.random.default_rng(0).permutation(40)
    np.testing.assert_allclose(oatt.attention_fp64(q, k[perm], v[perm], s), base, atol=1e-12)
    o1, l1 = oatt.attention_fp64(q, k[:13], v[:13], s), oatt.attention_lse_fp64(q, k[:13], s)
    o2, l2 = oatt.attention_fp64(q, k[13:], v[13:], s), oatt.attention_lse_fp64(q, k[13:], s)
    w1 = 1.0 / (1.0 + np.exp(l2 - l1))
    merged = o1 * w1[..., None] + o2 * (1 - w1)[..., None]
    np.testing.assert_allclose(merged, base, atol=1e-12)


def test_attention_matches_torch_sdpa():
    import torch

    q = _rand((33, 2, 64), 30)
    k = _rand((70, 2, 64), 31)
    v = _rand((70, 2, 64), 32)
    got = oatt.sdpa_cpu(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), 0.125).numpy()
    np.testing.assert_allclose(got, oatt.attention_fp64(q, k, v, 0.125), atol=2e-5)


def test_i8qk_attention_algebra():
    q = _rand((200, 2, 64), 40)
    kseg = [_rand((150, 2, 64), 41) + 0.7, _rand((90, 2, 64), 42) - 0.3]
    vseg = [_rand((150, 2, 64), 43), _rand((90, 2, 64), 44)]
    out, ops = oatt.i8qk_attention(q, kseg, vseg, 0.125)
    # dequantized operands: q ~ q_i8 * s_q, k ~ k_i8 * s_k + mean; the mean only shifts
    # each query row's logits by a constant, which softmax removes
    qb = np.arange(200) // 128
    q_deq = ops["q_i8"].astype(np.float64) * ops["q_scale"].T[qb][:, :, None]
    k_deq = []
    for kq, ks in zip(ops["k_i8"], ops["k_scale"]):
        kb = np.arange(kq.shape[0]) // 128
        k_deq.append(kq.astype(np.float64) * ks.T[kb][:, :, None])
    k_all = np.concatenate(k_deq)
    v_all = np.concatenate(vseg)
    np.testing.assert_allclose(oatt.attention_fp64(q_deq, k_all, v_all, 0.125), out, atol=1e-10)
    np.testing.assert_allclose(oatt.attention_fp64(q_deq, k_all + ops["mean"][None], v_all, 0.125), out, atol=1e-10)
    exact = oatt.attention_fp64(q, np.concatenate(kseg), v_all, 0.125)
    assert oatt.cosine(out, exact) > 0.999


def test_i8qk_cpu_baseline_equals_the_fp64_emulation():
    import torch

    q = _rand((300, 2, 64), 45)
    kseg = [_rand((200, 2, 64), 46) + 0.4, _rand((77, 2, 64), 47)]
    vseg = [_rand((200, 2, 64), 48), _rand((77, 2, 64), 49)]
    want, _ = oatt.i8qk_attention(q, kseg, vseg, 0.125)
    got = oatt.i8qk_attention_cpu(torch.from_numpy(q), [torch.from_numpy(k) for k in kseg],
                                  torch.from_numpy(np.concatenate(vseg)), 0.125).numpy()
    # same quantized operands: only fp32 rounding of the softmax and P.V differs
    np.testing.assert_allclose(got, want, atol=2e-6)


# ---------------------------------------------------------------- stream semantics
def test_packed_layout_hand_derived():
    tags, mask, bounds = ost.packed_layout(3, 2, 2, 4, align=8)
    assert tags.tolist() == [1, 1, 1, 0, 0, 2, 2, 0, 0, 0, 0] + [-1] * 5  # 11 rows aligned to 16
    assert mask.tolist() == [False] * 5 + [True] * 6 + [False] * 5
    assert bounds == (0, 11, 16)


def test_cache_ledger_hand_derived():
    layers = ("a", "b")
    c = ost.CacheOracle(layers)
    blocks = [(2, 2, 0, 0, 0), (0, 2, 0), (2, 0), (0, 0, 2)]
    base = 0
    for i, tags in enumerate(blocks):
        n = len(tags)
        k = np.arange(base, base + n, dtype=np.float32)[:, None, None]  # row id as the value
        c.begin_clean_commit(i)
        for layer in layers:
            c.stage(layer, k, -k, np.array(tags), np.ones(n, bool))
        c.commit()
        c.retain_sink_and_recent_commits(2)
        base += n
    # after b2: sink filtered to video rows 2,3,4; after b3: b1 evicted
    assert c.counts == [3, 2, 3]
    assert c.tags == [(0, 0, 0), (2, 0), (0, 0, 2)]
    assert c.history("a")[0][:, 0, 0].tolist() == [2, 3, 4, 8, 9, 10, 11, 12]
    assert np.array_equal(c.history("b")[1], -c.history("b")[0])
    with pytest.raises(ValueError):
        c.begin_clean_commit(3)  # out of order
    c.begin_clean_commit(4)
    with pytest.raises(ValueError):
        c.stage("a", np.zeros((2, 1, 1)), np.zeros((2, 1, 1)), np.array([0, 0]), np.ones(2, bool))  # no audio
    c.rollback()


def test_cache_fused_current_selection_hand_derived():
    c = ost.CacheOracle(("a",))
    for i, tags in enumerate([(2, 0, 0), (0, 2), (0, 0, 2, 2)]):
        n = len(tags)
        c.begin_clean_commit(i)
        c.stage("a", np.full((n, 1, 1), i, np.float32), np.zeros((n, 1, 1)), np.array(tags), np.ones(n, bool))
        c.commit()
        if i == 1:
            c.retain_sink_and_recent_commits(2)  # nothing evicted yet, flag set
    # 3 blocks, sink still has audio (no retain after the third commit)
    k = c.history_for_fused_current("a", use_sink=True, recent_blocks=2)[0][:, 0, 0]
    assert k.tolist() == [0, 0, 2, 2, 2, 2]  # sink video rows + newest block
    k = c.history_for_fused_current("a", use_sink=False, recent_blocks=2)[0][:, 0, 0]
    assert k.tolist() == [2, 2, 2, 2]
    assert c.history_for_fused_current("a", use_sink=True, recent_blocks=1)[0][:, 0, 0].tolist() == [0, 0]


def test_hook_oracle_visibility_hand_derived():
    rng = np.random.default_rng(7)
    T, Hh, Dd = 10, 1, 8
    q, k, v = (rng.standard_normal((T, Hh, Dd)).astype(np.float32) for _ in range(3))
    tags = np.array([1, 1, 1, 2, 0, 0, 0, -1, -1, -1])
    mask = np.array([False] * 3 + [True] * 4 + [False] * 3)
    bounds = (0, 7, 10)
    c = ost.CacheOracle(("a",))
    hist_k = rng.standard_normal((5, Hh, Dd)).astype(np.float32)
    hist_v = rng.standard_normal((5, Hh, Dd)).astype(np.float32)
    c.history_kv["a"] = (hist_k, hist_v)
    c.counts, c.tags, c.block_index = [5], [(2, 0, 0, 0, 0)], 1
    h = ost.HookOracle(c)
    h.activate("noisy", 1)
    out = h("a", q, k, v, tags, mask, bounds, 0.5)
    cond, media, pad = [0, 1, 2], [3, 4, 5, 6], [7, 8, 9]
    np.testing.assert_allclose(out[cond], oatt.attention_fp64(q[cond], k[cond], v[cond], 0.5), atol=1e-12)
    kv_k = np.concatenate([k[cond], hist_k, k[media]])
    kv_v = np.concatenate([v[cond], hist_v, v[media]])
    np.testing.assert_allclose(out[media], oatt.attention_fp64(q[media], kv_k, kv_v, 0.5), atol=1e-12)
    np.testing.assert_allclose(out[pad], oatt.attention_fp64(q[pad], k[pad], v[pad], 0.5), atol=1e-12)
    h.deactivate()
    with pytest.raises(RuntimeError):
        h("a", q, k, v, tags, mask, bounds, 0.5)


def test_hook_oracle_condition_cache_hand_derived():
    """Cached condition attention (attention_hook.py:445-465): the document's
    condition query rows read zero, its media rows are unchanged (they still
    attend over the condition keys); the compact output holds the kept rows
    in order, and a kept row nobody writes stays zero."""
    rng = np.random.default_rng(8)
    T, Hh, Dd = 10, 1, 8
    q, k, v = (rng.standard_normal((T, Hh, Dd)).astype(np.float32) for _ in range(3))
    tags = np.array([1, 1, 1, 2, 0, 0, 0, -1, -1, -1])
    mask = np.array([False] * 3 + [True] * 4 + [False] * 3)
    bounds = (0, 7, 10)
    c = ost.CacheOracle(("a",))
    h = ost.HookOracle(c)
    h.activate("noisy", 0)
    full = h("a", q, k, v, tags, mask, bounds, 0.5)
    cached = h("a", q, k, v, tags, mask, bounds, 0.5, cached_documents=(0,))
    assert np.all(cached[:3] == 0) and np.array_equal(cached[3:], full[3:])
    media_want = oatt.attention_fp64(q[3:7], k[:7], v[:7], 0.5)  # condition keys stay visible
    np.testing.assert_allclose(cached[3:7], media_want, atol=1e-12)
    assert np.array_equal(h("a", q, k, v, tags, mask, bounds, 0.5, cached_documents=(1,)), full)  # not live
    kept = [3, 4, 5, 6, 8, 9]
    compact = h("a", q, k, v, tags, mask, bounds, 0.5, cached_documents=(0,), compact_rows=kept)
    assert compact.shape == (6, Hh, Dd) and np.array_equal(compact, full[kept])
    with_cond = h("a", q, k, v, tags, mask, bounds, 0.5, cached_documents=(0,), compact_rows=[1, 4, 9])
    assert np.all(with_cond[0] == 0) and np.array_equal(with_cond[1:], full[[4, 9]])


# ---------------------------------------------------------------- QK norm + RoPE
from oracle import rope as orope  # noqa: E402


def test_round_bf16_bit_trick_matches_rne_and_edges():
    # finite values: the integer formula is round-to-nearest-even (independent implementation in oracle.bf16)
    x = np.random.default_rng(1).standard_normal(200000).astype(np.float32) * np.float32(3e4)
    assert np.array_equal(orope.round_bf16(x).view(np.uint32), bf16.round_f32(x).view(np.uint32))
    pats = np.array([0x3F808000, 0x3F818000, 0x7F7FFFFF, 0xFFFFFFFF, 0x7F800000, 0x80000000], np.uint32)
    got = orope.round_bf16(pats.view(np.float32)).view(np.uint32)
    # ties to even, overflow to inf, the all-ones NaN pattern wraps to +0 (as the fp32 add does), inf and -0 kept
    assert list(got) == [0x3F800000, 0x3F820000, 0x7F800000, 0x00000000, 0x7F800000, 0x80000000]


def test_lane_channels_partition_the_row_and_pair_rotations():
    for d, r in [(128, 128), (128, 64), (128, 0), (64, 64), (64, 32), (64, 16)]:
        ch = orope.lane_channels(d, r)
        assert ch.shape == (d // 8, 8) and sorted(ch.ravel()) == list(range(d))
        for j in range(r // 8):  # each rotary lane holds (d, d + r/2) pairs at the same places
            assert list(ch[j, 4:] - ch[j, :4]) == [r // 2] * 4 and ch[j, 3] < r // 2


def test_sum_squares_order_against_float64():
    x = np.random.default_rng(2).standard_normal((50, 128)).astype(np.float32)
    for r in (0, 64, 128):
        got = orope.sum_squares(x, r).astype(np.float64)
        want = (x.astype(np.float64) ** 2).sum(-1)
        assert np.all(np.abs(got - want) <= 1e-5 * want)
    # hand-derived order, head_dim 16 rotary 16: lane 0 holds channels 0-3 and
    # 8-11, lane 1 holds 4-7 and 12-15.  With 2^12 at channel 4, lane 1 starts
    # at 2^24 and each + 1 after it rounds back (ties to even); lane 0 sums
    # 8 ones; total 2^24 + 8.  Contiguous chunks of 8 would give
    # (1 + 1 + 1 + 1 + 2^24 ...) + 8 = 2^24 + 12, the ones first 2^24 + 16.
    y = np.ones((1, 16), np.float32)
    y[0, 4] = 2.0 ** 12
    assert orope.sum_squares(y, 16)[0] == np.float32(2.0 ** 24 + 8.0)
    assert orope.sum_squares(y, 0)[0] == np.float32(2.0 ** 24 + 12.0)
    # fused multiply-add: with x0 = 2^-59, x1 = 2^-68 (1 + 2^-7), x1^2 =
    # 2^-136 + 2^-142 + 2^-150 exactly.  2^-118 + x1^2 sits just above the
    # midpoint between float32 neighbours 2^-141 apart, so one rounding gives
    # 2^-118 + 2^-136 + 2^-141; a separate multiply would round x1^2 to
    # 2^-136 + 2^-142 (a float32 subnormal) and the add would tie to even at
    # 2^-118 + 2^-136.
    z = np.zeros((1, 16), np.float32)
    z[0, 0], z[0, 1] = 2.0 ** -59, 2.0 ** -68 * (1 + 2.0 ** -7)
    assert orope.sum_squares(z, 16)[0] == np.float32(2.0 ** -118 + 2.0 ** -136 + 2.0 ** -141)
    assert np.float32(z[0, 0] * z[0, 0]) + np.float32(z[0, 1] * z[0, 1]) == np.float32(2.0 ** -118 + 2.0 ** -136)


def _rope_case(tokens=7, heads=3, head_dim=128, rotary=128, seed=5):
    rng = np.random.default_rng(seed)
    qkv = bf16.round_f32(rng.standard_normal((tokens, 3 * heads * head_dim)).astype(np.float32) * 2)
    qw = bf16.round_f32(1.0 + 0.1 * rng.standard_normal(head_dim).astype(np.float32))
    kw = bf16.round_f32(1.0 + 0.1 * rng.standard_normal(head_dim).astype(np.float32))
    half = rotary // 2
    ang = rng.uniform(0, 6.3, (11, half))
    cache = bf16.round_f32(np.concatenate([np.cos(ang), np.sin(ang)], -1).astype(np.float32))
    pos = rng.integers(0, 11, tokens)
    return qkv, qw, kw, cache, pos


def test_qkv_norm_rope_closed_forms():
    qkv, qw, kw, cache, pos = _rope_case()
    T, H, D, R = 7, 3, 128, 128
    out = orope.qkv_norm_rope(qkv, qw, kw, cache, pos, 1e-6, H)
    # V untouched
    assert np.array_equal(out[:, 2 * H * D:], qkv[:, 2 * H * D:])
    # identity rotation (cos = 1, sin = 0): plain RMSNorm, within one bf16 ulp of the float64 formula
    ident = np.concatenate([np.ones((11, R // 2)), np.zeros((11, R // 2))], -1).astype(np.float32)
    nrm = orope.qkv_norm_rope(qkv, qw, kw, ident, pos, 1e-6, H)[:, : 2 * H * D].reshape(T, 2, H, D)
    x = qkv[:, : 2 * H * D].reshape(T, 2, H, D).astype(np.float64)
    w = np.stack([qw, kw]).astype(np.float64)[None, :, None, :]
    ref = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * w
    assert np.all(np.abs(nrm - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-30)
    # rotate-half in float64: out[d] = n[d] cos - n[d+h] sin (d < h), n[d] cos + n[d-h] sin (d >= h)
    h = R // 2
    rows = cache[pos].astype(np.float64)
    c = np.concatenate([rows[:, :h], rows[:, :h]], -1)[:, None, None, :]
    s = np.concatenate([rows[:, h:], rows[:, h:]], -1)[:, None, None, :]
    rot = np.concatenate([-nrm[..., h:], nrm[..., :h]], -1).astype(np.float64)
    want = nrm.astype(np.float64) * c + rot * s
    got = out[:, : 2 * H * D].reshape(T, 2, H, D)
    assert np.all(np.abs(got - want) <= 2.0 ** -6 * (np.abs(nrm) + np.abs(rot)) * 1.0 + 1e-30)
    # a rotation keeps the norm of each (d, d + h) pair
    n2 = nrm[..., :h].astype(np.float64) ** 2 + nrm[..., h:].astype(np.float64) ** 2
    g2 = got[..., :h].astype(np.float64) ** 2 + got[..., h:].astype(np.float64) ** 2
    assert np.allclose(g2, n2, rtol=3e-2, atol=1e-6)


def test_qkv_norm_rope_partial_rotary_and_weights_select_q_k():
    qkv, qw, kw, cache, pos = _rope_case(rotary=64)
    T, H, D, R = 7, 3, 128, 64
    out = orope.qkv_norm_rope(qkv, qw, kw, cache, pos, 1e-6, H)[:, : 2 * H * D].reshape(T, 2, H, D)
    ident = np.concatenate([np.ones((11, R // 2)), np.zeros((11, R // 2))], -1).astype(np.float32)
    nrm = orope.qkv_norm_rope(qkv, qw, kw, ident, pos, 1e-6, H)[:, : 2 * H * D].reshape(T, 2, H, D)
    # channels past the rotary span are only normalized
    assert np.array_equal(out[..., R:], nrm[..., R:])
    # Q uses q_weight and K uses k_weight: swapping the weights swaps nothing else
    sw = orope.qkv_norm_rope(qkv, kw, qw, ident, pos, 1e-6, H)[:, : 2 * H * D].reshape(T, 2, H, D)
    x = qkv[:, : 2 * H * D].reshape(T, 2, H, D)
    inv = np.float32(1) / np.sqrt(orope.sum_squares(x, R) / np.float32(D) + np.float32(1e-6))
    assert np.array_equal(sw[:, 0], orope.round_bf16((x[:, 0] * inv[:, 0, :, None]) * kw))
    assert np.array_equal(nrm[:, 1], orope.round_bf16((x[:, 1] * inv[:, 1, :, None]) * kw))


def test_qk_norm_rope_equals_merged_form_with_duplicated_tables():
    # the model's unmerged path builds per-token tables by repeating the cache
    # halves (model/layers.py:415-420); both reference kernels must then agree
    qkv, qw, kw, cache, pos = _rope_case(rotary=96)
    T, H, D, R = 7, 3, 128, 96
    merged = orope.qkv_norm_rope(qkv, qw, kw, cache, pos, 1e-6, H)[:, : 2 * H * D].reshape(T, 2, H, D)
    rows = cache[pos]
    cos = np.concatenate([rows[:, : R // 2], rows[:, : R // 2]], -1)
    sin = np.concatenate([rows[:, R // 2:], rows[:, R // 2:]], -1)
    x = qkv[:, : 2 * H * D].reshape(T, 2, H, D)
    assert np.array_equal(orope.qk_norm_rope(x[:, 0], qw, cos, sin, 1e-6), merged[:, 0])
    assert np.array_equal(orope.qk_norm_rope(x[:, 1], kw, cos, sin, 1e-6), merged[:, 1])


def test_qk_norm_rope_per_channel_tables_closed_form():
    rng = np.random.default_rng(8)
    T, H, D, R = 5, 2, 64, 48
    x = bf16.round_f32(rng.standard_normal((T, H, D)).astype(np.float32))
    w = bf16.round_f32(1 + 0.1 * rng.standard_normal(D).astype(np.float32))
    ang = rng.uniform(-3, 3, (T, R))  # every channel its own angle
    cos = bf16.round_f32(np.cos(ang).astype(np.float32))
    sin = bf16.round_f32(np.sin(ang).astype(np.float32))
    out = orope.qk_norm_rope(x, w, cos, sin, 1e-6).astype(np.float64)
    n = orope.qk_norm_rope(x, w, np.ones((T, R), np.float32), np.zeros((T, R), np.float32), 1e-6).astype(np.float64)
    h = R // 2
    c, s = cos[:, None, :].astype(np.float64), sin[:, None, :].astype(np.float64)
    want_lo = n[..., :h] * c[..., :h] - n[..., h:R] * s[..., :h]
    want_hi = n[..., h:R] * c[..., h:] + n[..., :h] * s[..., h:]
    tol = 2.0 ** -6 * (np.abs(n[..., :h]) + np.abs(n[..., h:R])) + 1e-30
    assert np.all(np.abs(out[..., :h] - want_lo) <= tol)
    assert np.all(np.abs(out[..., h:R] - want_hi) <= tol)
    assert np.array_equal(out[..., R:], n[..., R:])
    # float32 tables are rounded to bf16 on load: identical to pre-rounded tables
    cos32, sin32 = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    assert np.array_equal(orope.qk_norm_rope(x, w, cos32, sin32, 1e-6), orope.qk_norm_rope(x, w, cos, sin, 1e-6))


# ---------------------------------------------------------------- RMSNorm / AdaLN / gate rows
from oracle import adaln as oada  # noqa: E402


def test_row_sum_order_hand_cases():
    # 2^12 in chunk 0 (partial 0) and ones in chunk 1 (partial 1): partial 0
    # stays 2^24 (each + 1 ties back to even), the tree adds 8 -> 2^24 + 8.
    # One sequential chain over both chunks would give 2^24.
    y = np.zeros((1, 16), np.float32)
    y[0, 0] = 2.0 ** 12
    y[0, 1:8] = 1.0
    y[0, 8:] = 1.0
    assert oada.sum_squares_row(y)[0] == np.float32(2.0 ** 24 + 8.0)
    # two rounds: partial 0 holds chunks 0 then 64, in that order; ones first
    # (8), then 2^24 -> 2^24 + 8, and the ones after it tie back: 2^24 + 8.
    # Chunk 64 first would give 2^24.
    z = np.zeros((1, 1024), np.float32)
    z[0, :8] = 1.0
    z[0, 512] = 2.0 ** 12
    z[0, 513:520] = 1.0
    assert oada.sum_squares_row(z)[0] == np.float32(2.0 ** 24 + 8.0)
    # fused multiply-add inside a partial (see the rope case)
    f = np.zeros((1, 16), np.float32)
    f[0, 0], f[0, 1] = 2.0 ** -59, 2.0 ** -68 * (1 + 2.0 ** -7)
    assert oada.sum_squares_row(f)[0] == np.float32(2.0 ** -118 + 2.0 ** -136 + 2.0 ** -141)
    # random rows: float64 agreement
    x = np.random.default_rng(3).standard_normal((20, 5376)).astype(np.float32)
    want = (x.astype(np.float64) ** 2).sum(-1)
    assert np.all(np.abs(oada.sum_squares_row(x) - want) <= 1e-5 * want)


def test_modulate_and_gate_add_equal_the_reference_eager_bf16_path():
    # the reference's unfused fallback (model/layers.py:126-128, 146) runs in
    # bf16 torch, which rounds after every op: the fused kernels' R() chain
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(11)
    rows, cols, trows = 37, 256, 3
    x = bf16.round_f32(rng.standard_normal((rows, cols)).astype(np.float32) * 3)
    br = bf16.round_f32(rng.standard_normal((rows, cols)).astype(np.float32))
    scale = bf16.round_f32(rng.standard_normal((trows, cols)).astype(np.float32) * 0.3)
    shift = bf16.round_f32(rng.standard_normal((trows, cols)).astype(np.float32) * 0.3)
    gate = bf16.round_f32(rng.standard_normal((trows, cols)).astype(np.float32))
    idx = rng.integers(0, trows, rows)
    t = lambda a: torch.tensor(a, dtype=torch.float32).to(torch.bfloat16)
    ti = torch.tensor(idx, dtype=torch.long)
    eager_mod = (t(x) * (1.0 + t(scale).index_select(0, ti)) + t(shift).index_select(0, ti)).to(torch.bfloat16)
    eager_gate = (t(x) + t(gate).index_select(0, ti) * t(br)).to(torch.bfloat16)
    assert np.array_equal(oada.modulate(x, scale, shift, idx), eager_mod.float().numpy())
    assert np.array_equal(oada.gate_add(x, gate, br, idx), eager_gate.float().numpy())


def test_rms_norm_family_closed_forms():
    rng = np.random.default_rng(12)
    rows, cols = 9, 5376
    x = bf16.round_f32(rng.standard_normal((rows, cols)).astype(np.float32) * 2)
    w = bf16.round_f32(1 + 0.1 * rng.standard_normal(cols).astype(np.float32))
    out = oada.rms_norm(x, w, 1e-6).astype(np.float64)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + 1e-6) * w
    assert np.all(np.abs(out - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-30)
    # constant rows: x * inv = sign(x) within float rounding; eps pulls a zero row to zero
    c = np.full((2, 64), 3.0, np.float32)
    c[1] = 0.0
    n = oada.rms_norm(c, np.ones(64, np.float32), 1e-6)
    assert np.all(n[0] == 1.0) and np.all(n[1] == 0.0)
    # modulation identities: scale 0 / shift 0 keeps the normalized row; scale -1 gives shift
    idx = np.zeros(rows, np.int64)
    zeros = np.zeros((1, cols), np.float32)
    nrm = oada.rms_norm(x, w, 1e-6)
    assert np.array_equal(oada.rms_norm_modulate(x, w, zeros, zeros, idx, 1e-6), nrm)
    sh = bf16.round_f32(rng.standard_normal((1, cols)).astype(np.float32))
    assert np.array_equal(oada.rms_norm_modulate(x, w, zeros - 1, sh, idx, 1e-6), np.broadcast_to(sh, x.shape))
    # the residual form is gate-add then the same norm: gate 0 leaves the residual
    g0 = np.zeros((1, cols), np.float32)
    h, o = oada.residual_gate_rms_norm_modulate(x, x[::-1].copy(), g0, w, zeros, zeros, idx, 1e-6)
    assert np.array_equal(h, x) and np.array_equal(o, nrm)


def test_apply_rope_equals_the_reference_eager_bf16_path_and_identity():
    # the reference's unfused rotation (model/layers.py:194-197) in bf16 torch
    # rounds after every op: the fused kernel's R() chain
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(21)
    T, H, D, R = 9, 3, 128, 96
    x = bf16.round_f32(rng.standard_normal((T, H, D)).astype(np.float32) * 2)
    ang = rng.uniform(-4, 4, (T, R // 2))
    cos = bf16.round_f32(np.concatenate([np.cos(ang), np.cos(ang)], -1).astype(np.float32))
    sin = bf16.round_f32(np.concatenate([np.sin(ang), np.sin(ang)], -1).astype(np.float32))
    tb = lambda a: torch.tensor(a, dtype=torch.float32).to(torch.bfloat16)
    rot = tb(x)[..., :R]
    first, second = torch.chunk(rot, 2, dim=-1)
    eager = torch.cat((rot * tb(cos)[:, None] + torch.cat((-second, first), -1) * tb(sin)[:, None], tb(x)[..., R:]), -1)
    assert np.array_equal(orope.apply_rope(x, cos, sin), eager.float().numpy())
    ones, zeros = np.ones((T, R), np.float32), np.zeros((T, R), np.float32)
    assert np.array_equal(orope.apply_rope(x, ones, zeros), x)
    # norm + rope with an identity norm weight path: qk_norm_rope = apply_rope(normalized)
    n = orope.qk_norm_rope(x, np.ones(D, np.float32), ones, zeros, 1e-6)
    assert np.array_equal(orope.qk_norm_rope(x, np.ones(D, np.float32), cos, sin, 1e-6), orope.apply_rope(n, cos, sin))


def test_swiglu_closed_forms():
    # sigmoid(0) = 1/2 -> activation 0; large positive gates pass through
    # (g * 1), large negative gates vanish; R(R(g s) u) structure
    g = np.array([[0.0, 20.0, -20.0, 1.0]], np.float32)
    u = np.array([[3.0, 2.0, 5.0, 1.0]], np.float32)
    out = oada.swiglu(np.concatenate([g, u], -1))
    assert out[0, 0] == 0.0 and out[0, 1] == 40.0 and abs(out[0, 2]) < 1e-6
    want = 1.0 / (1.0 + np.exp(-1.0))  # silu(1) = sigmoid(1)
    assert abs(out[0, 3] - want) <= 2.0 ** -8 * want


# ---------------------------------------------------------------- Ulysses layouts
from oracle import ulysses as oul  # noqa: E402


@pytest.mark.parametrize("heads,world", [(8, 2), (28, 4), (7, 2), (10, 4), (5, 4), (3, 1)])
def test_ulysses_layouts_round_trip_and_reshape_form(heads, world):
    rng = np.random.default_rng(heads * 10 + world)
    dim, tokens = 8, 5
    local = oul.local_heads(heads, world)
    # every rank's merged projection; values tag (rank, token, part, head, channel)
    x = [rng.standard_normal((tokens, 3 * heads * dim)).astype(np.float32) for _ in range(world)]
    sends = [oul.qkv_send(xi, heads, dim, world) for xi in x]
    if heads % world == 0:
        for xi, si in zip(x, sends):
            assert np.array_equal(si, oul.qkv_send_reshape(xi, heads, dim, world))
    for si in sends:  # padded heads are zero
        pad = world * local - heads
        if pad:
            assert not si[-1, :, :, local - pad:].any()
    received = oul.all_to_all(sends)
    full = np.concatenate(x).reshape(world * tokens, 3, heads, dim)  # the whole sequence, rank order
    for r in range(world):
        q, k, v = oul.qkv_receive(received[r])
        for p, part in enumerate((q, k, v)):
            for l in range(local):
                head = r * local + l
                want = full[:, p, head] if head < heads else np.zeros((world * tokens, dim), np.float32)
                assert np.array_equal(part[:, l], want)
        tm = oul.all_to_all([oul.qkv_send_token_major(xi, heads, dim, world) for xi in x])[r]
        assert np.array_equal(tm.reshape(world * tokens, 3, local, dim).transpose(1, 0, 2, 3), np.stack([q, k, v]))
    # heads -> sequence: each rank's attention output over all tokens of its heads comes back
    outs = [oul.qkv_receive(received[r])[0] for r in range(world)]  # [U*T, L, D] per rank
    back = oul.all_to_all([o.reshape(world, tokens, local, dim) for o in outs])
    for r in range(world):
        got = oul.attention_receive(back[r], heads)
        assert np.array_equal(got, x[r].reshape(tokens, 3, heads, dim)[:, 0])
