"""Parity of the HIP kernels (called through the C ABI) against the oracle."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as oatt
from oracle import bf16
from oracle import quant as oq
from tests.helpers import err_stats, key_offset, randn_bf16, to_dev

pytestmark = pytest.mark.gpu

# BF16 attention gate: max abs <= 2e-2 and mean abs <= 1e-3 vs fp32/fp64 SDPA
BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 1e-3
# INT8-QK gate: cosine >= 0.999 vs fp32 SDPA on the unquantized inputs
I8_COSINE = 0.999


def _slots(torch, dev, k, v, splits):
    from taomate_hd_amd import KVSlot

    views, off = [], 0
    kd, vd = to_dev(k, dev), to_dev(v, dev)
    for n in splits:
        slot = KVSlot(torch, heads=k.shape[1], head_dim=k.shape[2], capacity=n, device=dev)
        slot.pack(kd, vd, row0=off, count=n)
        views.append(slot.view())
        off += n
    return views


def test_pack_roundtrip_and_padding(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import KVSlot, vt_position

    H, D, T = 3, 128, 150
    k = randn_bf16((T, H, D), 1)
    v = randn_bf16((T, H, D), 2)
    kd, vd = to_dev(k, dev), to_dev(v, dev)
    rows = torch.tensor([5, 149, 0, 77, 77, 3] + list(range(10, 100)), dtype=torch.int32, device=dev)
    slot = KVSlot(torch, heads=H, head_dim=D, capacity=200, device=dev)
    slot.k.fill_(7.0)
    slot.vt.fill_(7.0)
    slot.pack(kd, vd, rows=rows)
    torch.cuda.synchronize()
    sel = rows.cpu().numpy()
    kk = bf16.from_torch(slot.k)  # [H, cap, D]
    vt = bf16.from_torch(slot.vt)  # [H, D, cap]
    n = len(sel)
    assert np.array_equal(kk[:, :n, :], k[sel].transpose(1, 0, 2))
    cols = np.array([vt_position(t) for t in range(n)])
    assert np.array_equal(vt[:, :, cols], v[sel].transpose(1, 2, 0))
    pad_end = (n + 63) // 64 * 64
    assert np.all(kk[:, n:pad_end, :] == 0)
    pad_cols = np.array([vt_position(t) for t in range(n, pad_end)])
    assert np.all(vt[:, :, pad_cols] == 0)
    # untouched beyond the 64-row padding
    assert np.all(kk[:, pad_end:, :] == 7.0)
    # range form
    slot2 = KVSlot(torch, heads=H, head_dim=D, capacity=64, device=dev)
    slot2.pack(kd, vd, row0=100, count=50)
    torch.cuda.synchronize()
    assert np.array_equal(bf16.from_torch(slot2.k)[:, :50, :], k[100:150].transpose(1, 0, 2))
    key, value = slot2.token_major()
    assert np.array_equal(bf16.from_torch(key), k[100:150])
    assert np.array_equal(bf16.from_torch(value), v[100:150])


@pytest.mark.parametrize(
    "D,dst,n,zero_to,use_rows",
    [(128, 70, 50, 200, True), (128, 0, 150, 150, False), (64, 3, 61, 64, False), (64, 100, 0, 190, True),
     (128, 130, 1, 131, False), (128, 64, 64, 0, True)],
)
def test_pack_through_the_c_abi_every_position(torch_mod, dev, D, dst, n, zero_to, use_rows):
    """tmhd_kv_pack through the C ABI with unaligned ``dst`` and ``zero_to``:
    every slot position of K and of the transposed V is the data row, zero or
    the slot's earlier contents, as the position's class says (positions
    dst .. dst + n data, then zeros up to zero_to, the rest untouched)."""
    torch = torch_mod
    from taomate_hd_amd import _native, vt_position

    H, T, cap = 3, 160, 256
    k = randn_bf16((T, H, D), 11 + D)
    v = randn_bf16((T, H, D), 12 + D)
    sel = np.random.default_rng(n + dst).integers(0, T, size=n).astype(np.int32) if use_rows else np.arange(5, 5 + n)
    kd, vd = to_dev(k, dev), to_dev(v, dev)
    rows = torch.tensor(sel, dtype=torch.int32, device=dev) if use_rows else None
    gen = torch.Generator(device=dev).manual_seed(3)
    ks = torch.randn((H, cap, D), generator=gen, device=dev).to(torch.bfloat16)
    vts = torch.randn((H, D, cap), generator=gen, device=dev).to(torch.bfloat16)
    k0, v0 = bf16.from_torch(ks), bf16.from_torch(vts)
    lib = _native.load()
    st = lib.tmhd_kv_pack(_native.ptr(kd), _native.ptr(vd), kd.stride(0), kd.stride(1),
                          _native.ptr(rows) if use_rows and n else None, 5, n, _native.ptr(ks), _native.ptr(vts),
                          cap * D, cap * D, cap, dst, zero_to, H, D, _native.stream_ptr(torch, dev))
    _native.check(st, "tmhd_kv_pack")
    torch.cuda.synchronize()
    want_k, want_vt = k0.copy(), v0.copy()
    for p in range(cap):
        if dst <= p < dst + n:
            want_k[:, p, :] = k[sel[p - dst]]
        elif dst + n <= p < zero_to:
            want_k[:, p, :] = 0
        else:
            continue
        want_vt[:, :, (p // 64) * 64 + vt_position(p % 64)] = want_k[:, p, :] if p >= dst + n else v[sel[p - dst]]
    assert np.array_equal(bf16.from_torch(ks).view(np.uint16), want_k.view(np.uint16))
    assert np.array_equal(bf16.from_torch(vts).view(np.uint16), want_vt.view(np.uint16))


ATTN_CASES = [
    # heads, dim, lq, segment token counts
    (8, 64, 256, [768, 256]),  # plumbing config: 768 history + 256 self
    (2, 128, 300, [100, 37, 500]),
    (3, 128, 513, [64, 1, 63, 129]),
    (1, 128, 1, [5]),
    (2, 64, 700, [1000, 333, 4, 65, 2, 128, 7, 300]),
]


@pytest.mark.parametrize("heads,dim,lq,splits", ATTN_CASES)
def test_bf16_attention_matches_fp64(torch_mod, dev, heads, dim, lq, splits):
    torch = torch_mod
    from taomate_hd_amd import segment_attention

    n = sum(splits)
    q = randn_bf16((lq, heads, dim), 10)
    k = randn_bf16((n, heads, dim), 11, offset=key_offset(heads, dim, 13))
    v = randn_bf16((n, heads, dim), 12)
    views = _slots(torch, dev, k, v, splits)
    out = segment_attention(torch, to_dev(q, dev), views, scale=dim ** -0.5)
    torch.cuda.synchronize()
    got = bf16.from_torch(out)
    want = oatt.attention_fp64(q, k, v, dim ** -0.5)
    mx, mean = err_stats(got, want)
    assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (mx, mean)


def test_bf16_attention_row_gather_scatter(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import segment_attention

    H, D, T = 4, 128, 400
    q = randn_bf16((T, H, D), 20)
    k = randn_bf16((T, H, D), 21)
    v = randn_bf16((T, H, D), 22)
    views = _slots(torch, dev, k, v, [T])
    rng = np.random.default_rng(0)
    rows = np.sort(rng.choice(T, size=170, replace=False))
    qd = to_dev(q, dev)
    # strided query view: every other token of a doubled buffer
    qbig = torch.zeros((2 * T, H, D), dtype=torch.bfloat16, device=dev)
    qbig[::2] = qd
    out = torch.full((T, H, D), 3.0, dtype=torch.bfloat16, device=dev)
    rows_d = torch.tensor(rows, dtype=torch.int32, device=dev)
    segment_attention(torch, qbig[::2], views, scale=D ** -0.5, q_rows=rows_d, out=out, o_rows=rows_d)
    torch.cuda.synchronize()
    got = bf16.from_torch(out)
    want = oatt.attention_fp64(q[rows], k, v, D ** -0.5)
    mx, mean = err_stats(got[rows], want)
    assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS
    untouched = np.setdiff1d(np.arange(T), rows)
    assert np.all(got[untouched] == 3.0)


@pytest.mark.parametrize("heads,dim,lq,splits", [(4, 128, 600, [300, 700, 129]), (2, 64, 256, [768, 256])])
def test_i8qk_attention(torch_mod, dev, heads, dim, lq, splits):
    torch = torch_mod
    from taomate_hd_amd import segment_attention

    n = sum(splits)
    q = randn_bf16((lq, heads, dim), 30)
    k = randn_bf16((n, heads, dim), 31, offset=key_offset(heads, dim, 33))
    v = randn_bf16((n, heads, dim), 32)
    views = _slots(torch, dev, k, v, splits)
    out, qv = segment_attention(
        torch, to_dev(q, dev), views, scale=dim ** -0.5, backend="i8qk", return_quant=True
    )
    torch.cuda.synchronize()
    ksegs, vsegs, off = [], [], 0
    for s in splits:
        ksegs.append(k[off : off + s])
        vsegs.append(v[off : off + s])
        off += s
    want_q, ops = oatt.i8qk_attention(q, ksegs, vsegs, dim ** -0.5)
    # quantized operands: bit-exact
    assert np.array_equal(bf16.from_torch(qv["k_mean"]), ops["mean"])
    qi8 = qv["q_i8"].cpu().numpy()  # [H, qcap, D]
    assert np.array_equal(qi8[:, :lq, :], ops["q_i8"].transpose(1, 0, 2))
    assert np.all(qi8[:, lq:, :] == 0)
    nqb = ops["q_scale"].shape[1]
    assert np.array_equal(qv["q_scale"].cpu().numpy()[:, :nqb], ops["q_scale"])
    for i, s in enumerate(splits):
        ki8 = qv["k_i8"][i].cpu().numpy()
        assert np.array_equal(ki8[:, :s, :], ops["k_i8"][i].transpose(1, 0, 2))
        assert np.array_equal(qv["k_scale"][i].cpu().numpy()[:, : ops["k_scale"][i].shape[1]], ops["k_scale"][i])
    got = bf16.from_torch(out)
    ref32 = oatt.attention_fp64(q, k, v, dim ** -0.5)
    assert oatt.cosine(got, ref32) >= I8_COSINE
    mx, mean = err_stats(got, want_q)
    assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (mx, mean)


@pytest.mark.parametrize("dim", [64, 128])
def test_i8qk_largest_scores(torch_mod, dev, dim):
    """Every quantized operand at +-127, so every INT8 score is +-127^2 * D
    (2,064,512 at D 128), the largest |q.k| the path produces: each query row
    is +-p and the keys alternate +p / -p (p a fixed +-1 pattern per head), so
    the key mean is exactly 0.  The kernel's score chain start holds these
    exactly; a query row of sign s attends to the keys of sign s, a uniform
    average of their values."""
    torch = torch_mod
    from taomate_hd_amd import segment_attention

    heads, lq, splits = 2, 256, [300, 212]
    n = sum(splits)
    rng = np.random.default_rng(90 + dim)
    pat = rng.choice([-1.0, 1.0], size=(1, heads, dim)).astype(np.float32)
    qsign = rng.choice([-1.0, 1.0], size=(lq, 1, 1)).astype(np.float32)
    q = qsign * pat
    k = np.where(np.arange(n) % 2 == 0, 1.0, -1.0).astype(np.float32)[:, None, None] * pat
    v = randn_bf16((n, heads, dim), 92)
    views = _slots(torch, dev, k, v, splits)
    out, qv = segment_attention(
        torch, to_dev(q, dev), views, scale=dim ** -0.5, backend="i8qk", return_quant=True
    )
    torch.cuda.synchronize()
    assert np.all(np.abs(qv["q_i8"].cpu().numpy()[:, :lq].astype(np.int32)) == 127)
    for i, s in enumerate(splits):
        assert np.all(np.abs(qv["k_i8"][i].cpu().numpy()[:, :s].astype(np.int32)) == 127)
    got = bf16.from_torch(out)
    assert np.all(np.isfinite(got))
    ksegs = np.split(k, np.cumsum(splits)[:-1])
    vsegs = np.split(v, np.cumsum(splits)[:-1])
    want_q, _ = oatt.i8qk_attention(q, ksegs, vsegs, dim ** -0.5)
    mx, mean = err_stats(got, want_q)
    assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (mx, mean)
    # the keys of the other sign carry exp2(-2 * 127^2 * D * scale^2 * log2 e) of the weight: none at bf16
    even = v[0::2].astype(np.float64).mean(axis=0)
    odd = v[1::2].astype(np.float64).mean(axis=0)
    exact = np.where(qsign > 0, even[None], odd[None])
    assert oatt.cosine(got, exact) >= 0.9999
    mx, _ = err_stats(got, exact)
    assert mx <= BF16_MAX_ABS, mx


def test_gemm_beyond_32bit_row_offsets(torch_mod, dev):
    # a [m, k] activation of 4.3 GB: rows 524,288 and later start past 2^32 bytes,
    # so the GEMM takes the kernel with 64-bit row addressing; sampled rows on
    # both sides of the boundary are bit-exact (accumulators and epilogue)
    torch = torch_mod
    from taomate_hd_amd import quant

    m, n, k = 524288 + 64, 40, 8192
    g = torch.Generator(device=dev).manual_seed(9)
    ad = torch.randint(-128, 128, (m, k), dtype=torch.int8, device=dev, generator=g)
    wd = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
    sa = torch.rand((m, 1), device=dev, generator=g) * 0.05 + 1e-3
    sb = torch.rand((1, n), device=dev, generator=g) * 0.01 + 1e-4
    acc = quant.int8_mm_i32(ad, wd.t())
    out = quant.cutlass_scaled_mm(ad, wd.t(), sa, sb, torch.bfloat16)
    torch.cuda.synchronize()
    rows = torch.tensor(list(range(0, 16)) + list(range(524288 - 16, m)), device=dev)
    a = ad.index_select(0, rows).cpu().numpy()
    w = wd.cpu().numpy()
    want = oq.int_gemm(a, w)
    assert np.array_equal(acc.index_select(0, rows).cpu().numpy(), want)
    got = bf16.from_torch(out.index_select(0, rows))
    assert np.array_equal(got, oq.scaled_mm_epilogue(want, sa.index_select(0, rows).cpu().numpy().ravel(),
                                                      sb.cpu().numpy().ravel(), None))
    del ad, acc, out
    torch.cuda.empty_cache()


@pytest.mark.parametrize("backend", ["bf16", "i8qk"])
@pytest.mark.parametrize(
    "heads,dim,lq,splits",
    [
        (40, 128, 1792, [1000, 1560]),  # 280 (head, query-tile) items: a full round of 256 CUs plus 24
        (5, 64, 600, [64, 900, 3]),  # 15 items on 256 CUs: every item split, ranges cross segments
    ],
)
def test_split_last_round_matches_whole_items(torch_mod, dev, backend, heads, dim, lq, splits):
    """Items of a partial last round run as key ranges merged by log2-sum-exp;
    the result matches the unsplit run (and, for BF16, the fp64 oracle on the
    heads that were split)."""
    torch = torch_mod
    from taomate_hd_amd import segment_attention

    n = sum(splits)
    q = randn_bf16((lq, heads, dim), 40)
    k = randn_bf16((n, heads, dim), 41, offset=key_offset(heads, dim, 43))
    v = randn_bf16((n, heads, dim), 42)
    views = _slots(torch, dev, k, v, splits)
    qd = to_dev(q, dev)
    whole = segment_attention(torch, qd, views, scale=dim ** -0.5, backend=backend, split=False)
    split = segment_attention(torch, qd, views, scale=dim ** -0.5, backend=backend, split=True)
    torch.cuda.synchronize()
    a, b = bf16.from_torch(whole), bf16.from_torch(split)
    # same scores and probabilities, other summation order: at most a few bf16 ulps apart
    mx, mean = err_stats(b, a)
    assert mx <= 1.6e-2 and mean <= 2e-4, (mx, mean)
    if backend == "bf16":
        hs = list(range(max(0, heads - 4), heads))  # the last items are the split ones
        want = oatt.attention_fp64(q[:, hs], k[:, hs], v[:, hs], dim ** -0.5)
        mx, mean = err_stats(b[:, hs], want)
        assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (mx, mean)


def test_token_quant_bit_exact(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import quant

    x = randn_bf16((77, 5120), 40)
    x[:, 7] *= 20.0
    x = bf16.round_f32(x)
    x[3] = 0.0  # a zero row
    x[5, :] = 0.0
    x[5, 100] = -2.5
    q, s, azp = quant.scaled_int8_quant(to_dev(x, dev))
    torch.cuda.synchronize()
    assert azp is None
    wq, ws = oq.token_quant(x)
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(s.cpu().numpy().reshape(-1), ws)
    # rows where x * (127 / amax) and x / (amax / 127) round apart (63 vs 64):
    # the kernel multiplies, as stated
    from tests.test_oracle import FORM_ROWS

    xf = np.zeros((2, 512), np.float32)
    xf[:, :3] = FORM_ROWS
    qf, _, _ = quant.scaled_int8_quant(to_dev(xf, dev))
    assert qf.cpu().numpy()[:, :3].tolist() == [[127, 63, -63], [127, 64, -64]]
    # odd widths use the streaming variant
    x2 = randn_bf16((9, 8 * 64 * 17), 41)
    q2, s2, _ = quant.scaled_int8_quant(to_dev(x2, dev))
    wq2, ws2 = oq.token_quant(x2)
    assert np.array_equal(q2.cpu().numpy(), wq2)
    assert np.array_equal(s2.cpu().numpy().reshape(-1), ws2)


def test_weight_quant_bit_exact(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import quant

    w = randn_bf16((300, 1024), 50, std=0.02)
    w[7] = 0.0
    q, s = quant.quantize_weight(to_dev(w, dev))
    torch.cuda.synchronize()
    wq, wsc = oq.weight_quant(w)
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(s.cpu().numpy().reshape(-1), wsc)
    # the divide form of the weight quantizer (64 vs 63 where multiplying gives 63 vs 64)
    from tests.test_oracle import FORM_ROWS

    wf = np.zeros((2, 256), np.float32)
    wf[:, :3] = FORM_ROWS
    qf, _ = quant.quantize_weight(to_dev(wf, dev))
    assert qf.cpu().numpy()[:, :3].tolist() == [[127, 64, -64], [127, 63, -63]]


# k = 64 and 192 (odd multiples of 64) run the 8-wave kernel; 128 (one k block:
# the ring's tail alone), 640 (one whole pass of the 5-unit ring), 1024 and
# 5120 the one-wave-per-SIMD kernel
@pytest.mark.parametrize("m,n,k", [(12, 32, 64), (257, 300, 192), (130, 260, 128), (64, 512, 640), (300, 520, 1024),
                                   (513, 256, 5120)])
def test_gemm_accumulators_and_epilogue_bit_exact(torch_mod, dev, m, n, k):
    torch = torch_mod
    from taomate_hd_amd import quant

    rng = np.random.default_rng(m + n + k)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    a[0, :] = -128  # extreme accumulators
    w[0, :] = -127
    ad = torch.from_numpy(a).to(dev)
    wd = torch.from_numpy(w).to(dev)
    acc = quant.int8_mm_i32(ad, wd.t())
    torch.cuda.synchronize()
    want = oq.int_gemm(a, w)
    assert np.array_equal(acc.cpu().numpy(), want)
    sa = rng.random(m, dtype=np.float32) * 0.05 + 1e-3
    sb = rng.random(n, dtype=np.float32) * 0.01 + 1e-4
    bias = randn_bf16((n,), 60, std=0.02)
    out = quant.cutlass_scaled_mm(
        ad, wd.t(), torch.from_numpy(sa).to(dev).view(m, 1), torch.from_numpy(sb).to(dev).view(1, n),
        torch.bfloat16, to_dev(bias, dev),
    )
    torch.cuda.synchronize()
    assert np.array_equal(bf16.from_torch(out), oq.scaled_mm_epilogue(want, sa, sb, bias))
    out2 = quant.cutlass_scaled_mm(
        ad, wd.t(), torch.from_numpy(sa).to(dev).view(m, 1), torch.from_numpy(sb).to(dev).view(1, n)
    )
    torch.cuda.synchronize()
    assert np.array_equal(bf16.from_torch(out2), oq.scaled_mm_epilogue(want, sa, sb, None))


def test_gemm_split_round_equals_unsplit(torch_mod, dev):
    # 8 x 37 = 296 tiles: on 256 CUs one whole round plus a 40-tile round (more
    # than an eighth of the CUs, at most half) that is split along k; the
    # split + merge must equal the unsplit GEMM bit for bit
    torch = torch_mod
    from taomate_hd_amd import _native, quant

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    m, n, k = 8 * 256 - 100, 37 * 256 - 30, 1024
    last = (8 * 37) % cus
    if not (cus < 8 * last and 2 * last <= cus):
        pytest.skip(f"296 tiles leave a last round of {last} on {cus} CUs: not the k-split case")
    rng = np.random.default_rng(5)
    ad = torch.from_numpy(rng.integers(-128, 128, size=(m, k), dtype=np.int8)).to(dev)
    wd = torch.from_numpy(rng.integers(-127, 128, size=(n, k), dtype=np.int8)).to(dev)
    lib = _native.load()
    assert lib.tmhd_gemm_split_workspace_bytes(m, n, k) > 0
    stream = _native.stream_ptr(torch, dev)
    plain = torch.empty((m, n), dtype=torch.int32, device=dev)
    _native.check(lib.tmhd_gemm_i8_i32(_native.ptr(plain), _native.ptr(ad), _native.ptr(wd), m, n, k, k, k, n, stream),
                  "tmhd_gemm_i8_i32")
    split = quant.int8_mm_i32(ad, wd.t())
    torch.cuda.synchronize()
    assert torch.equal(plain, split)
    sa = torch.from_numpy(rng.random(m, dtype=np.float32) * 0.05 + 1e-3).to(dev)
    sb = torch.from_numpy(rng.random(n, dtype=np.float32) * 0.01 + 1e-4).to(dev)
    bias = to_dev(randn_bf16((n,), 61, std=0.02), dev)
    ref = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    _native.check(lib.tmhd_gemm_w8a8(_native.ptr(ref), _native.ptr(ad), _native.ptr(wd), _native.ptr(sa),
                                     _native.ptr(sb), _native.ptr(bias), m, n, k, k, k, n, stream), "tmhd_gemm_w8a8")
    out = quant.cutlass_scaled_mm(ad, wd.t(), sa.view(m, 1), sb.view(1, n), torch.bfloat16, bias)
    torch.cuda.synchronize()
    assert torch.equal(ref.view(torch.int16), out.view(torch.int16))


def test_gemm_sub_tile_last_round(torch_mod, dev):
    # 15 x 18 = 270 tiles: on 256 CUs one whole round plus a 14-tile round (at
    # most an eighth of the CUs), which runs as 64 x 128 sub-tiles over the
    # whole of k; int32 accumulators against an exact float64 product, and the
    # bf16 epilogue against the oracle, bit for bit (k = 384: a 3-block ring)
    torch = torch_mod
    from taomate_hd_amd import quant

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    m, n, k = 15 * 256 - 100, 18 * 256 - 30, 384
    last = (15 * 18) % cus
    if not (0 < 8 * last <= cus):
        pytest.skip(f"270 tiles leave a last round of {last} on {cus} CUs: not the sub-tile case")
    rng = np.random.default_rng(9)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    ad, wd = torch.from_numpy(a).to(dev), torch.from_numpy(w).to(dev)
    acc = quant.int8_mm_i32(ad, wd.t())
    sa = rng.random(m, dtype=np.float32) * 0.05 + 1e-3
    sb = rng.random(n, dtype=np.float32) * 0.01 + 1e-4
    bias = randn_bf16((n,), 62, std=0.02)
    out = quant.cutlass_scaled_mm(ad, wd.t(), torch.from_numpy(sa).to(dev).view(m, 1),
                                  torch.from_numpy(sb).to(dev).view(1, n), torch.bfloat16, to_dev(bias, dev))
    torch.cuda.synchronize()
    want = (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64)  # exact: |sum| < 2^53
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), want)
    got = bf16.from_torch(out)
    exp = oq.scaled_mm_epilogue(want.astype(np.int32), sa, sb, bias)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("backend", ["bf16", "i8qk"])
@pytest.mark.parametrize(
    "H,lq,splits",
    [
        (40, 4836, [1560, 4836, 4836, 4836]),  # 480p stage: Lkv 16,068 (anchor + two history chunks + self)
        (40, 12252, [4032, 12252, 12252, 12252]),  # 768p stage: Lkv 40,788
        # the model's own 768p call on one GPU's 14 heads: 10 x 1,032 video + 2 x 57 audio queries over a
        # 12-latent video sink, two history chunks and the chunk itself (Lkv 43,686; 574 items, split last round)
        (14, 10434, [12384, 10434, 10434, 10434]),
    ],
)
def test_full_size_stage_shapes_on_sampled_rows(torch_mod, dev, backend, H, lq, splits):
    """The stage shapes at full size (head_dim 128): the whole attention
    runs; 64 query rows of 3 heads are checked against the fp64 oracle over
    every key (BF16 gate, or the INT8-QK cosine gate)."""
    torch = torch_mod
    from taomate_hd_amd import KVSlot, segment_attention

    D = 128
    n = sum(splits)
    gen = torch.Generator(device=dev).manual_seed(lq)
    q = torch.randn(lq, H, D, generator=gen, device=dev).to(torch.bfloat16)
    off = 0.5 * torch.randn(H, D, generator=gen, device=dev)
    k = (torch.randn(n, H, D, generator=gen, device=dev) + off).to(torch.bfloat16)
    v = torch.randn(n, H, D, generator=gen, device=dev).to(torch.bfloat16)
    views, row = [], 0
    for c in splits:
        s = KVSlot(torch, heads=H, head_dim=D, capacity=c, device=dev)
        s.pack(k, v, row0=row, count=c)
        views.append(s.view())
        row += c
    out = segment_attention(torch, q, views, scale=D ** -0.5, backend=backend)
    torch.cuda.synchronize()
    rng = np.random.default_rng(lq)
    rows = np.unique(np.concatenate([[0, lq - 1], rng.integers(0, lq, 62)]))
    heads = [0, H // 2 - 3, H - 1]
    qs = bf16.from_torch(q[torch.tensor(rows, device=dev)][:, heads].contiguous())
    ks = bf16.from_torch(k[:, heads].contiguous())
    vs = bf16.from_torch(v[:, heads].contiguous())
    got = bf16.from_torch(out[torch.tensor(rows, device=dev)][:, heads].contiguous())
    want = oatt.attention_fp64(qs, ks, vs, D ** -0.5)
    assert np.all(np.isfinite(got))
    if backend == "bf16":
        mx, mean = err_stats(got, want)
        assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (mx, mean)
    else:
        assert oatt.cosine(got, want) >= I8_COSINE


def test_row_lists_checked_before_any_launch(torch_mod, dev):
    """Row lists are device tensors with in-range entries; anything else is
    refused before a kernel could read through it."""
    torch = torch_mod
    from taomate_hd_amd import KVSlot, segment_attention

    H, D, T = 2, 128, 40
    k = randn_bf16((T, H, D), 1)
    kd = to_dev(k, dev)
    q = to_dev(randn_bf16((T, H, D), 2), dev)
    slot = KVSlot(torch, heads=H, head_dim=D, capacity=64, device=dev)
    with pytest.raises(ValueError, match="on the GPU"):
        slot.pack(kd, kd, rows=torch.tensor([0, 1, 2], dtype=torch.int32))
    with pytest.raises(ValueError, match=r"in \[0, 40\)"):
        slot.pack(kd, kd, rows=torch.tensor([0, 40], dtype=torch.int32, device=dev))
    slot.pack(kd, kd, rows=torch.tensor([3, 39, 0], dtype=torch.int32, device=dev))
    view = [slot.view()]
    with pytest.raises(ValueError, match="on the GPU"):
        segment_attention(torch, q, view, scale=0.1, q_rows=torch.tensor([1, 2], dtype=torch.int32))
    with pytest.raises(ValueError, match=r"in \[0, 40\)"):
        segment_attention(torch, q, view, scale=0.1, q_rows=torch.tensor([-1, 2], dtype=torch.int32, device=dev))
    out = torch.zeros((5, H, D), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match=r"in \[0, 5\)"):
        segment_attention(torch, q, view, scale=0.1, q_rows=torch.tensor([1, 2], dtype=torch.int32, device=dev),
                          out=out, o_rows=torch.tensor([4, 5], dtype=torch.int32, device=dev))
    res = segment_attention(torch, q, view, scale=0.1, q_rows=torch.tensor([7, 2], dtype=torch.int32, device=dev),
                            out=out, o_rows=torch.tensor([4, 0], dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert res is out and bool(torch.isfinite(out).all())


def test_i8qk_key_sum_memo_hits_and_invalidation(torch_mod, dev):
    """The smooth-K key sums memoised per slot view give the same quantised
    operands and output as summing afresh; re-packing a slot drops its memo,
    so the next call sees the new keys (compared with a fresh slot)."""
    torch = torch_mod
    from taomate_hd_amd import segment_attention

    heads, dim, lq, splits = 3, 128, 300, [400, 333]
    q = to_dev(randn_bf16((lq, heads, dim), 60), dev)
    k = randn_bf16((sum(splits), heads, dim), 61, offset=key_offset(heads, dim, 62))
    v = randn_bf16((sum(splits), heads, dim), 63)
    views = _slots(torch, dev, k, v, splits)

    def run(vs):
        out, qv = segment_attention(torch, q, vs, scale=dim ** -0.5, backend="i8qk", return_quant=True)
        torch.cuda.synchronize()
        return out.clone(), qv["k_mean"].clone(), [t.clone() for t in qv["k_i8"]]

    first = run(views)
    assert all(len(vw.slot.key_sums) == 1 for vw in views)
    second = run(views)  # memo hits
    assert torch.equal(first[0].view(torch.int16), second[0].view(torch.int16))
    assert torch.equal(first[1].view(torch.int16), second[1].view(torch.int16))
    assert all(torch.equal(a, b) for a, b in zip(first[2], second[2]))
    # new keys in the second slot: its memo is dropped by the pack
    k2 = randn_bf16((splits[1], heads, dim), 64, offset=key_offset(heads, dim, 65))
    views[1].slot.pack(to_dev(k2, dev), to_dev(v[splits[0]:], dev))
    assert not views[1].slot.key_sums
    third = run(views)
    fresh = run(_slots(torch, dev, np.concatenate([k[: splits[0]], k2]), v, splits))
    assert torch.equal(third[1].view(torch.int16), fresh[1].view(torch.int16))
    assert not torch.equal(third[1].view(torch.int16), first[1].view(torch.int16))
    assert torch.equal(third[0].view(torch.int16), fresh[0].view(torch.int16))


@pytest.mark.parametrize("backend", ["sdpa", "sage_attn"])
def test_plumbing_config_exact_inputs_through_the_hook(torch_mod, dev, backend):
    """The CPU-runnable plumbing configuration exactly: batch 1, 8 heads, head_dim
    64, 256 chunk queries over 1,024 keys (768 cached history + 256 self), no
    mask, Q / K / V ~ N(0, 1) fp32 then cast to bf16 with torch generators
    seeded 0 (Q), 1 (K) and 2 (V), no key offset; one noisy hook call over a
    cache holding the 768 history keys, against torch SDPA on the CPU (the
    reference's serial backend) and the fp64 oracle."""
    torch = torch_mod
    from oracle.attention import sdpa_cpu
    from taomate_hd_amd import HeadMajorRingKVCache, HookMode, KVContract, StreamingAttentionHook

    H, D, LQ, HIST = 8, 64, 256, 768

    def draw(seed, rows):
        return torch.randn(rows, H, D, generator=torch.Generator().manual_seed(seed), dtype=torch.float32)

    q = draw(0, LQ).to(torch.bfloat16)
    k = draw(1, HIST + LQ).to(torch.bfloat16)
    v = draw(2, HIST + LQ).to(torch.bfloat16)
    layer = "blocks.0.attn"
    cache = HeadMajorRingKVCache(KVContract(layer_names=(layer,), local_heads=H, head_dim=D))
    cache.begin_clean_commit(0)
    tags = torch.tensor([2] * 16 + [0] * (HIST - 16), device=dev)
    cache.stage(layer, k[:HIST].to(dev), v[:HIST].to(dev), tags, torch.ones(HIST, dtype=torch.bool, device=dev))
    cache.commit()
    hook = StreamingAttentionHook(cache, attention_backend=backend)
    hook.activate(mode=HookMode.NOISY, block_index=1)

    class Attn:
        softmax_scale = D ** -0.5

    out = hook(attention=Attn(), layer_name=layer, query=q.to(dev), key=k[HIST:].to(dev), value=v[HIST:].to(dev),
               token_tags=torch.tensor([2] * 16 + [0] * (LQ - 16), device=dev),
               commit_mask=torch.ones(LQ, dtype=torch.bool, device=dev), cu_seqlens=None,
               cu_seqlens_host=(0, LQ), max_seqlen=LQ)
    torch.cuda.synchronize()
    got = bf16.from_torch(out)
    ref = sdpa_cpu(q.float(), k.float(), v.float(), D ** -0.5).numpy()
    exact = oatt.attention_fp64(bf16.from_torch(q), bf16.from_torch(k), bf16.from_torch(v), D ** -0.5)
    if backend == "sdpa":
        for want in (ref, exact):
            mx, mean = err_stats(got, want)
            assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (mx, mean)
    else:
        assert oatt.cosine(got, ref) >= I8_COSINE and oatt.cosine(got, exact) >= I8_COSINE


@pytest.mark.parametrize("backend", ["bf16", "i8qk"])
def test_repeated_calls_bit_identical(torch_mod, dev, backend):
    """Run-to-run determinism at the 768p stage shape (the split last round,
    its merge and, for INT8-QK, the smooth-K key sums and quantization
    included): five calls on the same inputs give the same bits."""
    torch = torch_mod
    from taomate_hd_amd import KVSlot, segment_attention

    H, D, lq, splits = 40, 128, 12252, [4032, 12252, 12252, 12252]
    n = sum(splits)
    gen = torch.Generator(device=dev).manual_seed(11)
    q = torch.randn(lq, H, D, generator=gen, device=dev).to(torch.bfloat16)
    k = (torch.randn(n, H, D, generator=gen, device=dev) + 0.5 * torch.randn(H, D, generator=gen, device=dev)).to(
        torch.bfloat16)
    v = torch.randn(n, H, D, generator=gen, device=dev).to(torch.bfloat16)
    views, row = [], 0
    for c in splits:
        s = KVSlot(torch, heads=H, head_dim=D, capacity=c, device=dev)
        s.pack(k, v, row0=row, count=c)
        views.append(s.view())
        row += c
    outs = [segment_attention(torch, q, views, scale=D ** -0.5, backend=backend) for _ in range(5)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))


@pytest.mark.parametrize("backend", ["bf16", "i8qk"])
def test_more_segments_than_one_launch_takes(torch_mod, dev, backend):
    """21 ragged segments, every third a view at a nonzero tile row of its
    slot: more than one launch takes, so the oldest are merged into one
    temporary slot; the call still matches attention over all the keys."""
    torch = torch_mod
    from taomate_hd_amd import KVSlot, SlotView, segment_attention
    from taomate_hd_amd._native import MAX_SEGMENTS

    heads, dim, lq = 3, 128, 200
    sizes = [1, 17, 64, 65, 130, 3, 700, 40, 2, 96, 33, 64, 5, 128, 90, 7, 11, 300, 19, 64, 23]
    assert len(sizes) > MAX_SEGMENTS
    n = sum(sizes)
    q = randn_bf16((lq, heads, dim), 301)
    k = randn_bf16((n, heads, dim), 302, offset=key_offset(heads, dim, 303))
    v = randn_bf16((n, heads, dim), 304)
    kd, vd = to_dev(k, dev), to_dev(v, dev)
    views, row = [], 0
    for i, c in enumerate(sizes):
        dst = 64 * (1 + i % 2) if i % 3 == 1 else 0
        s = KVSlot(torch, heads=heads, head_dim=dim, capacity=dst + c, device=dev)
        s.pack(kd, vd, row0=row, count=c, dst=dst)
        views.append(SlotView(s, c, dst))
        row += c
    got = bf16.from_torch(segment_attention(torch, to_dev(q, dev), views, scale=dim ** -0.5, backend=backend))
    torch.cuda.synchronize()
    want = oatt.attention_fp64(q, k, v, dim ** -0.5)
    if backend == "bf16":
        mx, mean = err_stats(got, want)
        assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (mx, mean)
    else:
        assert oatt.cosine(got, want) >= I8_COSINE
