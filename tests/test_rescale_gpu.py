"""The attention kernel's lazy rescale on peaky logits, both backends.

The kernel keeps a running reference per query row and only moves it (and
rescales the output accumulators and the row sum) when a later score exceeds
it by more than 8 in log2 units.  N(0, 1) inputs never get there, so these
cases are built to: Q scaled x4 / x8, a dominant key planted in the last tile
of the last segment, a low first tile followed by a high one, and a first
segment shorter than one 32-key sub-tile.  A host check confirms that the
rows do move their reference; the outputs are checked against the fp64 oracle
(BF16 gate, or the INT8-QK cosine gate and the BF16 gate against exact
attention of the quantized operands), for whole items and for items split
into key ranges, at the plumbing size and on sampled rows of the 768p shape.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as oatt
from oracle import bf16
from tests.helpers import PEAKY_KINDS, err_stats, peaky_case, rescale_rows_fraction, to_dev

pytestmark = pytest.mark.gpu

BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 1e-3
I8_COSINE = 0.999
# least fraction of (row, head) pairs that must move their reference, per case
# (Q x4 over 1,024 keys moves a third of the rows; the other cases most rows)
MIN_RESCALED = {"q4": 0.3, "q8": 0.7, "planted": 0.6, "low_first": 0.9, "partial_first": 0.7}


def _views(torch, dev, k, v, splits):
    from taomate_hd_amd import KVSlot

    views, off = [], 0
    kd, vd = to_dev(k, dev), to_dev(v, dev)
    for n in splits:
        slot = KVSlot(torch, heads=k.shape[1], head_dim=k.shape[2], capacity=n, device=dev)
        slot.pack(kd, vd, row0=off, count=n)
        views.append(slot.view())
        off += n
    return views


def _check_bf16(got, want):
    mx, mean = err_stats(got, want)
    assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (mx, mean)


CASES = [
    # heads, dim, lq, segment token counts (partial_first uses a first segment of 5)
    (8, 64, 256, [768, 256]),
    (2, 128, 300, [100, 600, 129]),
]


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("backend", ["bf16", "i8qk"])
@pytest.mark.parametrize("kind", PEAKY_KINDS)
@pytest.mark.parametrize("heads,dim,lq,splits", CASES)
def test_peaky_logits_match_oracle(torch_mod, dev, heads, dim, lq, splits, kind, backend, split):
    torch = torch_mod
    from taomate_hd_amd import segment_attention

    if kind == "partial_first":
        splits = [5, splits[0] - 5, *splits[1:]]
    q, k, v = peaky_case(kind, heads, dim, lq, splits, seed=70 + dim)
    scale = dim ** -0.5
    frac = rescale_rows_fraction(q, k, scale, first=min(32, splits[0]))
    assert frac >= MIN_RESCALED[kind], frac  # the rows do take the rescale branch
    views = _views(torch, dev, k, v, splits)
    out = segment_attention(torch, to_dev(q, dev), views, scale=scale, backend=backend, split=split)
    torch.cuda.synchronize()
    got = bf16.from_torch(out)
    assert np.all(np.isfinite(got))
    want = oatt.attention_fp64(q, k, v, scale)
    if backend == "bf16":
        _check_bf16(got, want)
        return
    assert oatt.cosine(got, want) >= I8_COSINE
    ksegs = np.split(k, np.cumsum(splits)[:-1])
    vsegs = np.split(v, np.cumsum(splits)[:-1])
    want_q, _ = oatt.i8qk_attention(q, ksegs, vsegs, scale)
    _check_bf16(got, want_q)


def _quantized_logits(qv, rows, heads, splits, scale):
    """Exact logits of the quantized operands for the sampled rows / heads."""
    q8 = qv["q_i8"].cpu().numpy()
    qs = qv["q_scale"].cpu().numpy()
    out = []
    for h in heads:
        parts = []
        for i, n in enumerate(splits):
            k8 = qv["k_i8"][i][h, :n].cpu().numpy().astype(np.float64)
            ks = qv["k_scale"][i][h].cpu().numpy().astype(np.float64)
            acc = q8[h, rows].astype(np.float64) @ k8.T
            parts.append(acc * qs[h, rows // 128][:, None] * ks[np.arange(n) // 128][None, :])
        out.append(np.concatenate(parts, axis=1) * scale)
    return out


@pytest.mark.parametrize("backend", ["bf16", "i8qk"])
def test_peaky_logits_768p_sampled_rows(torch_mod, dev, backend):
    """The 768p stage shape (H 40, D 128, Lq 12,252 over 40,788 keys in four
    segments) with Q x4: the whole attention runs (its last round split into
    key ranges); 64 query rows of 3 heads, one of them in the split items,
    are checked over every key."""
    torch = torch_mod
    from taomate_hd_amd import KVSlot, segment_attention

    H, D, lq, splits = 40, 128, 12252, [4032, 12252, 12252, 12252]
    n = sum(splits)
    gen = torch.Generator(device=dev).manual_seed(4)
    q = (4.0 * torch.randn(lq, H, D, generator=gen, device=dev)).to(torch.bfloat16)
    off = 0.5 * torch.randn(H, D, generator=gen, device=dev)
    k = (torch.randn(n, H, D, generator=gen, device=dev) + off).to(torch.bfloat16)
    v = (0.25 * torch.randn(n, H, D, generator=gen, device=dev)).to(torch.bfloat16)
    views, row = [], 0
    for c in splits:
        s = KVSlot(torch, heads=H, head_dim=D, capacity=c, device=dev)
        s.pack(k, v, row0=row, count=c)
        views.append(s.view())
        row += c
    res = segment_attention(torch, q, views, scale=D ** -0.5, backend=backend, return_quant=backend == "i8qk")
    out, qv = res if backend == "i8qk" else (res, None)
    torch.cuda.synchronize()
    rng = np.random.default_rng(12)
    rows = np.unique(np.concatenate([[0, lq - 1], rng.integers(0, lq, 62)]))
    heads = [0, 17, 39]  # head 39's query tiles are in the split last round
    rows_d = torch.tensor(rows, device=dev)
    qs = bf16.from_torch(q[rows_d][:, heads].contiguous())
    ks = bf16.from_torch(k[:, heads].contiguous())
    vs = bf16.from_torch(v[:, heads].contiguous())
    frac = rescale_rows_fraction(qs, ks, D ** -0.5)
    assert frac >= 0.6, frac
    got = bf16.from_torch(out[rows_d][:, heads].contiguous())
    assert np.all(np.isfinite(got))
    want = oatt.attention_fp64(qs, ks, vs, D ** -0.5)
    if backend == "bf16":
        _check_bf16(got, want)
        return
    assert oatt.cosine(got, want) >= I8_COSINE
    logits = _quantized_logits(qv, rows, heads, splits, D ** -0.5)
    want_q = np.empty_like(want)
    for j, s in enumerate(logits):
        p = np.exp(s - s.max(axis=1, keepdims=True))
        want_q[:, j] = (p / p.sum(axis=1, keepdims=True)) @ vs[:, j].astype(np.float64)
    _check_bf16(got, want_q)
