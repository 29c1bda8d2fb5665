"""Dense attention over the documents of a packed sequence (packed_sdpa, the
drop-in for model/layers.py:202-255): the BF16 kernel against the fp64
oracle, document by document."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as oatt
from oracle import bf16
from tests.helpers import err_stats, randn_bf16, to_dev

pytestmark = pytest.mark.gpu

BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 1e-3


@pytest.mark.parametrize("lengths", [(0, 37, 130, 0, 64, 5), (200,), (1, 1, 63, 65)])
def test_packed_sdpa_matches_per_document_attention(torch_mod, dev, lengths):
    torch = torch_mod
    from taomate_hd_amd import packed_sdpa

    H, D = 3, 128
    T = sum(lengths)
    qkv = randn_bf16((T, 3, H, D), seed=len(lengths) + T)
    merged = to_dev(qkv.reshape(T, 3 * H * D), dev)
    q, k, v = (merged[:, i * H * D : (i + 1) * H * D].view(T, H, D) for i in range(3))  # strided views
    bounds = tuple(int(b) for b in np.concatenate([[0], np.cumsum(lengths)]))
    scale = D ** -0.5
    out = packed_sdpa(q, k, v, cu_seqlens=torch.tensor(bounds, dtype=torch.int32, device=dev), cu_seqlens_host=None,
                      max_seqlen=max(lengths), scale=scale)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (T, H, D) and out.is_contiguous()
    got = bf16.from_torch(out)
    for start, stop in zip(bounds[:-1], bounds[1:]):
        if start == stop:
            continue
        want = oatt.attention_fp64(qkv[start:stop, 0], qkv[start:stop, 1], qkv[start:stop, 2], scale)
        mx, mean = err_stats(got[start:stop], want)
        assert mx <= BF16_MAX_ABS and mean <= BF16_MEAN_ABS, (start, stop, mx, mean)
    # the same call with host boundaries gives the same bits (pooled slot reused)
    again = packed_sdpa(q, k, v, cu_seqlens=None, cu_seqlens_host=bounds, max_seqlen=max(lengths), scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(again, out)


def test_packed_sdpa_rejects_bad_boundaries(torch_mod, dev):
    torch = torch_mod
    from taomate_hd_amd import packed_sdpa

    q = to_dev(randn_bf16((10, 2, 128), seed=1), dev)
    with pytest.raises(ValueError, match="cumulative lengths are invalid"):
        packed_sdpa(q, q, q, cu_seqlens=None, cu_seqlens_host=(0, 4, 9), max_seqlen=5, scale=0.1)
    with pytest.raises(ValueError, match="cumulative lengths are invalid"):
        packed_sdpa(q, q, q, cu_seqlens=None, cu_seqlens_host=(0, 4, 10), max_seqlen=4, scale=0.1)
    with pytest.raises(ValueError, match="no live segment"):
        packed_sdpa(q[:0], q[:0], q[:0], cu_seqlens=None, cu_seqlens_host=(0, 0), max_seqlen=0, scale=0.1)
