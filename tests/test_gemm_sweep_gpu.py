"""Seeded random sweep of the scaled INT8 GEMM against the oracle, bit for bit:
random m, n (odd widths take the scalar scale / bias loads and the per-element
tail stores), k (odd multiples of 64 run the 8-wave kernel, multiples of 128
the one-wave-per-SIMD kernel, split along k when its tiles leave the CUs
idle), padded row strides of both operands and of the output (a row stride
that is not a multiple of 8 takes the epilogue without LDS staging), with and
without bias.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import bf16
from oracle import quant as oq
from tests.helpers import randn_bf16, to_dev

pytestmark = pytest.mark.gpu

# a wider sweep: TMHD_SWEEP_CASES=<cases> TMHD_SWEEP_SEED=<another base>
N_CASES = int(os.environ.get("TMHD_SWEEP_CASES", "24"))
SEED0 = int(os.environ.get("TMHD_SWEEP_SEED", "777"))


def _case(c: int) -> dict:
    rng = np.random.default_rng(SEED0 + c)
    return dict(m=int(rng.integers(1, 400)), n=int(rng.integers(1, 520)), k=64 * int(rng.integers(1, 21)),
                apad=16 * int(rng.integers(0, 3)), bpad=16 * int(rng.integers(0, 3)), opad=int(rng.integers(0, 10)),
                bias=bool(rng.integers(0, 2)), seed=5000 + c + 1000 * (SEED0 - 777))


CASES = [_case(c) for c in range(N_CASES)]


@pytest.mark.parametrize("case", CASES, ids=[f"m{c['m']}-n{c['n']}-k{c['k']}-ldo+{c['opad']}{'-bias' if c['bias'] else ''}"
                                            for c in CASES])
def test_random_gemm_case_bit_exact(torch_mod, dev, case):
    torch = torch_mod
    from taomate_hd_amd import quant

    m, n, k = case["m"], case["n"], case["k"]
    rng = np.random.default_rng(case["seed"])
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    abuf = np.zeros((m, k + case["apad"]), np.int8)
    abuf[:, :k] = a
    wbuf = np.zeros((n, k + case["bpad"]), np.int8)
    wbuf[:, :k] = w
    ad = torch.from_numpy(abuf).to(dev)[:, :k]
    wd = torch.from_numpy(wbuf).to(dev)[:, :k]
    want_acc = oq.int_gemm(a, w)
    acc = quant.int8_mm_i32(ad, wd.t())
    torch.cuda.synchronize()
    assert np.array_equal(acc.cpu().numpy(), want_acc)

    sa = rng.random(m, dtype=np.float32) * 0.05 + 1e-3
    sb = rng.random(n, dtype=np.float32) * 0.01 + 1e-4
    bias = randn_bf16((n,), case["seed"] + 1, std=0.02) if case["bias"] else None
    obuf = torch.full((m, n + case["opad"]), 7.0, dtype=torch.bfloat16, device=dev)
    out = obuf[:, :n]
    quant.cutlass_scaled_mm_out(out, ad, wd.t(), torch.from_numpy(sa).to(dev).view(m, 1),
                                torch.from_numpy(sb).to(dev).view(1, n), None if bias is None else to_dev(bias, dev))
    torch.cuda.synchronize()
    got = bf16.from_torch(obuf)
    assert np.array_equal(got[:, :n], oq.scaled_mm_epilogue(want_acc, sa, sb, bias))
    assert np.all(got[:, n:] == 7.0)  # the row padding is not written
