"""Decode-shaped forwards (M <= 64) with one large outlier per activation row,
in the fp32 math mode: max relative error 1e-5 against float64 products of
the oracle's dequantized weights, over the whole output and per row."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, rel_err, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits,G", [(4, 128), (8, 64)])
@pytest.mark.parametrize("M", [1, 7, 16, 33, 64])
@pytest.mark.parametrize("scale", [1e2, 1e4])
def test_outlier_per_row(gpu, dgm, orc, bits, G, M, scale):
    import torch
    N, K = 256, 4096
    rng = np.random.default_rng(M * 13 + int(np.log10(scale)) + bits)
    x = rng.standard_normal((M, K)).astype(np.float32)
    cols = rng.integers(0, K, size=M)
    x[np.arange(M), cols] *= np.float32(scale)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q = torch.zeros(N * K // (2 if bits == 4 else 1), dtype=torch.uint8 if bits == 4 else torch.int8, device="cuda")
    s = torch.zeros(N * (K // G), device="cuda")
    y = torch.full((M * N,), float("nan"), device="cuda")
    gpu.begin()
    gpu.quantize(to_dev(w), q, s, N, K, bits, G)
    gpu.gemmNT(bits, None, q, s, to_dev(x.ravel()), None, y, M, N, K, G)
    gpu.end()
    qh = from_dev(q)
    wd = orc.dequant(qh.view(np.int8) if bits == 8 else qh, from_dev(s), N, K, G, bits).reshape(N, K)
    ref = x.astype(np.float64) @ wd.astype(np.float64).T
    got = from_dev(y).reshape(M, N)
    assert rel_err(got, ref) <= 1e-5
    worst = max(rel_err(got[m], ref[m]) for m in range(M))
    assert worst <= 1e-5, worst
