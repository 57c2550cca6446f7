"""GPU parity of the K-sliced decode-shaped forward (gemm_slab.hip): gemm_nt_i4 /
gemm_nt_i8 (metal/kernels.metal:152-209) through dgm_gemmNT, at shapes the
library routes to it (two 128-byte chunks of each W row per slice, at least
64 workgroups of 448 output columns x one slice; M <= 16 in the fp32 mode,
M <= 8 in the reduced mode, the other rows of the table taking the
one-launch kernel).

Bars (max|got - ref| / max|ref|, ref = float64 product of the oracle's
dequantized weights, Check.swift:433-458), per output row:
  * fp32 math mode (the default): <= 1e-5;
  * reduced-precision mode (DGM_MATH_BF16): <= 1e-2.
Rows of very different magnitude and a large outlier per row keep those bars
(each row has its own power of two per slice); a row with a non-finite value
gives NaN and leaves the other rows alone; repeated calls are bitwise equal
(the slices are summed in a fixed order).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, rel_err, to_dev

pytestmark = pytest.mark.gpu

# (bits, G, K, N): 8 or 4 slices, ragged N (not a multiple of 448).
SHAPES = [(4, 128, 4096, 3600), (4, 256, 2048, 7200), (8, 64, 2048, 3600), (8, 128, 1024, 7200)]


def _quantize(gpu, w, N, K, G, bits):
    import torch
    q = torch.zeros(N * K // (2 if bits == 4 else 1), dtype=torch.uint8 if bits == 4 else torch.int8, device="cuda")
    s = torch.zeros(N * (K // G), dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.quantize(to_dev(w), q, s, N, K, bits, G)
    gpu.end()
    return q, s


def _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, math):
    import torch
    y = torch.full((M * N,), float("nan"), device="cuda")
    gpu.set_math(math)
    try:
        gpu.begin()
        gpu.gemmNT(bits, None, q, s, to_dev(x.ravel()), None if bias is None else to_dev(bias), y, M, N, K, G)
        gpu.end()
    finally:
        gpu.set_math(dgm.DGM_MATH_FP32)
    return from_dev(y).reshape(M, N)


def _dequant(orc, q, s, N, K, G, bits):
    qh = from_dev(q)
    return orc.dequant(qh.view(np.int8) if bits == 8 else qh, from_dev(s), N, K, G, bits).reshape(N, K)


@pytest.mark.parametrize("bits,G,K,N", SHAPES)
@pytest.mark.parametrize("M", [2, 4, 5, 9, 16])
def test_slab_parity(gpu, dgm, orc, bits, G, K, N, M):
    rng = np.random.default_rng(M * 101 + K + N + bits)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0] *= np.float32(1e-3)                        # a row far smaller than the others
    x[1, rng.integers(0, K)] *= np.float32(1e4)     # an outlier
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if M % 2 else None
    q, s = _quantize(gpu, w, N, K, G, bits)
    ref = x.astype(np.float64) @ _dequant(orc, q, s, N, K, G, bits).astype(np.float64).T
    if bias is not None:
        ref = ref + bias.astype(np.float64)
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_FP32)
    worst = max(rel_err(y[m], ref[m]) for m in range(M))
    assert worst <= 1e-5, worst
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_BF16)
    worst = max(rel_err(y[m], ref[m]) for m in range(M))
    assert worst <= 1e-2, worst


@pytest.mark.parametrize("bits,G,K,N,M", [(4, 128, 8192, 3584, 1), (4, 128, 8192, 3584, 3), (4, 512, 4096, 3585, 7),
                                          (8, 256, 4096, 4000, 12), (8, 64, 512, 14337, 16)])
def test_slab_more_shapes(gpu, dgm, orc, bits, G, K, N, M):
    """M = 1 and 3 at K = 8192 (more chunks than the streaming kernel takes),
    N one row past a multiple of 448, groups spanning a whole slice (G = 512)
    or half of one (int8 G = 256), two slices at N = 14337."""
    rng = np.random.default_rng(M * 7 + K + N + bits)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    q, s = _quantize(gpu, w, N, K, G, bits)
    ref = x.astype(np.float64) @ _dequant(orc, q, s, N, K, G, bits).astype(np.float64).T + bias.astype(np.float64)
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_FP32)
    worst = max(rel_err(y[m], ref[m]) for m in range(M))
    assert worst <= 1e-5, worst
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_BF16)
    worst = max(rel_err(y[m], ref[m]) for m in range(M))
    assert worst <= 1e-2, worst


def test_slab_extreme_rows_and_non_finite(gpu, dgm, orc):
    bits, G, K, N, M = 4, 128, 4096, 3600, 8
    rng = np.random.default_rng(11)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[1] *= np.float32(1e-20)
    x[2] *= np.float32(1e20)
    x[3] = 0.0
    x[5, 3000] = np.inf          # slice 5 of row 5
    x[6, 10] = np.nan            # slice 0 of row 6
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q, s = _quantize(gpu, w, N, K, G, bits)
    ref = x.astype(np.float64) @ _dequant(orc, q, s, N, K, G, bits).astype(np.float64).T
    for math, bar in ((dgm.DGM_MATH_FP32, 1e-5), (dgm.DGM_MATH_BF16, 1e-2)):
        y = _forward(gpu, dgm, bits, q, s, x, None, M, N, K, G, math)
        for m in (0, 1, 2, 4, 7):
            assert rel_err(y[m], ref[m]) <= bar, (math, m)
        assert np.all(y[3] == 0.0)
        assert np.all(np.isnan(y[5])) and np.all(np.isnan(y[6]))


def test_slab_repeatable(gpu, dgm, orc):
    import torch
    bits, G, K, N, M = 4, 128, 4096, 14336, 16
    rng = np.random.default_rng(12)
    x = to_dev(rng.standard_normal(M * K).astype(np.float32))
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q, s = _quantize(gpu, w, N, K, G, bits)
    for math in (dgm.DGM_MATH_FP32, dgm.DGM_MATH_BF16):
        gpu.set_math(math)
        try:
            ys = []
            for _ in range(3):
                y = torch.full((M * N,), float("nan"), device="cuda")
                gpu.begin()
                gpu.gemmNT(bits, None, q, s, x, None, y, M, N, K, G)
                gpu.end()
                ys.append(from_dev(y))
        finally:
            gpu.set_math(dgm.DGM_MATH_FP32)
        assert np.all(np.isfinite(ys[0]))
        assert np.array_equal(ys[0].view(np.uint32), ys[1].view(np.uint32))
        assert np.array_equal(ys[0].view(np.uint32), ys[2].view(np.uint32))
