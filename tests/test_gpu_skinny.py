"""GPU parity of the decode-shaped (M <= 64) quantized forward: gemm_nt_i4 /
gemm_nt_i8 (metal/kernels.metal:152-209) through dgm_gemmNT, whichever kernel
the library routes the shape to: the streaming int8-MFMA kernel (a few rows
whose activation pieces fit LDS, gemm_stream.hip), the K-sliced int8-MFMA
kernel (up to 16 rows of weights large enough to split K over the CUs,
gemm_slab.hip), the int8-MFMA skinny kernel (other shapes of up to 3 rows, and shapes outside the decode kernels'
domain, gemm_skinny.hip), or the f16 / bf16 decode kernels (4 <= M <= 64,
gemm_decode.hip).

Bars (max|got - ref| / max|ref|, ref = float64 product of the oracle's
dequantized weights, Check.swift:433-458):
  * fp32 math mode (the default): <= 1e-5;
  * reduced-precision mode (DGM_MATH_BF16): <= 1e-2.
Every shape here has G % 128 == 0 (int4) or G % 64 == 0 (int8) and M <= 64.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, rel_err, to_dev

pytestmark = pytest.mark.gpu


def _quantize(gpu, wd, N, K, G, bits):
    import torch
    q = torch.zeros(N * K // (2 if bits == 4 else 1), dtype=torch.uint8 if bits == 4 else torch.int8, device="cuda")
    s = torch.zeros(N * (K // G), dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.quantize(wd, q, s, N, K, bits, G)
    gpu.end()
    return q, s


def _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, math):
    import torch
    y = torch.full((M * N,), float("nan"), device="cuda")
    gpu.set_math(math)
    try:
        gpu.begin()
        gpu.gemmNT(bits, None, q, s, to_dev(x), None if bias is None else to_dev(bias), y, M, N, K, G)
        gpu.end()
    finally:
        gpu.set_math(dgm.DGM_MATH_FP32)
    return from_dev(y)


def _ref(orc, q, s, x, bias, M, N, K, G, bits):
    qh = from_dev(q)
    wd = orc.dequant(qh.view(np.int8) if bits == 8 else qh, from_dev(s), N, K, G, bits)
    y = x.reshape(M, K).astype(np.float64) @ wd.reshape(N, K).astype(np.float64).T
    if bias is not None:
        y = y + bias.astype(np.float64)
    return y.ravel()


@pytest.mark.parametrize("M", [1, 16, 64])
def test_config4_decode_shapes(gpu, dgm, orc, M):
    """c4: X[M,4096] ~ N(0,1), W[14336,4096] ~ N(0,0.02) int4 G=128, seed 1004
    (draw order X, W as in Check.swift:99-112)."""
    N, K, G = 14336, 4096, 128
    rng = orc.RNG(1004)
    x = rng.randn(M * K, 1.0)
    w = rng.randn(N * K, 0.02)
    q, s = _quantize(gpu, to_dev(w), N, K, G, 4)
    ref = _ref(orc, q, s, x, None, M, N, K, G, 4)
    y32 = _forward(gpu, dgm, 4, q, s, x, None, M, N, K, G, dgm.DGM_MATH_FP32)
    assert rel_err(y32, ref) <= 1e-5
    # The Metal kernel order restated on the CPU agrees too.
    if M == 1:
        qh = from_dev(q)
        yk = orc.gemm_nt_q(qh, from_dev(s), x, None, M, N, K, G, 4)
        assert rel_err(y32, yk.astype(np.float64)) <= 1e-5
    ylp = _forward(gpu, dgm, 4, q, s, x, None, M, N, K, G, dgm.DGM_MATH_BF16)
    assert rel_err(ylp, ref) <= 1e-2


@pytest.mark.parametrize("bits,G", [(4, 128), (4, 256), (8, 64), (8, 128)])
@pytest.mark.parametrize("M,N,Kb", [(1, 1, 1), (2, 17, 3), (3, 100, 2), (5, 33, 4), (6, 40, 2),
                                    (7, 257, 5), (16, 31, 8), (17, 48, 2), (33, 70, 3), (64, 129, 4)])
def test_ragged_skinny(gpu, dgm, orc, bits, G, M, N, Kb):
    K = G * Kb
    rng = np.random.default_rng(M * 1000 + N + K + bits)
    x = (rng.standard_normal(M * K) * rng.choice([1e-3, 1.0, 50.0])).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.05).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if M % 2 else None
    q, s = _quantize(gpu, to_dev(w), N, K, G, bits)
    ref = _ref(orc, q, s, x, bias, M, N, K, G, bits)
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_FP32)
    assert rel_err(y, ref) <= 1e-5
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_BF16)
    assert rel_err(y, ref) <= 1e-2


@pytest.mark.parametrize("bits,G,K", [(4, 128, 4096), (4, 256, 2048), (8, 64, 2048), (8, 128, 1536)])
@pytest.mark.parametrize("M", [6, 8, 16, 22, 43, 64])
def test_tiled_decode_many_chunks(gpu, dgm, orc, bits, G, K, M):
    """8 <= P*M <= 192 virtual rows with long K: the tiled decode kernel (fragment-major
    pieces, double-buffered chunks, ragged N); both math modes."""
    N = 300
    rng = np.random.default_rng(M * 31 + K + bits)
    x = rng.standard_normal(M * K).astype(np.float32)
    x[: K] *= np.float32(1e-3)                     # rows of different magnitude
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if M % 2 == 0 else None
    q, s = _quantize(gpu, to_dev(w), N, K, G, bits)
    ref = _ref(orc, q, s, x, bias, M, N, K, G, bits).reshape(M, N)
    # Per row: row 0 is 1e-3 of the others, so a whole-output metric would
    # let its error hide under the larger rows' maximum.
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_FP32).reshape(M, N)
    worst = max(rel_err(y[m], ref[m]) for m in range(M))
    assert worst <= 1e-5, worst
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_BF16).reshape(M, N)
    worst = max(rel_err(y[m], ref[m]) for m in range(M))
    assert worst <= 1e-2, worst


@pytest.mark.parametrize("bits,G,K,M", [(4, 128, 8192, 5), (4, 128, 16384, 33), (8, 64, 8192, 64),
                                        (8, 64, 8704, 20), (4, 128, 16640, 17)])
def test_tiled_decode_scale_staging(gpu, dgm, orc, bits, G, K, M):
    """Long K around the limits of the tiled kernel's scale staging: up to 128
    groups the workgroup's scales sit in LDS, more (136, 130 groups) keep the
    per-block gathers; M <= 16 with more than 63 groups also lands here."""
    N = 70
    rng = np.random.default_rng(M * 13 + K + bits)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    w[5 * K: 6 * K] *= np.float32(40.0)            # one row with much larger scales
    bias = rng.standard_normal(N).astype(np.float32)
    q, s = _quantize(gpu, to_dev(w), N, K, G, bits)
    ref = _ref(orc, q, s, x, bias, M, N, K, G, bits)
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_FP32)
    assert rel_err(y, ref) <= 1e-5
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_BF16)
    assert rel_err(y, ref) <= 1e-2


@pytest.mark.parametrize("M,N,K,G", [(17, 70, 512, 128), (40, 300, 4096, 128), (64, 129, 1024, 256),
                                     (64, 14336, 4096, 128)])
def test_tiled_decode_bf16_arithmetic(gpu, dgm, orc, M, N, K, G):
    """Reduced mode, int4, 16 < M <= 64: the tiled kernel takes bf16(x) against
    the exact codes (offset by 136, removed by an fp32 term per block) and
    applies the group scale in fp32, so it agrees with float64 products of
    bf16(X) and the dequantized weights to 1e-5 per row; rows 1e-20 and 1e20
    of the others keep that accuracy."""
    rng = np.random.default_rng(M * 7 + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[1] *= np.float32(1e-20)
    x[2] *= np.float32(1e20)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if M % 2 == 0 else None
    q, s = _quantize(gpu, to_dev(w), N, K, G, 4)
    wd = orc.dequant(from_dev(q), from_dev(s), N, K, G, 4).reshape(N, K).astype(np.float64)
    ref = _bf16_round(x) @ wd.T
    if bias is not None:
        ref = ref + bias.astype(np.float64)
    y = _forward(gpu, dgm, 4, q, s, x.ravel(), bias, M, N, K, G, dgm.DGM_MATH_BF16).reshape(M, N)
    worst = max(rel_err(y[m], ref[m]) for m in range(M))
    assert worst <= 1e-5, worst


def test_tiled_decode_bf16_non_finite(gpu, dgm, orc):
    """Reduced mode, M > 16: a NaN or an infinity in a row makes that row NaN;
    the other rows are unaffected."""
    M, N, K, G = 20, 64, 512, 128
    rng = np.random.default_rng(6)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[3, 7] = np.inf
    x[5, 300] = np.nan
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q, s = _quantize(gpu, to_dev(w), N, K, G, 4)
    y = _forward(gpu, dgm, 4, q, s, x.ravel(), None, M, N, K, G, dgm.DGM_MATH_BF16).reshape(M, N)
    ref = _ref(orc, q, s, x.ravel(), None, M, N, K, G, 4).reshape(M, N)
    assert np.all(np.isnan(y[3])) and np.all(np.isnan(y[5]))
    for m in (0, 1, 2, 4, 6, M - 1):
        assert rel_err(y[m], ref[m]) <= 1e-2, m


def test_rows_of_very_different_magnitude(gpu, dgm, orc):
    """Each row carries its own power-of-two scale: a tiny row next to a huge
    one keeps its own relative accuracy."""
    M, N, K, G = 4, 64, 512, 128
    rng = np.random.default_rng(3)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[1] *= np.float32(1e-20)
    x[2] *= np.float32(1e20)
    x[3] = 0.0
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q, s = _quantize(gpu, to_dev(w), N, K, G, 4)
    ref = _ref(orc, q, s, x.ravel(), None, M, N, K, G, 4).reshape(M, N)
    y = _forward(gpu, dgm, 4, q, s, x.ravel(), None, M, N, K, G, dgm.DGM_MATH_FP32).reshape(M, N)
    for m in range(3):
        assert rel_err(y[m], ref[m]) <= 1e-5, m
    assert np.all(y[3] == 0.0)


def test_non_finite_row_gives_nan(gpu, dgm, orc):
    M, N, K, G = 3, 32, 256, 128
    rng = np.random.default_rng(4)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[1, 7] = np.inf
    x[2, 100] = np.nan
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q, s = _quantize(gpu, to_dev(w), N, K, G, 4)
    y = _forward(gpu, dgm, 4, q, s, x.ravel(), None, M, N, K, G, dgm.DGM_MATH_FP32).reshape(M, N)
    ref = _ref(orc, q, s, x.ravel(), None, M, N, K, G, 4).reshape(M, N)
    assert rel_err(y[0], ref[0]) <= 1e-5
    assert np.all(np.isnan(y[1])) and np.all(np.isnan(y[2]))


def test_skinny_repeatable_and_kernel_entry(gpu, dgm, orc):
    """Bitwise identical results on repeated calls (fixed reduction order), and
    the kernel-level entry takes the same path as the wrapper."""
    import torch
    M, N, K, G = 8, 300, 1024, 128
    rng = np.random.default_rng(5)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q, s = _quantize(gpu, to_dev(w), N, K, G, 4)
    xd = to_dev(x)
    y1 = torch.zeros(M * N, device="cuda")
    y2 = torch.zeros(M * N, device="cuda")
    gpu.begin()
    gpu.gemm_nt_i4(q, s, xd, None, y1, dgm.GemmP(M, N, K, 0, G, 0, 0, 0))
    gpu.gemmNT(4, None, q, s, xd, None, y2, M, N, K, G)
    gpu.end()
    assert np.array_equal(from_dev(y1), from_dev(y2))
    assert rel_err(from_dev(y1), _ref(orc, q, s, x, None, M, N, K, G, 4)) <= 1e-5


# ---- large-M reduced-precision path (bf16 MFMA, W dequantized in LDS) -------

@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K,G", [(65, 33, 128, 32), (256, 256, 256, 128), (300, 500, 384, 64),
                                     (512, 768, 768, 32), (1000, 260, 1024, 128),
                                     (129, 40, 192, 64)])   # K % 128 != 0: fp32 tile path
def test_bf16_large_m(gpu, dgm, orc, bits, M, N, K, G):
    rng = np.random.default_rng(M + N + K + bits)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if M % 2 == 0 else None
    q, s = _quantize(gpu, to_dev(w), N, K, G, bits)
    ref = _ref(orc, q, s, x, bias, M, N, K, G, bits)
    y = _forward(gpu, dgm, bits, q, s, x, bias, M, N, K, G, dgm.DGM_MATH_BF16)
    assert rel_err(y, ref) <= 1e-2
    if K % 128 == 0:
        # The bf16 kernel's own arithmetic: float64 products of bf16(X) and
        # bf16(dequant(W)), fp32 accumulation (max relative error 1e-5).
        assert rel_err(y, _ref_bf16(orc, q, s, x, bias, M, N, K, G, bits)) <= 1e-5


def _bf16_round(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to(torch.float64).numpy()


def _ref_bf16(orc, q, s, x, bias, M, N, K, G, bits, rows=None):
    wd = orc.dequant(from_dev(q), from_dev(s), N, K, G, bits).reshape(N, K)
    xm = np.asarray(x, np.float32).reshape(M, K)
    if rows is not None:
        xm = xm[rows]
    y = _bf16_round(xm) @ _bf16_round(wd).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y.ravel()


@pytest.mark.parametrize("bits", [4, 8])
def test_config5_prefill_bf16(gpu, dgm, orc, bits):
    """c5: X[8192,4096] ~ N(0,1), W[14336,4096] ~ N(0,0.02) int4 / int8 G=128,
    bf16 path. The float64 references are checked on a sample of 96 rows."""
    import torch
    M, N, K, G = 8192, 14336, 4096, 128
    gen = torch.Generator(device="cpu").manual_seed(1005)
    x = torch.randn(M * K, generator=gen)
    w = torch.randn(N * K, generator=gen) * 0.02
    q, s = _quantize(gpu, w.to("cuda"), N, K, G, bits)
    y = _forward(gpu, dgm, bits, q, s, x.numpy(), None, M, N, K, G, dgm.DGM_MATH_BF16).reshape(M, N)
    wd = orc.dequant(from_dev(q), from_dev(s), N, K, G, bits).reshape(N, K).astype(np.float64)
    rows = np.random.default_rng(0).choice(M, 96, replace=False)
    ref = x.numpy().reshape(M, K)[rows].astype(np.float64) @ wd.T
    assert rel_err(y[rows], ref) <= 1e-2
    assert rel_err(y[rows].ravel(), _ref_bf16(orc, q, s, x.numpy(), None, M, N, K, G, bits, rows)) <= 1e-5
    assert np.all(np.isfinite(y))
