"""Dequant bit-exactness on the device, the reference's STE learning check and
the quantized GPT's default GEMM shapes, all through the C ABI.

1. Dequant (src/Check.swift:433-458, metal/kernels.metal:69-75, 170-176) is
   fused into every forward and dX kernel, so it is pinned through them with
   one-hot operands: Y = I_K deq(W)^T and dX = I_N deq(W) select single
   dequantized weights, every other product being an exact zero. The fp32
   paths (tile kernels, the pipelined forward, the decode kernels at M <= 64)
   must return orc_dequant's bytes; the bf16 MFMA prefill path must return
   bf16(orc_dequant) (round to nearest even), as fp32.
2. checkLinearLearns (src/Check.swift:342-389): a 16x16x16 linear trained
   against a teacher with gemmNT -> MSE gradient -> gemmDW -> adam for 40
   steps must more than halve its loss for bits 32 / 8 / 4. The first step is
   compared with the oracle where the oracle is exact (codes, scales, and
   AdamW applied to the same gradient bytes).
3. The quantized GPT's default shapes (src/Train.swift:112-117,
   src/Params.swift:5, src/GPT.swift:340-425): batch 16 x block 64 = M 1024,
   embd 128, mlp 512, vocab 65 (tied lm head), qGroup 8, bias on the block
   linears: forward, dX and dW within max relative error 1e-5 of float64, and
   the forward within 1e-5 of the Metal kernel order restated on the CPU.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, rel_err, to_dev
from test_gpu_gemm import _check_all, run_step

pytestmark = pytest.mark.gpu


def _quantize(gpu, w, N, K, G, bits):
    import torch
    q = torch.zeros(N * K // (2 if bits == 4 else 1), dtype=torch.uint8 if bits == 4 else torch.int8,
                    device="cuda")
    s = torch.zeros(N * (K // G), dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.quantize(to_dev(w), q, s, N, K, bits, G)
    gpu.end()
    return q, s


def _weights(N, K, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(N * K) * 0.05).astype(np.float32)
    w[: K // 2] = 0.0                 # an all-zero half row: scale 1e-8, codes 0
    return w


def _deq(orc, q, s, N, K, G, bits):
    qh = from_dev(q)
    return orc.dequant(qh.view(np.int8) if bits == 8 else qh, from_dev(s), N, K, G, bits).reshape(N, K)


def _bf16_bits(a):
    """fp32 -> bf16 (nearest even) -> fp32, on the bit patterns."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


def _same_bits(got, want):
    got = np.ascontiguousarray(got, np.float32)
    want = np.ascontiguousarray(want, np.float32)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    return bad.size == 0, (bad[:5], got.ravel()[bad[:5]], want.ravel()[bad[:5]])


def _forward(gpu, dgm, bits, q, s, x, M, N, K, G, math):
    import torch
    y = torch.full((M * N,), float("nan"), device="cuda")
    gpu.set_math(math)
    try:
        gpu.begin()
        gpu.gemmNT(bits, None, q, s, to_dev(x), None, y, M, N, K, G)
        gpu.end()
    finally:
        gpu.set_math(dgm.DGM_MATH_FP32)
    return from_dev(y).reshape(M, N)


# Forward shapes with M = K > 64, one per fp32 kernel family: the generic
# tile kernel (G = 8), the LDS-staged kernel (c1's K = 192), the pipelined
# kernel (c2's K = 768), the register-direct kernel (K / G not a multiple of
# 4) and the deep kernel (K = 2048).
FWD_TILES = [(8, 64, 96, 8), (4, 64, 96, 8), (8, 192, 128, 32), (4, 192, 128, 32), (8, 768, 64, 32),
             (4, 768, 64, 32), (8, 256, 80, 128), (4, 256, 80, 128), (8, 2048, 48, 128), (4, 2048, 48, 32)]


@pytest.mark.parametrize("bits,K,N,G", FWD_TILES)
def test_dequant_exact_fp32_tiles(gpu, dgm, orc, bits, K, N, G):
    w = _weights(N, K, K + N + G + bits)
    q, s = _quantize(gpu, w, N, K, G, bits)
    x = np.eye(K, dtype=np.float32).ravel()
    y = _forward(gpu, dgm, bits, q, s, x, K, N, K, G, dgm.DGM_MATH_FP32)
    ok, info = _same_bits(y.T, _deq(orc, q, s, N, K, G, bits))
    assert ok, info


@pytest.mark.parametrize("bits,G", [(4, 128), (4, 256), (8, 64), (8, 128)])
@pytest.mark.parametrize("M", [1, 16, 64])
@pytest.mark.parametrize("math", ["fp32", "bf16"])
@pytest.mark.parametrize("span", [2, 4])
def test_dequant_exact_decode(gpu, dgm, orc, bits, G, M, math, span):
    """M <= 64: the decode kernels (f16 MFMA over exact activation pieces;
    span 4 gives a multiple of four groups, the one-launch kernel's domain at
    M <= 16). Each call selects M weights per row of W with a one-hot row per
    output row; the calls cover every k of the matrix (M = 1: the first group
    and a spread of single columns)."""
    N, K = 72, span * max(G, 128)
    w = _weights(N, K, M + G + bits)
    q, s = _quantize(gpu, w, N, K, G, bits)
    deq = _deq(orc, q, s, N, K, G, bits)
    mode = dgm.DGM_MATH_FP32 if math == "fp32" else dgm.DGM_MATH_BF16
    starts = range(0, K, M) if M > 1 else list(range(0, G)) + [G, G + 1, K // 2 + 3, K - 2, K - 1]
    for k0 in starts:
        rows = min(M, K - k0)
        x = np.zeros((M, K), np.float32)
        x[np.arange(rows), k0 + np.arange(rows)] = 1.0
        if rows < M:
            x[rows:, 0] = 1.0
        y = _forward(gpu, dgm, bits, q, s, x.ravel(), M, N, K, G, mode)
        ok, info = _same_bits(y[:rows].T, deq[:, k0:k0 + rows])
        assert ok, (k0, info)


@pytest.mark.parametrize("bits,G", [(4, 32), (4, 128), (8, 32), (8, 128)])
@pytest.mark.parametrize("K", [256, 512])
def test_dequant_exact_bf16_prefill(gpu, dgm, orc, bits, G, K):
    """M > 64 in the reduced-precision mode: bf16 MFMA on W dequantized in LDS.
    Y = I_K deq(W)^T is bf16(deq(W)) exactly (bf16(1) = 1, one nonzero
    product per output, fp32 accumulation)."""
    N = 272
    w = _weights(N, K, K + G + bits)
    q, s = _quantize(gpu, w, N, K, G, bits)
    x = np.eye(K, dtype=np.float32).ravel()
    y = _forward(gpu, dgm, bits, q, s, x, K, N, K, G, dgm.DGM_MATH_BF16)
    ok, info = _same_bits(y.T, _bf16_bits(_deq(orc, q, s, N, K, G, bits)))
    assert ok, info


# dX = I_N deq(W): the LDS-staged dX kernel (N % 64 == 0, N <= 448), the deep
# kernel (N > 448) and the generic one (G = 8), alone and inside gemmBwd.
DX_CASES = [(8, 192, 768, 32), (4, 192, 768, 32), (8, 512, 256, 128), (4, 512, 256, 128), (8, 40, 64, 8),
            (4, 40, 64, 8)]


@pytest.mark.parametrize("bits,N,K,G", DX_CASES)
def test_dequant_exact_dx(gpu, dgm, orc, bits, N, K, G):
    import torch
    w = _weights(N, K, N + K + bits)
    q, s = _quantize(gpu, w, N, K, G, bits)
    deq = _deq(orc, q, s, N, K, G, bits)
    dy = to_dev(np.eye(N, dtype=np.float32).ravel())
    x = to_dev(np.zeros(N * K, np.float32))
    dx1 = torch.full((N * K,), float("nan"), device="cuda")
    dx2 = torch.full((N * K,), float("nan"), device="cuda")
    dw = torch.zeros(N * K, device="cuda")
    gpu.begin()
    gpu.gemmDX(bits, None, q, s, dy, dx1, N, N, K, G)
    gpu.gemmBwd(bits, None, q, s, dy, x, dx2, dw, N, N, K, G, False)
    gpu.end()
    for got in (dx1, dx2):
        ok, info = _same_bits(from_dev(got).reshape(N, K), deq)
        assert ok, info


# ---- checkLinearLearns (src/Check.swift:342-389) -----------------------------


def _loss_and_dy(y, target, M, N):
    """The reference's host loop: loss += d*d in fp32, dy = d * (2 / (M*N))."""
    d = (y - target).astype(np.float32)
    loss = np.float32(0)
    for v in d:
        loss = np.float32(loss + v * v)
    inv = np.float32(2) / np.float32(M * N)
    return float(loss / np.float32(M * N)), (d * inv).astype(np.float32)


@pytest.mark.parametrize("bits", [32, 8, 4])
def test_check_linear_learns(gpu, orc, bits):
    import torch
    M = N = K = 16
    G = 8
    rng = orc.RNG(20 + bits)
    x = rng.randn(M * K, 0.5)
    teacher = rng.randn(N * K, 0.3)
    target = orc.gemm_nt(x, teacher, np.zeros(N, np.float32), M, N, K)
    w0 = rng.randn(N * K, 0.02)                       # fillNormal(w, std: 0.02)
    wd, xd = to_dev(w0), to_dev(x)
    m, v = torch.zeros(N * K, device="cuda"), torch.zeros(N * K, device="cuda")
    dwd, yd = torch.zeros(N * K, device="cuda"), torch.zeros(M * N, device="cuda")
    q = s = None
    if bits != 32:
        q = torch.zeros(N * K // (2 if bits == 4 else 1), dtype=torch.uint8 if bits == 4 else torch.int8,
                        device="cuda")
        s = torch.zeros(N * (K // G), device="cuda")

    def loss_of():
        gpu.begin()
        if bits != 32:
            gpu.quantize(wd, q, s, N, K, bits, G)
        gpu.gemmNT(bits, wd, q, s, xd, None, yd, M, N, K, G)
        gpu.end()
        return _loss_and_dy(from_dev(yd), target, M, N)

    initial, dy = loss_of()
    if bits != 32:
        qr, sr = orc.quant(w0, N, K, G, bits)
        assert np.array_equal(from_dev(q).view(qr.dtype), qr) and np.array_equal(from_dev(s), sr)
    lr = np.float32(0.05 if bits == 4 else 0.08)
    b1, b2 = np.float32(0.9), np.float32(0.95)
    for step in range(1, 41):
        ibc1 = float(np.float32(1) / (np.float32(1) - b1 ** np.float32(step)))
        ibc2 = float(np.float32(1) / (np.float32(1) - b2 ** np.float32(step)))
        w_before, m_before, v_before = from_dev(wd), from_dev(m), from_dev(v)
        dyd = to_dev(dy)
        gpu.begin()
        gpu.gemmDW(dyd, xd, dwd, M, N, K)
        gpu.adam(wd, dwd, m, v, N * K, float(lr), float(b1), float(b2), 1e-8, 0.0, ibc1, ibc2)
        gpu.end()
        if step == 1:
            g = from_dev(dwd)
            ref_g = dy.reshape(M, N).astype(np.float64).T @ x.reshape(M, K).astype(np.float64)
            assert rel_err(g, ref_g.ravel()) <= 1e-5
            rw, rm, rv = orc.adamw(w_before, g, m_before, v_before, float(lr), float(b1), float(b2), 1e-8, 0.0,
                                   ibc1, ibc2)
            for got, want in ((wd, rw), (m, rm), (v, rv)):
                assert np.array_equal(from_dev(got).view(np.uint32), want.view(np.uint32))
        _, dy = loss_of()
    final, _ = loss_of()
    assert np.isfinite(final) and final < initial * 0.5, (bits, initial, final)


# ---- the quantized GPT's default GEMM shapes ---------------------------------

GPT_SHAPES = [(128, 128, True), (512, 128, True), (128, 512, True), (65, 128, False)]


@pytest.mark.parametrize("bits", [32, 8, 4])
@pytest.mark.parametrize("N,K,has_bias", GPT_SHAPES)
def test_gpt_default_shapes(gpu, orc, bits, N, K, has_bias):
    """M = 16 x 64 tokens; wq/wk/wv/wo [128,128], wfc [512,128], wproj
    [128,512] with bias; the tied lm head wte [65,128] without; qGroup 8."""
    M, G = 1024, 8
    rng = np.random.default_rng(N * 7 + K + bits)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32) if has_bias else None
    dy = (rng.standard_normal(M * N) * 1e-2).astype(np.float32)
    dw0 = (rng.standard_normal(N * K) * 1e-2).astype(np.float32)
    out = run_step(gpu, bits, x, w, bias, dy, M, N, K, G, dw_init=dw0)
    errs = _check_all(orc, out, x, w, bias, dy, M, N, K, G, bits, dw_init=dw0)
    assert max(errs.values()) <= 1e-5, errs
    if bits != 32:
        qh = out["q"]
        yk = orc.gemm_nt_q(qh.view(np.int8) if bits == 8 else qh, out["s"], x, bias, M, N, K, G, bits)
        assert rel_err(out["y"], yk.astype(np.float64)) <= 1e-5
