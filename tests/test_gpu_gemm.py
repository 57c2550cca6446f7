"""GPU parity of the fp32 GEMM family through the C ABI:
gemm_nt_{f32,i8,i4} (metal/kernels.metal:128-209), STE gemm_dx_{f32,i8,i4}
(211-268), gemm_dw / gemm_dw_acc (270-283, 1014-1027).

Bars (stated per assert):
  * the reference's own check (Check.swift:97-136): same shapes, seeds and
    distributions, max abs error < 2e-3 against dequant + cpuGemm*;
  * max relative error max|got - ref| / max|ref| <= 1e-5 against float64
    products of the same dequantized weights (the fp32 path's tolerance).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, rel_err, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-5


def quantize_dev(gpu, w_dev, N, K, G, bits):
    import torch
    q = torch.zeros(max(N * K // (2 if bits == 4 else 1), 1), dtype=torch.uint8 if bits == 4 else torch.int8,
                    device="cuda")
    s = torch.zeros(max(N * (K // G), 1), dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.quantize(w_dev, q, s, N, K, bits, G)
    gpu.end()
    return q, s


def host_codes(q):
    a = from_dev(q)
    return a


def run_step(gpu, bits, x, w, bias, dy, M, N, K, G, dw_init=None):
    """quantize -> gemmNT -> gemmDX -> gemmDW (+ gemmDWAcc) through the wrappers."""
    import torch
    xd, wd, dyd = to_dev(x), to_dev(w), to_dev(dy)
    bd = None if bias is None else to_dev(bias)
    q = s = None
    if bits != 32:
        q, s = quantize_dev(gpu, wd, N, K, G, bits)
    y = torch.zeros(max(M * N, 1), device="cuda")
    dx = torch.zeros(max(M * K, 1), device="cuda")
    dw = torch.zeros(max(N * K, 1), device="cuda")
    dwa = to_dev(dw_init) if dw_init is not None else None
    gpu.begin()
    gpu.gemmNT(bits, wd, q, s, xd, bd, y, M, N, K, G)
    gpu.gemmDX(bits, wd, q, s, dyd, dx, M, N, K, G)
    gpu.gemmDW(dyd, xd, dw, M, N, K)
    if dwa is not None:
        gpu.gemmDWAcc(dyd, xd, dwa, M, N, K)
    gpu.end()
    out = dict(y=from_dev(y)[: M * N], dx=from_dev(dx)[: M * K], dw=from_dev(dw)[: N * K])
    if dwa is not None:
        out["dwa"] = from_dev(dwa)
    if q is not None:
        out["q"], out["s"] = from_dev(q), from_dev(s)
    return out


def dequant_host(orc, out, w, N, K, G, bits):
    if bits == 32:
        return np.asarray(w, np.float32)
    q = out["q"][: (N * K if bits == 8 else N * K // 2)]
    if bits == 8:
        q = q.view(np.int8)
    return orc.dequant(q, out["s"][: N * (K // G)], N, K, G, bits)


@pytest.mark.parametrize("bits", [32, 8, 4])
def test_reference_check_gemm(gpu, orc, bits):
    """Check.swift:97-136 verbatim in shapes, seeds and draw order (G = 8)."""
    cases = [(3, 5, 7), (17, 13, 16), (8, 24, 32)] if bits == 32 else [(3, 5, 8), (15, 13, 16), (8, 24, 32)]
    rng = orc.RNG(1000 + bits)
    worst_abs, worst_rel = 0.0, 0.0
    for M, N, K in cases:
        x = rng.randn(M * K, 0.5)
        w = rng.randn(N * K, 0.5)
        bias = rng.randn(N, 0.1)
        dy = rng.randn(M * N, 0.2)
        out = run_step(gpu, bits, x, w, bias, dy, M, N, K, 8)
        if bits != 32:
            qr, sr = orc.quant(w, N, K, 8, bits)
            assert np.array_equal(out["q"][: qr.size].view(qr.dtype), qr)
        wd = dequant_host(orc, out, w, N, K, 8, bits)
        y_ref = orc.gemm_nt(x, wd, bias, M, N, K)
        dx_ref = orc.gemm_dx(dy, wd, M, N, K)
        dw_ref = orc.gemm_dw(dy, x, M, N, K)
        for got, ref in ((out["y"], y_ref), (out["dx"], dx_ref), (out["dw"], dw_ref)):
            worst_abs = max(worst_abs, float(np.max(np.abs(got - ref))))
        w64, x64, dy64 = (a.astype(np.float64) for a in (wd.reshape(N, K), x.reshape(M, K), dy.reshape(M, N)))
        worst_rel = max(worst_rel, rel_err(out["y"], (x64 @ w64.T + bias).ravel()),
                        rel_err(out["dx"], (dy64 @ w64).ravel()), rel_err(out["dw"], (dy64.T @ x64).ravel()))
    assert worst_abs < 2e-3, f"reference bar: max abs {worst_abs:.3e}"
    assert worst_rel <= TOL, f"fp32 bar: max rel {worst_rel:.3e}"


def _check_all(orc, out, x, w, bias, dy, M, N, K, G, bits, dw_init=None):
    wd = dequant_host(orc, out, w, N, K, G, bits).reshape(N, K).astype(np.float64)
    x64 = np.asarray(x, np.float64).reshape(M, K)
    dy64 = np.asarray(dy, np.float64).reshape(M, N)
    y_ref = x64 @ wd.T + (0 if bias is None else np.asarray(bias, np.float64))
    errs = {
        "y": rel_err(out["y"], y_ref.ravel()),
        "dx": rel_err(out["dx"], (dy64 @ wd).ravel()),
        "dw": rel_err(out["dw"], (dy64.T @ x64).ravel()),
    }
    if dw_init is not None:
        errs["dwa"] = rel_err(out["dwa"], (dy64.T @ x64).ravel() + dw_init)
    return errs


@pytest.mark.parametrize("bits", [8, 4])
def test_config1_and_config2_shapes(gpu, orc, bits):
    """c1: X[512,192], W[768,192] int8 G32. c2: X[512,768], W[192,768] int4 G32,
    dY ~ N(0, 1e-3). Inputs drawn X, W, dY from RNG(1000 + config)."""
    M, N, K = (512, 768, 192) if bits == 8 else (512, 192, 768)
    rng = orc.RNG(1001 if bits == 8 else 1002)
    x = rng.randn(M * K, 1.0)
    w = rng.randn(N * K, 0.02)
    dy = rng.randn(M * N, 1e-3)
    dw0 = rng.randn(N * K, 1e-2)
    out = run_step(gpu, bits, x, w, None, dy, M, N, K, 32, dw_init=dw0)
    errs = _check_all(orc, out, x, w, None, dy, M, N, K, 32, bits, dw_init=dw0)
    assert max(errs.values()) <= TOL, errs
    # Agreement with the Metal kernel order restated on the CPU.
    q = out["q"][: (N * K if bits == 8 else N * K // 2)]
    y_k = orc.gemm_nt_q(q.view(np.int8) if bits == 8 else q, out["s"], x, None, M, N, K, 32, bits)
    assert rel_err(out["y"], y_k.astype(np.float64)) <= TOL


@pytest.mark.parametrize("bits,G", [(32, 1), (8, 2), (4, 2), (8, 10), (4, 14), (8, 32), (4, 128)])
@pytest.mark.parametrize("M,N,K_groups", [(1, 1, 1), (1, 37, 3), (33, 47, 5), (70, 3, 2), (129, 65, 7)])
def test_ragged_shapes(gpu, orc, bits, G, M, N, K_groups):
    K = G * K_groups if bits != 32 else 5 * K_groups + 3
    rng = np.random.default_rng(M * 7 + N + K)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.1).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    dy = rng.standard_normal(M * N).astype(np.float32)
    dw0 = rng.standard_normal(N * K).astype(np.float32)
    out = run_step(gpu, bits, x, w, bias, dy, M, N, K, max(G, 1), dw_init=dw0)
    errs = _check_all(orc, out, x, w, bias, dy, M, N, K, max(G, 1), bits, dw_init=dw0)
    assert max(errs.values()) <= TOL, errs


@pytest.mark.parametrize("M,N,K,G,bits", [(33, 47, 256, 32, 4), (16, 16, 512, 16, 8), (100, 20, 1024, 128, 4),
                                          (17, 200, 768, 32, 8), (5, 9, 512, 1, 32), (64, 30, 256, 1, 32),
                                          (512, 192, 1024, 32, 4), (48, 16, 1024, 16, 8), (80, 24, 256, 128, 4),
                                          (72, 40, 512, 256, 8), (512, 200, 768, 32, 8)])
def test_forward_split_contraction(gpu, orc, M, N, K, G, bits):
    """Forwards with a contraction that is a multiple of 256 and a 4-way
    contraction split: int4/int8 codes with K / G % 4 == 0 take the pipelined
    16 x 32 kernel (codes, scales and X staged in LDS), the others and fp32
    weights the 16 x 16 kernel that reads X straight into registers; rows and
    columns past the matrix are clamped on load and masked on store."""
    rng = np.random.default_rng(M + 5 * N + K + bits)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.1).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if N % 2 == 0 else None
    dy = rng.standard_normal(M * N).astype(np.float32)
    out = run_step(gpu, bits, x, w, bias, dy, M, N, K, G)
    errs = _check_all(orc, out, x, w, bias, dy, M, N, K, G, bits)
    assert max(errs.values()) <= TOL, errs


@pytest.mark.parametrize("M,N,K,G,bits", [(48, 32, 40, 8, 8), (16, 48, 70, 14, 4), (80, 16, 24, 2, 4),
                                          (32, 64, 100, 10, 8), (64, 16, 27, 1, 32), (17, 32, 48, 16, 4),
                                          (96, 48, 36, 4, 8), (512, 192, 768, 32, 4), (512, 768, 192, 32, 8),
                                          (1000, 272, 1040, 16, 8), (33, 64, 96, 32, 4), (70, 128, 80, 16, 8),
                                          (9, 448, 36, 1, 32), (130, 256, 160, 32, 4), (1, 64, 64, 64, 8)])
def test_multiple_of_16_contractions(gpu, orc, M, N, K, G, bits):
    """Contractions that are multiples of 16 or 64 (K for the forward, N for
    dX, M for dW) with ragged output tiles: the deep-prefetch and LDS-staged
    kernels, whose rows and columns past the matrix are clamped rather than
    masked."""
    rng = np.random.default_rng(M + 3 * N + 7 * K + bits)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.1).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if M % 2 == 0 else None
    dy = rng.standard_normal(M * N).astype(np.float32)
    dw0 = rng.standard_normal(N * K).astype(np.float32)
    out = run_step(gpu, bits, x, w, bias, dy, M, N, K, G, dw_init=dw0)
    errs = _check_all(orc, out, x, w, bias, dy, M, N, K, G, bits, dw_init=dw0)
    assert max(errs.values()) <= TOL, errs


@pytest.mark.parametrize("M,N,K", [(64, 20, 36), (128, 36, 100), (448, 52, 44), (192, 12, 8), (512, 192, 768),
                                   (64, 4, 4), (320, 100, 260), (128, 30, 48), (256, 66, 20), (128, 100, 1280),
                                   (64, 68, 2048)])
def test_dw_shapes(gpu, orc, M, N, K):
    """dW / dW += over contractions that are multiples of 64 with ragged output
    tiles (rows and columns past N or K clamped, never stored): 64-row tiles
    (four dY columns per lane) where they need fewer rounds of workgroups on a
    256-CU part ((512, 192, 768), and ragged in N: (128, 100, 1280),
    (64, 68, 2048)), 32-row tiles otherwise (N = 30 and 66: two columns per
    lane always)."""
    import torch
    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal(M * K).astype(np.float32)
    dy = rng.standard_normal(M * N).astype(np.float32)
    dw0 = rng.standard_normal(N * K).astype(np.float32)
    xd, dyd = to_dev(x), to_dev(dy)
    dw = torch.full((N * K,), float("nan"), device="cuda")
    dwa = to_dev(dw0)
    gpu.begin()
    gpu.gemmDW(dyd, xd, dw, M, N, K)
    gpu.gemmDWAcc(dyd, xd, dwa, M, N, K)
    gpu.end()
    ref = dy.reshape(M, N).astype(np.float64).T @ x.reshape(M, K).astype(np.float64)
    assert rel_err(from_dev(dw), ref.ravel()) <= TOL
    assert rel_err(from_dev(dwa), ref.ravel() + dw0) <= TOL


def test_unaligned_operands(gpu, orc):
    import torch
    M, N, K, G = 20, 24, 64, 16
    rng = np.random.default_rng(5)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = rng.standard_normal(N * K).astype(np.float32)
    xs = torch.zeros(M * K + 1, device="cuda")
    xs[1:] = to_dev(x)
    wd = to_dev(w)
    q, s = quantize_dev(gpu, wd, N, K, G, 8)
    qs = torch.zeros(N * K + 1, dtype=torch.int8, device="cuda")
    qs[1:] = q
    y = torch.zeros(M * N, device="cuda")
    gpu.begin()
    gpu.gemmNT(8, None, qs[1:], s, xs[1:], None, y, M, N, K, G)
    gpu.end()
    wdq = orc.dequant(from_dev(q), from_dev(s), N, K, G, 8).reshape(N, K).astype(np.float64)
    assert rel_err(from_dev(y), (x.reshape(M, K).astype(np.float64) @ wdq.T).ravel()) <= TOL


def test_kernel_level_entries_and_bias_flag(gpu, dgm, orc):
    import torch
    M, N, K, G = 16, 32, 64, 32
    rng = np.random.default_rng(6)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = rng.standard_normal(N * K).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    wd, xd, bd = to_dev(w), to_dev(x), to_dev(b)
    q, s = quantize_dev(gpu, wd, N, K, G, 4)
    y1 = torch.zeros(M * N, device="cuda")
    y0 = torch.zeros(M * N, device="cuda")
    gpu.begin()
    gpu.gemm_nt_i4(q, s, xd, bd, y1, dgm.GemmP(M, N, K, 1, G, 0, 0, 0))
    gpu.gemm_nt_i4(q, s, xd, bd, y0, dgm.GemmP(M, N, K, 0, G, 0, 0, 0))   # hasBias = 0 ignores bias
    gpu.end()
    assert gpu.lastKernel == "gemm_nt_i4"
    wdq = orc.dequant(from_dev(q), from_dev(s), N, K, G, 4).reshape(N, K).astype(np.float64)
    ref0 = x.reshape(M, K).astype(np.float64) @ wdq.T
    assert rel_err(from_dev(y0), ref0.ravel()) <= TOL
    assert rel_err(from_dev(y1), (ref0 + b).ravel()) <= TOL


def test_gemm_error_paths(gpu, dgm):
    import torch
    t = torch.zeros(4096, device="cuda")
    q = torch.zeros(4096, dtype=torch.int8, device="cuda")
    with pytest.raises(dgm.DgmError) as e:
        gpu.gemmNT(8, None, q, t, t, None, t, 4, 4, 16, 8)
    assert e.value.code == dgm.DGM_ERR_NOT_BEGUN
    gpu.begin()
    with pytest.raises(dgm.DgmError) as e:       # K % qGroup != 0 (GPU.swift:229)
        gpu.gemmNT(8, None, q, t, t, None, t, 4, 4, 12, 8)
    assert e.value.code == dgm.DGM_ERR_SHAPE
    gpu.begin()
    with pytest.raises(dgm.DgmError) as e:       # GPU.swift:247
        gpu.gemmDX(4, None, q, t, t, t, 4, 4, 12, 8)
    assert e.value.code == dgm.DGM_ERR_SHAPE
    gpu.begin()
    with pytest.raises(dgm.DgmError) as e:
        gpu.gemmNT(16, t, q, t, t, None, t, 4, 4, 16, 8)
    assert e.value.code == dgm.DGM_ERR_BITS
    gpu.begin()
    with pytest.raises(dgm.DgmError) as e:
        gpu.gemmNT(8, None, None, t, t, None, t, 4, 4, 16, 8)
    assert e.value.code == dgm.DGM_ERR_ARG
    gpu.begin()
    gpu.gemmNT(8, None, q, t, t, None, t, 0, 4, 16, 8)     # M = 0: nothing to do
    gpu.gemmDW(t, t, t, 0, 4, 16)                           # M = 0: dW = 0
    gpu.end()
    assert float(t[:64].abs().sum()) == 0.0


# ---- gemmBwd: the gemmDW(+Acc) / gemmDX pair in one launch ---------------------

# One launch with LDS dX tiles (N % 64 == 0, N <= 448, M % 64 == 0; 32-row
# tiles for codes when N >= 128 and they fill half the CUs: (512, 192, 768),
# (1024, 192, 768), (512, 256, 800) with a ragged last column tile,
# (512, 128, 1024)), one launch with deep dX tiles (longer N, small dX:
# (512, 768, 192), (512, 48, 192)), or the two calls ((512, 768, 768): dX
# large enough for its own launch; M % 64 or N % 16 off).
BWD_SHAPES = [(512, 192, 768, 32), (512, 768, 192, 32), (512, 48, 192, 32), (512, 192, 192, 32),
              (64, 64, 128, 16), (128, 448, 64, 32), (1024, 192, 768, 32), (512, 256, 800, 32),
              (512, 128, 1024, 32),
              (512, 768, 768, 32), (100, 192, 768, 32), (64, 62, 128, 16)]


@pytest.mark.parametrize("bits", [32, 8, 4])
@pytest.mark.parametrize("M,N,K,G", BWD_SHAPES)
@pytest.mark.parametrize("acc", [False, True])
def test_gemm_bwd_is_the_pair(gpu, orc, bits, M, N, K, G, acc):
    import torch
    rng = np.random.default_rng(M + N + K + bits)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (0.02 * rng.standard_normal(N * K)).astype(np.float32)
    dy = (1e-3 * rng.standard_normal(M * N)).astype(np.float32)
    dw0 = rng.standard_normal(N * K).astype(np.float32)
    xd, wd, dyd = to_dev(x), to_dev(w), to_dev(dy)
    q = s = None
    if bits != 32:
        q, s = quantize_dev(gpu, wd, N, K, G, bits)
    dx1, dx2 = (torch.zeros(M * K, device="cuda") for _ in range(2))
    dw1, dw2 = to_dev(dw0), to_dev(dw0)
    gpu.begin()
    gpu.gemmBwd(bits, wd, q, s, dyd, xd, dx1, dw1, M, N, K, G, accumulate=acc)
    name = gpu.lastKernel
    (gpu.gemmDWAcc if acc else gpu.gemmDW)(dyd, xd, dw2, M, N, K)
    gpu.gemmDX(bits, wd, q, s, dyd, dx2, M, N, K, G)
    gpu.end()
    assert np.array_equal(from_dev(dx1).view(np.uint32), from_dev(dx2).view(np.uint32))
    assert np.array_equal(from_dev(dw1).view(np.uint32), from_dev(dw2).view(np.uint32))
    cpu = 32 if bits == 4 else 16 if bits == 8 else 4    # codes per 16-byte unit of the LDS dX tile
    lds_pair = N % 64 == 0 and N <= 448 and K % cpu == 0 and (bits == 32 or G % cpu == 0)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    deep_pair = N % 16 == 0 and -(-M // 16) * -(-K // 32) < 2 * cus
    fused = M % 64 == 0 and (lds_pair or deep_pair)
    assert (name == {32: "gemm_bwd_f32", 8: "gemm_bwd_i8", 4: "gemm_bwd_i4"}[bits]) == fused, name
    # and against float64 products of the dequantized weights
    wq = w if bits == 32 else orc.dequant(host_codes(q), from_dev(s), N, K, G, bits)
    wq = wq.reshape(N, K).astype(np.float64)
    ref_dx = dy.reshape(M, N).astype(np.float64) @ wq
    ref_dw = dy.reshape(M, N).astype(np.float64).T @ x.reshape(M, K).astype(np.float64)
    assert rel_err(from_dev(dx1), ref_dx.ravel()) <= TOL
    got_dw = from_dev(dw1).astype(np.float64) - (dw0 if acc else 0.0)
    assert rel_err(got_dw, ref_dw.ravel()) <= (1e-4 if acc else TOL)
