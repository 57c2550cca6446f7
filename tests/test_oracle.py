"""Pins the CPU oracle (oracle/oracle.c) without restating its formulas.

Each check is a known answer worked out by hand, a published test vector, an
invariant that a plausible mistake breaks (dropped term, wrong sign, wrong
index, swapped operand), or a float64 numpy computation of the same
mathematics. Reference routines: src/GPU.swift:4-29 (RNG),
src/Check.swift:399-494 (quant, dequant, CPU GEMMs), metal/kernels.metal
(kernel orders and DiT block pieces).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

# ---- RNG -----------------------------------------------------------------


def test_splitmix64_published_vector(orc):
    # Published splitmix64 outputs for seed 1234567 (Vigna's reference
    # generator, also used by the xoshiro test suites).
    r = orc.RNG(1234567)
    got = [r.next() for _ in range(5)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]


def test_rng_seed_zero_is_remapped(orc):
    # GPU.swift:6-8: seed 0 becomes 0x1234_5678_9abc_def0.
    a, b = orc.RNG(0), orc.RNG(0x123456789ABCDEF0)
    assert [a.next() for _ in range(3)] == [b.next() for _ in range(3)]


def test_uniform_is_24_bit_grid_in_unit_interval(orc):
    r = orc.RNG(99)
    r2 = orc.RNG(99)
    for _ in range(2000):
        u = r.uniform()
        top = r2.next() >> 40
        # (top + 1) / 2^24 is exact in fp32 for top < 2^24.
        assert u == (top + 1) / 16777216.0
        assert 0.0 < u <= 1.0


def test_normal_matches_float64_box_muller(orc):
    r, r2 = orc.RNG(7), orc.RNG(7)
    pi_toward_zero = float(np.frombuffer(np.uint32(0x40490FDA).tobytes(), np.float32)[0])
    for _ in range(2000):
        z = r.normal()
        u1 = max(r2.uniform(), 1e-7)
        u2 = r2.uniform()
        ref = math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * pi_toward_zero * u2)
        assert abs(z - ref) <= 4e-6 * max(1.0, abs(ref))


def test_normal_moments(orc):
    z = orc.RNG(31337).randn(200_000, 1.0).astype(np.float64)
    assert abs(z.mean()) < 0.01
    assert abs(z.std() - 1.0) < 0.01


def test_randn_stream_equals_scalar_draws(orc):
    a = orc.RNG(5)
    b = orc.RNG(5)
    v = a.randn(37, 0.3)
    w = np.array([b.normal() for _ in range(37)], dtype=np.float32) * np.float32(0.3)
    assert np.array_equal(v, w)
    assert a.state == b.state


# ---- quantization known answers --------------------------------------------


def _f(x):
    return np.float32(x)


def test_quant_int8_ties_to_even_kat(orc):
    u = 2.0 ** -10
    # maxAbs = 127 * 2^-10 -> s = 2^-10 exactly; w / s is exact, so the codes
    # are rint of the listed multipliers: 2.5 -> 2, 3.5 -> 4, 0.5 -> 0, 1.5 -> 2.
    w = np.array([127, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5], dtype=np.float64) * u
    q, s = orc.quant(w.astype(np.float32), 1, 8, 8, 8)
    assert s[0] == _f(u)
    assert q.tolist() == [127, 2, 4, -2, -4, 0, 0, 2]


def test_quant_int4_ties_and_nibbles_kat(orc):
    u = 2.0 ** -4
    w = np.array([7, 2.5, 3.5, -2.5, -3.5, 0.5, -1.5, -7], dtype=np.float64) * u
    q, s = orc.quant(w.astype(np.float32), 1, 8, 8, 4)
    assert s[0] == _f(u)
    # codes 7, 2, 4, -2, -4, 0, -2, -7 -> nibbles 7,2,4,E,C,0,E,9; even k low.
    assert q.tolist() == [0x27, 0xE4, 0x0C, 0x9E]


def test_quant_negative_nibble_encodings(orc):
    # A group whose codes are -7 and -1: -7 -> 0x9, -1 -> 0xF; byte = lo | hi << 4.
    w = np.array([-7, -1], dtype=np.float32) * _f(0.125)
    q, s = orc.quant(w, 1, 2, 2, 4)
    assert s[0] == _f(0.125)
    assert q.tolist() == [0xF9]


def test_quant_all_zero_group(orc):
    for bits in (8, 4):
        q, s = orc.quant(np.zeros(16, np.float32), 1, 16, 8, bits)
        assert s.tolist() == [_f(1e-8), _f(1e-8)]
        assert not np.any(q)


def test_quant_single_nonzero_per_group(orc):
    w = np.zeros(32, np.float32)
    w[3] = -0.3
    w[17] = 0.05
    q, s = orc.quant(w, 1, 32, 16, 8)
    assert s[0] == _f(0.3) / _f(127) and s[1] == _f(0.05) / _f(127)
    assert q[3] == -127 and q[17] == 127
    assert np.count_nonzero(q) == 2


def test_quant_tiny_group_scale_floor(orc):
    # maxAbs / 127 below 1e-8 -> s = 1e-8f; codes = rint(w / 1e-8).
    w = np.array([1e-7, -2.6e-8, 0.0, 4e-9], dtype=np.float32)
    q, s = orc.quant(w, 1, 4, 4, 8)
    assert s[0] == _f(1e-8)
    assert q.tolist() == [10, -3, 0, 0]


def test_quant_code_clamps(orc):
    assert orc.quant_code(1000.0, 1.0, 127) == 127
    assert orc.quant_code(-1000.0, 1.0, 7) == -7
    assert orc.quant_code(6.5, 1.0, 7) == 6     # tie to even
    assert orc.quant_code(-7.5, 1.0, 7) == -7   # rint -8, clamped


def test_quant_rejects_odd_int4_group(orc):
    with pytest.raises(ValueError):
        orc.quant(np.zeros(9, np.float32), 1, 9, 3, 4)     # odd group for int4


def test_quant_partial_last_group_is_left_alone(orc):
    # cols = 10, G = 4: floor(10/4) = 2 groups per row are quantized, the two
    # tail columns keep their prior codes, scales are strided by 2
    # (Check.swift:401-405 loops g in 0..<cols/group).
    u = 2.0 ** -5
    w = np.array([[127, 1, 2, 3, 64, -127, 0, 5, 9, 9],
                  [0, 0, 0, 0, 1, 2, 3, -127, 7, 7]], dtype=np.float64) * u
    prior = np.full(20, 99, np.int8)
    q, s = orc.quant(w.astype(np.float32).ravel(), 2, 10, 4, 8, init=prior)
    assert s.tolist() == [np.float32(u), np.float32(u), np.float32(1e-8), np.float32(u)]
    assert q.reshape(2, 10).tolist() == [[127, 1, 2, 3, 64, -127, 0, 5, 99, 99],
                                         [0, 0, 0, 0, 1, 2, 3, -127, 99, 99]]


def _unpack4(q, n):
    lo = (q & 0xF).astype(np.int32)
    hi = (q >> 4).astype(np.int32)
    c = np.empty(n, np.int32)
    c[0::2], c[1::2] = lo, hi
    return np.where(c >= 8, c - 16, c)


@pytest.mark.parametrize("bits,group,rows,cols", [
    (8, 8, 5, 16), (4, 8, 5, 16), (8, 32, 24, 192), (4, 32, 12, 768),
    (4, 128, 6, 4096), (8, 2, 3, 10), (4, 6, 4, 36), (8, 128, 3, 256)])
def test_quant_invariants_and_float32_brute_force(orc, bits, group, rows, cols):
    rng = np.random.default_rng(bits * 1000 + group)
    w = (rng.standard_normal(rows * cols) * rng.choice([0.02, 0.3, 3.0])).astype(np.float32)
    q, s = orc.quant(w, rows, cols, group, bits)
    lim = 7 if bits == 4 else 127
    codes = q.astype(np.int32) if bits == 8 else _unpack4(q, rows * cols)
    wg = w.reshape(rows, cols // group, group)
    cg = codes.reshape(rows, cols // group, group)
    # Scale: max(maxAbs / qmax, 1e-8f) with a float32 IEEE divide (numpy).
    max_abs = np.abs(wg).max(axis=2)
    s_ref = np.maximum(max_abs / np.float32(lim), np.float32(1e-8)).astype(np.float32)
    assert np.array_equal(s.reshape(rows, -1), s_ref)
    assert np.all(np.abs(cg) <= lim)
    # The group's arg-max element codes to +-lim.
    am = np.abs(wg).argmax(axis=2)
    top = np.take_along_axis(cg, am[..., None], axis=2)[..., 0]
    big = max_abs / lim >= 1e-8
    assert np.all(np.abs(top[big]) == lim)
    # Rounding error at most half a step (1 ulp slack for w / s).
    err = np.abs(cg * s_ref[..., None].astype(np.float64) - wg.astype(np.float64))
    assert np.all(err <= s_ref[..., None] * (0.5 + 2 ** -20))
    # float32 numpy brute force of the definition (np.rint rounds half to even).
    ref = np.clip(np.rint(wg / s_ref[..., None]), -lim, lim).astype(np.int32)
    assert np.array_equal(cg, ref)
    assert q.size == (rows * cols if bits == 8 else rows * cols // 2)
    assert s.size == rows * cols // group


# ---- dequant -----------------------------------------------------------------


def test_dequant_hand_built_codes(orc):
    q4 = np.array([0x27, 0xE4, 0x0C, 0x9E], np.uint8)   # 7,2,4,-2,-4,0,-2,-7
    s = np.array([0.5, 0.25], np.float32)                # G = 4
    out = orc.dequant(q4, s, 1, 8, 4, 4)
    assert out.tolist() == [3.5, 1.0, 2.0, -1.0, -1.0, 0.0, -0.5, -1.75]
    q8 = np.array([127, -127, 1, 0], np.int8)
    out = orc.dequant(q8, np.array([0.1], np.float32), 1, 4, 4, 8)
    assert out.tolist() == [_f(127) * _f(0.1), _f(-127) * _f(0.1), _f(0.1), 0.0]


@pytest.mark.parametrize("bits", [8, 4])
def test_dequant_round_trip(orc, bits):
    rng = np.random.default_rng(3)
    rows, cols, G = 7, 64, 16
    w = (rng.standard_normal(rows * cols) * 0.5).astype(np.float32)
    q, s = orc.quant(w, rows, cols, G, bits)
    d = orc.dequant(q, s, rows, cols, G, bits)
    step = np.repeat(s.reshape(rows, -1), G, axis=1).reshape(-1)
    assert np.all(np.abs(d.astype(np.float64) - w) <= step * (0.5 + 2 ** -20))


# ---- GEMMs against float64 ------------------------------------------------


def _rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.parametrize("M,N,K", [(3, 5, 7), (17, 13, 16), (8, 24, 32), (1, 9, 64)])
def test_cpu_gemms_match_float64(orc, M, N, K):
    rng = np.random.default_rng(M * 100 + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((N, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    dy = rng.standard_normal((M, N)).astype(np.float32)
    x64, w64, dy64 = x.astype(np.float64), w.astype(np.float64), dy.astype(np.float64)
    assert _rel(orc.gemm_nt(x, w, b, M, N, K), (x64 @ w64.T + b).ravel()) < 1e-6
    assert _rel(orc.gemm_nt(x, w, None, M, N, K), (x64 @ w64.T).ravel()) < 1e-6
    assert _rel(orc.gemm_dx(dy, w, M, N, K), (dy64 @ w64).ravel()) < 1e-6
    assert _rel(orc.gemm_dw(dy, x, M, N, K), (dy64.T @ x64).ravel()) < 1e-6
    base = rng.standard_normal(N * K).astype(np.float32)
    assert _rel(orc.gemm_dw(dy, x, M, N, K, dw=base), (dy64.T @ x64).ravel() + base) < 1e-6


def test_cpu_gemm_identity_and_one_hot(orc):
    K = 6
    x = np.arange(2 * K, dtype=np.float32).reshape(2, K)
    eye = np.eye(K, dtype=np.float32)
    b = np.arange(K, dtype=np.float32) * 10
    assert np.array_equal(orc.gemm_nt(x, eye, b, 2, K, K), (x + b).ravel())
    # One-hot dY selects one row of W for dX and one row of X for dW.
    w = np.arange(3 * K, dtype=np.float32).reshape(3, K)
    dy = np.zeros((2, 3), np.float32)
    dy[1, 2] = 1
    dx = orc.gemm_dx(dy, w, 2, 3, K).reshape(2, K)
    assert np.array_equal(dx[1], w[2]) and not np.any(dx[0])
    dw = orc.gemm_dw(dy, x, 2, 3, K).reshape(3, K)
    assert np.array_equal(dw[2], x[1]) and not np.any(dw[:2])


@pytest.mark.parametrize("bits,G", [(8, 8), (4, 8), (8, 32), (4, 32)])
def test_kernel_order_quantized_gemms_match_float64(orc, bits, G):
    rng = np.random.default_rng(G + bits)
    M, N, K = 9, 11, 4 * G
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.3).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    dy = rng.standard_normal((M, N)).astype(np.float32)
    q, s = orc.quant(w, N, K, G, bits)
    wd = orc.dequant(q, s, N, K, G, bits).reshape(N, K).astype(np.float64)
    x64, dy64 = x.astype(np.float64), dy.astype(np.float64)
    assert _rel(orc.gemm_nt_q(q, s, x, b, M, N, K, G, bits), (x64 @ wd.T + b).ravel()) < 1e-6
    assert _rel(orc.gemm_dx_q(q, s, dy, M, N, K, G, bits), (dy64 @ wd).ravel()) < 1e-6
    # The two reference orders (Check.swift dequant-then-GEMM; kernel order) agree.
    y_cpu = orc.gemm_nt(x, wd.astype(np.float32), b, M, N, K)
    assert _rel(orc.gemm_nt_q(q, s, x, b, M, N, K, G, bits), y_cpu.astype(np.float64)) < 1e-6


# ---- DiT block pieces ----------------------------------------------------------


def test_rmsnorm_unit_rows_and_float64(orc):
    rows, cols = 4, 8
    x = np.ones((rows, cols), np.float32)
    x[1] *= -1
    w = np.arange(1, cols + 1, dtype=np.float32)
    y, rstd = orc.rmsnorm_fwd(x, w, rows, cols, 0.0)
    assert np.array_equal(y.reshape(rows, cols)[0], w)
    assert np.array_equal(y.reshape(rows, cols)[1], -w)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    y, rstd = orc.rmsnorm_fwd(x, w, rows, cols, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert _rel(y, ref.ravel()) < 1e-6


def test_rope_identity_at_t0_and_norm_preserving(orc):
    B, T, H, D = 2, 5, 3, 8
    c, s = orc.rope_tables(T, D, 10000.0)
    assert np.all(c.reshape(T, D)[0] == 1) and np.all(s.reshape(T, D)[0] == 0)
    # Half-duplicated tables; angle t * theta^(-2i/D) in float64.
    i = np.arange(D // 2)
    ang = np.arange(T)[:, None] * 10000.0 ** (-2.0 * i / D)
    assert np.allclose(c.reshape(T, D)[:, : D // 2], np.cos(ang), atol=2e-6)
    assert np.allclose(s.reshape(T, D)[:, D // 2:], np.sin(ang), atol=2e-6)
    x = np.random.default_rng(2).standard_normal(B * T * H * D).astype(np.float32)
    y = orc.rope_fwd(x, c, s, B, T, H, D).reshape(B, T, H, D)
    xr = x.reshape(B, T, H, D)
    assert np.array_equal(y[:, 0], xr[:, 0])
    nx = xr[..., : D // 2] ** 2 + xr[..., D // 2:] ** 2
    ny = y[..., : D // 2].astype(np.float64) ** 2 + y[..., D // 2:].astype(np.float64) ** 2
    assert np.allclose(nx, ny, rtol=1e-5, atol=1e-6)
    # First half rotates as (x1 cos - x2 sin), second as (x2 cos + x1 sin).
    ct, st = np.cos(ang)[None, :, None, :], np.sin(ang)[None, :, None, :]
    x1, x2 = xr[..., : D // 2].astype(np.float64), xr[..., D // 2:].astype(np.float64)
    assert np.allclose(y[..., : D // 2], x1 * ct - x2 * st, atol=1e-5)
    assert np.allclose(y[..., D // 2:], x2 * ct + x1 * st, atol=1e-5)


def test_attention_equal_keys_uniform_average(orc):
    # Equal keys -> uniform softmax -> av is the mean of v over s
    # (the closed form behind Check.swift's attention check).
    B, T, H, D = 1, 4, 2, 4
    rng = np.random.default_rng(4)
    q = rng.standard_normal(B * T * H * D).astype(np.float32)
    k = np.ones(B * T * H * D, np.float32)
    v = rng.standard_normal((B, T, H, D)).astype(np.float32)
    _, probs, av = orc.attn_fwd(q, k, v, B, T, H, D)
    assert np.allclose(probs, 1.0 / T, atol=1e-7)
    ref = np.broadcast_to(v.astype(np.float64).mean(axis=1, keepdims=True), v.shape)
    assert np.allclose(av.reshape(v.shape), ref, atol=1e-6)


def test_attention_float64(orc):
    B, T, H, D = 2, 6, 2, 8
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((B, T, H, D)).astype(np.float32) for _ in range(3))
    scores, probs, av = orc.attn_fwd(q, k, v, B, T, H, D, 0)
    q64, k64, v64 = (a.astype(np.float64).transpose(0, 2, 1, 3) for a in (q, k, v))
    sc = q64 @ k64.transpose(0, 1, 3, 2) / math.sqrt(D)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    o = (p @ v64).transpose(0, 2, 1, 3)
    assert _rel(probs, p.ravel()) < 1e-5
    assert np.allclose(probs.reshape(B, H, T, T).sum(-1), 1.0, atol=1e-6)
    assert _rel(av, o.ravel()) < 1e-5
    # causal flag masks s > t.
    _, pc, _ = orc.attn_fwd(q, k, v, B, T, H, D, 1)
    assert np.all(np.triu(pc.reshape(B, H, T, T), 1) == 0)


def test_swiglu_and_mix(orc):
    g = np.array([0.0, 1.0, -2.0, 30.0, -30.0], np.float32)
    u = np.array([5.0, 2.0, 1.0, 1.0, 1.0], np.float32)
    y = orc.swiglu_fwd(g, u)
    g64 = g.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * u
    assert y[0] == 0.0
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-12)
    a = np.array([1.0, 2.0], np.float32)
    b = np.array([3.0, -4.0], np.float32)
    assert orc.mix(a, b, 0.5, 0.5).tolist() == [2.0, -1.0]


def test_repeat_heads(orc):
    B, T, H, D = 2, 3, 4, 2
    src = np.arange(B * T * D, dtype=np.float32)
    dst = orc.repeat_heads(src, B, T, H, D).reshape(B, T, H, D)
    for h in range(H):
        assert np.array_equal(dst[:, :, h, :], src.reshape(B, T, D))


def _dit_float64(cfg, W, x):
    """Independent float64 numpy statement of src/DiT.swift:520-550 using
    matrix products, with the already-dequantized weights."""
    B, T, C, H, D = cfg.B, cfg.T, cfg.C, cfg.H, cfg.D
    M = B * T

    def rms(a, w):
        return a / np.sqrt((a * a).mean(axis=1, keepdims=True) + cfg.eps) * w

    i = np.arange(D // 2)
    ang = np.arange(T)[:, None] * float(cfg.theta) ** (-2.0 * i / D)
    cos, sin = np.cos(ang), np.sin(ang)

    def rope(a):   # a: [B, T, h, D]
        x1, x2 = a[..., : D // 2], a[..., D // 2:]
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)

    vfirst = None
    for loop in range(cfg.loops):
        ln1 = rms(x, W["n1"])
        q = (ln1 @ W["wq"].T).reshape(B, T, H, D)
        k = (ln1 @ W["wk"].T).reshape(B, T, 1, D)
        v = ln1 @ W["wv"].T
        if loop == 0:
            vfirst = v
        else:
            v = (1 - cfg.mix) * v + cfg.mix * vfirst
        q = rope(q).transpose(0, 2, 1, 3)
        k = rope(k).transpose(0, 2, 1, 3)
        v = v.reshape(B, T, 1, D).transpose(0, 2, 1, 3)
        sc = q @ k.transpose(0, 1, 3, 2) / math.sqrt(D)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        av = (p @ v).transpose(0, 2, 1, 3).reshape(M, C)
        mid = x + rms(av @ W["wo"].T, W["n1b"])
        ln2 = rms(mid, W["n2"])
        gt, up = ln2 @ W["wgate"].T, ln2 @ W["wup"].T
        sw = gt / (1 + np.exp(-gt)) * up
        pre = mid + rms(sw @ W["wdown"].T, W["n2b"])
        x = rms(pre, W["nf"])
    return x


@pytest.mark.parametrize("bits", [8, 4])
def test_dit_block_forward_float64(orc, bits):
    cfg = orc.DiTCfg(B=2, T=8, C=32, F=64, H=4, D=8, loops=3, group=16, bits=bits)
    rng = orc.RNG(456)
    shapes = {"wq": (32, 32), "wk": (8, 32), "wv": (8, 32), "wo": (32, 32),
              "wgate": (64, 32), "wup": (64, 32), "wdown": (32, 64)}
    qw, W = {}, {}
    for name, (n, k) in shapes.items():
        w = rng.randn(n * k, 0.2)
        q, s = orc.quant(w, n, k, cfg.group, bits)
        qw[name] = (q, s)
        W[name] = orc.dequant(q, s, n, k, cfg.group, bits).reshape(n, k).astype(np.float64)
    for name in orc.DIT_NORMS:
        qw[name] = (1.0 + 0.1 * rng.randn(cfg.C, 1.0)).astype(np.float32)
        W[name] = qw[name].astype(np.float64)
    x0 = rng.randn(cfg.B * cfg.T * cfg.C, 1.0)
    got = orc.dit_forward(cfg, qw, x0)
    ref = _dit_float64(cfg, W, x0.reshape(-1, cfg.C).astype(np.float64))
    assert _rel(got, ref.ravel()) < 1e-5
