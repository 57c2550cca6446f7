"""Pins the oracle's training-step functions (CPU only).

The reference holds no stored vectors for these kernels, so each oracle
function is checked against what the mathematics fixes: hand-derived exact
steps, integer-valued inputs whose sums are exact in any order, an independent
library routine (torch.optim.AdamW in float64, numpy scatter-add), and the
reference's own checkEmbed case (src/Check.swift:312-340).
"""
from __future__ import annotations

import numpy as np
import pytest


def _bc(b1, b2, step):
    # GPT.step (src/GPT.swift:205-206): invBC = 1 / (1 - b^step), in fp32.
    f = np.float32
    return f(1) / (f(1) - f(b1) ** f(step)), f(1) / (f(1) - f(b2) ** f(step))


def test_adamw_exact_first_step(orc):
    # b1 = 1/2, b2 = 3/4, eps = 0: from m = v = 0 the bias-corrected moments of a
    # power-of-two gradient are g and g^2 exactly, so the update is exactly
    # sign(g); with power-of-two lr, wd and w the new weight is exact too.
    g = np.array([2.0 ** -3, -2.0 ** 5, 1.0, -2.0 ** -20], np.float32)
    w = np.array([1.0, -0.5, 2.0 ** -4, 8.0], np.float32)
    z = np.zeros(4, np.float32)
    lr, wd = 2.0 ** -6, 2.0 ** -2
    w1, m1, v1 = orc.adamw(w, g, z, z, lr, 0.5, 0.75, 0.0, wd, 2.0, 4.0)
    assert np.array_equal(m1, 0.5 * g) and np.array_equal(v1, 0.25 * g * g)
    assert np.array_equal(w1, (w - lr * (np.sign(g) + wd * w)).astype(np.float32))


def test_adamw_pure_decay_and_zero_grad(orc):
    w = np.array([1.0, -3.0, 0.25, 0.0], np.float32)
    z = np.zeros(4, np.float32)
    # g = 0, m = v = 0: upd = 0 / (0 + eps) = 0 and only the decoupled decay acts.
    w1, m1, v1 = orc.adamw(w, z, z, z, 0.125, 0.9, 0.95, 1e-8, 0.5, 10.0, 20.0)
    assert np.array_equal(w1, w - np.float32(0.125) * (np.float32(0.5) * w))
    assert not m1.any() and not v1.any()
    w2, _, _ = orc.adamw(w, z, z, z, 0.125, 0.9, 0.95, 1e-8, 0.0, 10.0, 20.0)
    assert np.array_equal(w2, w)


def test_adamw_matches_torch_adamw(orc):
    # torch.optim.AdamW (decoupled decay applied to the pre-update weight, bias
    # corrections 1 - b^t) is the same update in exact arithmetic.
    import torch
    rng = np.random.default_rng(3)
    n, lr, b1, b2, eps, wd = 513, 3e-3, 0.9, 0.95, 1e-8, 0.1
    w = rng.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    p = torch.nn.Parameter(torch.from_numpy(w.astype(np.float64)))
    opt = torch.optim.AdamW([p], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    for step in range(1, 6):
        g = rng.standard_normal(n).astype(np.float32)
        bc1, bc2 = _bc(b1, b2, step)
        w, m, v = orc.adamw(w, g, m, v, lr, b1, b2, eps, wd, bc1, bc2)
        p.grad = torch.from_numpy(g.astype(np.float64))
        opt.step()
        ref = p.detach().numpy()
        assert np.max(np.abs(w - ref)) <= 1e-5 * np.max(np.abs(ref)), step
    st = opt.state[p]
    assert np.allclose(m, st["exp_avg"].numpy(), rtol=1e-5, atol=1e-7)
    assert np.allclose(v, st["exp_avg_sq"].numpy(), rtol=1e-5, atol=1e-9)


def test_adam_quantize_is_adamw_then_quant(orc):
    rng = np.random.default_rng(4)
    rows, cols, G = 6, 64, 16
    w = (0.05 * rng.standard_normal(rows * cols)).astype(np.float32)
    g = rng.standard_normal(rows * cols).astype(np.float32)
    z = np.zeros_like(w)
    for bits in (8, 4):
        w1, m1, v1, q, s = orc.adam_quantize(w, g, z, z, rows, cols, G, bits, 1e-2, 0.9, 0.95, 1e-8, 0.1,
                                             10.0, 20.0)
        w2, _, _ = orc.adamw(w, g, z, z, 1e-2, 0.9, 0.95, 1e-8, 0.1, 10.0, 20.0)
        assert np.array_equal(w1, w2)
        deq = orc.dequant(q, s, rows, cols, G, bits)
        lim = 7 if bits == 4 else 127
        s_rep = np.repeat(s, G)
        assert np.all(np.abs(deq - w1) <= s_rep / 2 * (1 + 1e-6))
        assert np.array_equal(s, np.maximum(np.abs(w1).reshape(-1, G).max(1) / np.float32(lim),
                                            np.float32(1e-8)).astype(np.float32))


def test_reduce_sumsq(orc):
    # Integer squares whose every partial sum stays below 2^24: exact in any order.
    x = (np.arange(3000) % 17 - 8).astype(np.float32)
    assert orc.reduce_sumsq(x) == float(np.sum(x.astype(np.int64) ** 2))
    assert orc.reduce_sumsq(np.zeros(0, np.float32)) == 0.0
    rng = np.random.default_rng(5)
    y = rng.standard_normal(100003).astype(np.float32)
    ref = float(np.sum(y.astype(np.float64) ** 2))
    assert abs(orc.reduce_sumsq(y) - ref) <= 1e-5 * ref


def test_scale(orc):
    x = np.array([1.0, -2.0, 3.5], np.float32)
    assert np.array_equal(orc.scale(x, 0.5), x * np.float32(0.5))


def _check_embed_case():
    # src/Check.swift:312-327: B 2, T 3, C 8, V 4, G 8, RNG(5), std 0.4 / 0.2.
    return 2, 3, 8, 4, 8, np.array([1, 0, 3, 1, 2, 0], np.uint32)


def test_embed_reference_check(orc):
    B, T, C, V, G, toks = _check_embed_case()
    rng = orc.RNG(5)
    master = rng.randn(V * C, 0.4)
    wpe = rng.randn(T * C, 0.2)
    q, s = orc.quant(master, V, C, G, 8)
    y = orc.embed(toks, None, q, s, wpe, B, T, C, G, 8)
    # Check.swift:331-337 (one group per row since C == G).
    expect = np.zeros(B * T * C, np.float32)
    for bt in range(B * T):
        tok, t = int(toks[bt]), bt % T
        expect[bt * C:(bt + 1) * C] = q[tok * C:(tok + 1) * C].astype(np.float32) * s[tok] + wpe[t * C:(t + 1) * C]
    assert np.max(np.abs(y - expect)) < 1e-5
    assert np.array_equal(y, expect)


@pytest.mark.parametrize("bits", [32, 8, 4])
def test_embed_one_hot_rows(orc, bits):
    # Table row v holds the value v + 1 (exactly representable after quantizing:
    # every group is constant, so s = (v+1)/qmax and the code is qmax);
    # wpe row t holds 100 * t. y[bt, c] must be (tok + 1) + 100 * (bt % T).
    B, T, C, V, G = 3, 5, 16, 7, 8
    table = np.repeat(np.arange(1, V + 1, dtype=np.float32), C)
    wpe = np.repeat(100.0 * np.arange(T, dtype=np.float32), C)
    toks = np.array([(3 * i + 1) % V for i in range(B * T)], np.uint32)
    if bits == 32:
        y = orc.embed(toks, table, None, None, wpe, B, T, C, G, 32)
    else:
        q, s = orc.quant(table, V, C, G, bits)
        y = orc.embed(toks, None, q, s, wpe, B, T, C, G, bits)
    want = np.repeat((toks.astype(np.float64) + 1) + 100.0 * (np.arange(B * T) % T), C)
    assert np.allclose(y, want, rtol=1e-6, atol=0)


def test_embed_bwd_scatter_add(orc):
    rng = np.random.default_rng(6)
    B, T, C, V = 4, 16, 24, 9
    toks = rng.integers(0, V, B * T).astype(np.uint32)
    dx = rng.integers(-50, 50, B * T * C).astype(np.float32)     # integer: exact sums
    dwe = rng.integers(-9, 9, V * C).astype(np.float32)
    got = orc.embed_bwd(toks, dx, dwe, B, T, C, V)
    ref = dwe.reshape(V, C).astype(np.float64).copy()
    np.add.at(ref, toks.astype(np.int64), dx.reshape(B * T, C).astype(np.float64))
    assert np.array_equal(got, ref.reshape(-1).astype(np.float32))
    # Real values: float64 scatter-add to fp32 rounding.
    dxr = rng.standard_normal(B * T * C).astype(np.float32)
    got = orc.embed_bwd(toks, dxr, np.zeros(V * C, np.float32), B, T, C, V)
    ref = np.zeros((V, C))
    np.add.at(ref, toks.astype(np.int64), dxr.reshape(B * T, C).astype(np.float64))
    assert np.max(np.abs(got - ref.reshape(-1))) <= 1e-5 * np.max(np.abs(ref))


def test_pos_bwd_and_bias_grad(orc):
    rng = np.random.default_rng(7)
    B, T, C = 5, 7, 12
    dx = rng.integers(-100, 100, B * T * C).astype(np.float32)
    got = orc.pos_bwd(dx, B, T, C)
    assert np.array_equal(got, dx.reshape(B, T * C).astype(np.float64).sum(0).astype(np.float32))
    M, N = 37, 11
    dy = rng.integers(-100, 100, M * N).astype(np.float32)
    assert np.array_equal(orc.bias_grad(dy, M, N), dy.reshape(M, N).astype(np.float64).sum(0).astype(np.float32))
    dyr = rng.standard_normal(M * N).astype(np.float32)
    ref = dyr.reshape(M, N).astype(np.float64).sum(0)
    assert np.max(np.abs(orc.bias_grad(dyr, M, N) - ref)) <= 1e-5 * np.max(np.abs(ref))
