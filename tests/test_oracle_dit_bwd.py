"""Pins the oracle's DiT block backward (CPU only).

orc_dit_train restates the reference's loop backward (src/DiT.swift:566-626)
kernel by kernel (metal/kernels.metal:508-612, 827-868, 891-1010). It is
checked against torch autograd in float64 of the same block forward written
as whole-tensor operations (not the kernels' loops), and its pieces against
closed forms: the RMSNorm backward of a unit-RMS row, RoPE's backward as the
transpose of the forward rotation, SwiGLU's derivative at 0, the attention
backward against autograd of softmax attention.
"""
from __future__ import annotations

import numpy as np
import pytest


def _torch():
    import torch
    return torch


def _block_t64(cfg, Wd, Nd, x0, cos, sin):
    """The looped block forward (src/DiT.swift:520-550) in float64 torch ops."""
    torch = _torch()
    B, T, C, H, D, mix, eps = cfg.B, cfg.T, cfg.C, cfg.H, cfg.D, cfg.mix, cfg.eps
    cos = torch.from_numpy(cos.astype(np.float64)).view(T, D)
    sin = torch.from_numpy(sin.astype(np.float64)).view(T, D)

    def rms(x, w):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w

    def rope(x):   # x [B, T, h, D]; rotate-half
        half = D // 2
        rot = torch.cat([-x[..., half:], x[..., :half]], -1)
        return x * cos[None, :, None, :] + rot * sin[None, :, None, :]

    x = x0.view(B * T, C)
    vfirst = None
    for _ in range(cfg.loops):
        ln1 = rms(x, Nd["n1"])
        q = ln1 @ Wd["wq"].T
        k = ln1 @ Wd["wk"].T
        v = ln1 @ Wd["wv"].T
        if vfirst is None:
            vfirst, vm = v, v
        else:
            vm = (1 - mix) * v + mix * vfirst
        qh = rope(q.view(B, T, H, D))
        kh = rope(k.view(B, T, 1, D)).expand(B, T, H, D)
        vh = vm.view(B, T, 1, D).expand(B, T, H, D)
        sc = torch.einsum("bthd,bshd->bhts", qh, kh) / np.sqrt(D)
        pr = torch.softmax(sc, -1)
        av = torch.einsum("bhts,bshd->bthd", pr, vh).reshape(B * T, C)
        attn = av @ Wd["wo"].T
        mid = x + rms(attn, Nd["n1b"])
        ln2 = rms(mid, Nd["n2"])
        g = ln2 @ Wd["wgate"].T
        u = ln2 @ Wd["wup"].T
        sw = g * torch.sigmoid(g) * u
        mlp = sw @ Wd["wdown"].T
        pre = mid + rms(mlp, Nd["n2b"])
        x = rms(pre, Nd["nf"])
    return x


def _rel(a, b):
    b = np.asarray(b, np.float64).ravel()
    return float(np.max(np.abs(np.asarray(a, np.float64).ravel() - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.parametrize("bits", [32, 8])
def test_dit_train_matches_float64_autograd(orc, bits):
    torch = _torch()
    cfg = orc.DiTCfg(B=2, T=8, C=32, F=64, H=4, D=8, loops=3, group=8, bits=bits)
    shapes = {"wq": (32, 32), "wk": (8, 32), "wv": (8, 32), "wo": (32, 32), "wgate": (64, 32),
              "wup": (64, 32), "wdown": (32, 64)}
    rng = orc.RNG(77 + bits)
    masters = {n: rng.randn(r * c_, 0.2) for n, (r, c_) in shapes.items()}
    norms = {n: (1.0 + 0.1 * rng.randn(cfg.C, 1.0)).astype(np.float32) for n in orc.DIT_NORMS}
    x0 = rng.randn(cfg.B * cfg.T * cfg.C, 1.0)
    gy = rng.randn(cfg.B * cfg.T * cfg.C, 1.0)
    if bits == 32:
        lin, eff = masters, masters
    else:
        lin = {n: orc.quant(masters[n], *shapes[n], cfg.group, bits) for n in shapes}
        eff = {n: orc.dequant(*lin[n], *shapes[n], cfg.group, bits) for n in shapes}
    xo, gx, gw, gn = orc.dit_train(cfg, lin, norms, x0, gy)

    cos, sin = orc.rope_tables(cfg.T, cfg.D, cfg.theta)
    Wd = {n: torch.tensor(eff[n].astype(np.float64).reshape(shapes[n]), requires_grad=True) for n in shapes}
    Nd = {n: torch.tensor(norms[n].astype(np.float64), requires_grad=True) for n in orc.DIT_NORMS}
    xt = torch.tensor(x0.astype(np.float64), requires_grad=True)
    out = _block_t64(cfg, Wd, Nd, xt, cos, sin)
    (out.reshape(-1) * torch.from_numpy(gy.astype(np.float64))).sum().backward()
    assert _rel(xo, out.detach().numpy()) <= 1e-5
    assert _rel(gx, xt.grad.numpy()) <= 1e-5
    for n in shapes:
        assert _rel(gw[n], Wd[n].grad.numpy()) <= 1e-5, n
    for n in orc.DIT_NORMS:
        assert _rel(gn[n], Nd[n].grad.numpy()) <= 1e-5, n


def test_rms_bwd_closed_forms(orc):
    # A unit-RMS row with unit weight and eps = 0: rstd = 1, and for dy = x the
    # input gradient vanishes (x is its own normalization's radial direction).
    C = 16
    x = np.where(np.arange(C) % 2 == 0, 1.0, -1.0).astype(np.float32)
    dx, dw = orc.rms_bwd(x, np.ones(1, np.float32), np.ones(C, np.float32), x, np.zeros(C, np.float32), 1, C)
    assert np.array_equal(dx, np.zeros(C, np.float32))
    assert np.array_equal(dw, np.ones(C, np.float32))          # dy*x*rstd = 1
    # A gradient orthogonal to x passes scaled by rstd * weight.
    dy = np.zeros(C, np.float32)
    dy[0], dy[2] = 1.0, -1.0
    dx, _ = orc.rms_bwd(x, np.full(1, 0.5, np.float32), np.full(C, 2.0, np.float32), dy, np.zeros(C, np.float32), 1, C)
    assert np.array_equal(dx, dy * np.float32(1.0))


def test_rope_bwd_is_transpose(orc):
    # <rope(x), y> == <x, rope_bwd(y)> for the same tables (exact up to fp32 rounding).
    B, T, H, D = 2, 5, 3, 8
    cos, sin = orc.rope_tables(T, D, 1e4)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(B * T * H * D).astype(np.float32)
    y = rng.standard_normal(B * T * H * D).astype(np.float32)
    lhs = float(np.dot(orc.rope_fwd(x, cos, sin, B, T, H, D).astype(np.float64), y))
    rhs = float(np.dot(x.astype(np.float64), orc.rope_bwd(y, cos, sin, B, T, H, D)))
    assert abs(lhs - rhs) <= 1e-5 * max(abs(lhs), 1.0)


def test_swiglu_bwd_values(orc):
    dg, du = orc.swiglu_bwd(np.zeros(3, np.float32), np.array([1, 2, 3], np.float32), np.ones(3, np.float32))
    # silu'(0) = 1/2, silu(0) = 0.
    assert np.array_equal(dg, np.array([0.5, 1.0, 1.5], np.float32)) and not du.any()
    z = np.linspace(-6, 6, 41).astype(np.float32)
    dg, du = orc.swiglu_bwd(z, np.ones_like(z), np.ones_like(z))
    z64 = z.astype(np.float64)
    s = 1 / (1 + np.exp(-z64))
    assert np.max(np.abs(dg - s * (1 + z64 * (1 - s)))) <= 2e-6
    assert np.max(np.abs(du - z64 * s)) <= 2e-6


def test_attn_bwd_matches_autograd(orc):
    torch = _torch()
    B, T, H, D = 2, 6, 3, 4
    rng = np.random.default_rng(2)
    q, k, v, dout = (rng.standard_normal(B * T * H * D).astype(np.float32) for _ in range(4))
    _, probs, _ = orc.attn_fwd(q, k, v, B, T, H, D, 0)
    dq, dk, dv, dp, ds = orc.attn_bwd(q, k, v, probs, dout, B, T, H, D)
    Q, K, V = (torch.tensor(a.astype(np.float64).reshape(B, T, H, D), requires_grad=True) for a in (q, k, v))
    sc = torch.einsum("bthd,bshd->bhts", Q, K) / np.sqrt(D)
    out = torch.einsum("bhts,bshd->bthd", torch.softmax(sc, -1), V)
    (out * torch.from_numpy(dout.astype(np.float64).reshape(B, T, H, D))).sum().backward()
    for got, ref in ((dq, Q.grad), (dk, K.grad), (dv, V.grad)):
        assert _rel(got, ref.numpy()) <= 1e-5
    # dscores rows of a softmax Jacobian sum to zero.
    assert np.max(np.abs(ds.reshape(-1, T).astype(np.float64).sum(1))) <= 1e-5


def test_sum_heads_and_acc_scale(orc):
    B, T, H, D = 2, 3, 4, 5
    src = np.arange(B * T * H * D, dtype=np.float32)
    got = orc.sum_heads(src, B, T, H, D)
    assert np.array_equal(got, src.reshape(B, T, H, D).astype(np.float64).sum(2).reshape(-1).astype(np.float32))
    a = np.array([1.0, 2.0], np.float32)
    assert np.array_equal(orc.acc_scale(a, np.array([4.0, 8.0], np.float32), 0.25), np.array([2.0, 4.0], np.float32))
