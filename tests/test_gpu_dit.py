"""GPU parity of the looped DiT block forward (src/DiT.swift:520-550) and of the
non-GEMM wrappers it calls (src/GPU.swift:211-410), through the C ABI, against
the CPU oracle on the same inputs.

Bars:
  * repeatHeads, copy, add, mix, ropeFwd: bit-exact (one rounding per product
    and sum, the same operations in the same order as the oracle);
  * rmsFwd: max rel error <= 2e-6 (the sum of squares is reduced across a
    wave, not sequentially);
  * swigluFwd: <= 2e-6 (device expf);
  * attnFwd: probs and av <= 1e-5, scores <= 1e-5 (dot products in the
    reference's sequential d order, then the same scale);
  * the whole block (c3: 8x64 tokens, embd 192, 4 loops, int8 group-32
    linears): xs[4] within max relative error 1e-5 of the oracle's forward in
    the Metal kernel order.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, rel_err, to_dev

pytestmark = pytest.mark.gpu


def _run(gpu, fn):
    gpu.begin()
    fn()
    gpu.end()


@pytest.mark.parametrize("rows,cols", [(512, 192), (3, 768), (1, 1), (70, 65), (5, 1000)])
def test_rms_fwd(gpu, orc, rows, cols):
    import torch
    rng = np.random.default_rng(rows * 7 + cols)
    x = (rng.standard_normal(rows * cols) * rng.choice([1e-3, 1.0, 30.0])).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    y = torch.full((rows * cols,), float("nan"), device="cuda")
    rstd = torch.full((rows,), float("nan"), device="cuda")
    xd, wd = to_dev(x), to_dev(w)
    _run(gpu, lambda: gpu.rmsFwd(xd, y, rstd, wd, rows, cols, 1e-6))
    ry, rr = orc.rmsnorm_fwd(x, w, rows, cols, 1e-6)
    assert rel_err(from_dev(y), ry) <= 2e-6
    assert rel_err(from_dev(rstd), rr) <= 2e-6


@pytest.mark.parametrize("B,T,H,D", [(8, 64, 4, 48), (8, 64, 1, 48), (2, 5, 3, 2), (1, 1, 1, 8), (3, 17, 2, 10)])
def test_rope_fwd_bit_exact(gpu, dgm, orc, B, T, H, D):
    import torch
    cos, sin = dgm.rope_tables(T, D, 1e4)
    rng = np.random.default_rng(B + T + H + D)
    x = rng.standard_normal(B * T * H * D).astype(np.float32)
    y = torch.full((x.size,), float("nan"), device="cuda")
    xd, cd, sd = to_dev(x), to_dev(cos), to_dev(sin)
    _run(gpu, lambda: gpu.ropeFwd(xd, y, cd, sd, B, T, H, D))
    ref = orc.rope_fwd(x, cos, sin, B, T, H, D)
    assert np.array_equal(from_dev(y), ref)


def test_repeat_copy_add_mix_bit_exact(gpu, orc):
    import torch
    B, T, H, D = 8, 64, 4, 48
    rng = np.random.default_rng(9)
    src = rng.standard_normal(B * T * D).astype(np.float32)
    a = rng.standard_normal(1000).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    dst = torch.full((B * T * H * D,), float("nan"), device="cuda")
    cp = torch.full((1000,), float("nan"), device="cuda")
    ad = torch.full((1000,), float("nan"), device="cuda")
    mx = torch.full((1000,), float("nan"), device="cuda")
    s_d, a_d, b_d = to_dev(src), to_dev(a), to_dev(b)

    def go():
        gpu.repeatHeads(s_d, dst, B, T, H, D)
        gpu.copy(a_d, cp, 1000)
        gpu.add(a_d, b_d, ad, 1000)
        gpu.mix(a_d, b_d, mx, 1000, 0.25, 0.75)
    _run(gpu, go)
    assert np.array_equal(from_dev(dst), orc.repeat_heads(src, B, T, H, D))
    assert np.array_equal(from_dev(cp), a)
    assert np.array_equal(from_dev(ad), a + b)
    assert np.array_equal(from_dev(mx), orc.mix(a, b, 0.25, 0.75))


def test_swiglu_fwd(gpu, orc):
    import torch
    rng = np.random.default_rng(10)
    n = 512 * 768 + 3
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    g[:4] = [0.0, -0.0, 90.0, -90.0]
    u = rng.standard_normal(n).astype(np.float32)
    y = torch.full((n,), float("nan"), device="cuda")
    gd, ud = to_dev(g), to_dev(u)
    _run(gpu, lambda: gpu.swigluFwd(gd, ud, y, n))
    assert rel_err(from_dev(y), orc.swiglu_fwd(g, u)) <= 2e-6


@pytest.mark.parametrize("B,T,H,D,causal", [(8, 64, 4, 48, 0), (2, 64, 4, 48, 1), (1, 17, 3, 10, 0),
                                            (2, 33, 2, 16, 1), (1, 1, 1, 4, 0), (1, 128, 2, 64, 0)])
def test_attn_fwd(gpu, orc, B, T, H, D, causal):
    import torch
    rng = np.random.default_rng(B * 100 + T + H + D + causal)
    q, k, v = (rng.standard_normal(B * T * H * D).astype(np.float32) for _ in range(3))
    sc = torch.full((B * H * T * T,), float("nan"), device="cuda")
    pr = torch.full((B * H * T * T,), float("nan"), device="cuda")
    av = torch.full((B * T * H * D,), float("nan"), device="cuda")
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    _run(gpu, lambda: gpu.attnFwd(qd, kd, vd, sc, pr, av, B, T, H, D, causal=bool(causal)))
    rs, rp, ra = orc.attn_fwd(q, k, v, B, T, H, D, causal)
    assert rel_err(from_dev(sc), rs) <= 1e-5
    assert rel_err(from_dev(pr), rp) <= 1e-5
    assert rel_err(from_dev(av), ra) <= 1e-5
    if causal:
        assert np.all(np.triu(from_dev(pr).reshape(B, H, T, T), 1) == 0)


def test_attn_rejects_oversized_tile(gpu, dgm):
    import torch
    t = torch.zeros(16, device="cuda")
    gpu.begin()
    with pytest.raises(dgm.DgmError) as e:
        gpu.attnFwd(t, t, t, t, t, t, 1, 2048, 1, 16, causal=False)
    assert e.value.code == dgm.DGM_ERR_UNSUPPORTED
    with pytest.raises(dgm.DgmError):
        gpu.end()


def _dit_weights(orc, cfg, seed=456):
    """DiT init (src/DiT.swift:308-316): RNG(seed), std 0.02, in the order
    wPatch [C,P], wHead [P,C], wTime1 [C,freq], wTime2 [C,C], then the block's
    linears; norms = 1. photos-dit: P = 16*16*3, freq = 192."""
    rng = orc.RNG(seed)
    P, freq, C = 16 * 16 * 3, 192, cfg.C
    for n in (C * P, P * C, C * freq, C * C):
        rng.randn(n, 0.02)
    shapes = cfg.linear_shapes()
    w = {name: rng.randn(shapes[name][0] * shapes[name][1], 0.02) for name in orc.DIT_LINEARS}
    for name in orc.DIT_NORMS:
        w[name] = np.ones(C, dtype=np.float32)
    return w


def _oracle_forward(orc, cfg, w, x0, codes):
    ocfg = orc.DiTCfg(B=cfg.B, T=cfg.T, C=cfg.C, F=cfg.F, H=cfg.H, D=cfg.D, loops=cfg.loops,
                      group=cfg.group, bits=cfg.bits, eps=cfg.eps, theta=cfg.theta, mix=cfg.mix)
    qw = dict(codes)
    for name in orc.DIT_NORMS:
        qw[name] = w[name]
    return orc.dit_forward(ocfg, qw, x0)


def _check_block(gpu, dgm, orc, cfg, w, x0, bar):
    import torch
    dev = {k: to_dev(v) for k, v in w.items()}
    blk = dgm.DiTBlock(gpu, cfg, dev)
    codes = {}
    for name in orc.DIT_LINEARS:
        N, K = cfg.linear_shapes()[name]
        q, s = orc.quant(w[name], N, K, cfg.group, cfg.bits)
        gq = from_dev(blk.codes[name])[: q.size]
        assert np.array_equal(gq.view(q.dtype), q), name           # quantized once, bit-exact
        assert np.array_equal(from_dev(blk.scales[name])[: s.size], s), name
        codes[name] = (q, s)
    x = to_dev(x0)
    gpu.begin()
    blk.forward(x)
    gpu.end()
    ref = _oracle_forward(orc, cfg, w, x0, codes)
    err = rel_err(from_dev(x), ref)
    assert err <= bar, err
    # Re-running on the same input reproduces the result bit for bit.
    x2 = to_dev(x0)
    gpu.begin()
    blk.forward(x2)
    gpu.end()
    assert torch.equal(x, x2)
    return blk, x


def test_config3_dit_block_forward(gpu, dgm, orc):
    """c3: photos-dit looped block, 8x64 tokens, embd 192, SwiGLU 768, 4 loops,
    int8 group-32 linears, RNG(456) init, xs[0] ~ N(0,1)."""
    cfg = dgm.DiTConfig()
    w = _dit_weights(orc, cfg)
    x0 = orc.RNG(1003).randn(cfg.B * cfg.T * cfg.C, 1.0)
    blk, x = _check_block(gpu, dgm, orc, cfg, w, x0, 1e-5)
    # The workspace keeps the last loop's probabilities: rows sum to one.
    probs = from_dev(blk.workspace_view("probs")).reshape(cfg.B, cfg.H, cfg.T, cfg.T)
    assert np.allclose(probs.sum(-1), 1.0, atol=1e-5)


@pytest.mark.parametrize("B,loops,bits", [(8, 4, 4), (3, 2, 8), (11, 1, 8), (1, 3, 4)])
def test_dit_block_c3_shape_variants(gpu, dgm, orc, B, loops, bits):
    """The c3 block shape (T 64, embd 192, 4 heads of 48, SwiGLU 768, group
    32) at other batch sizes (sequences per XCD: none, one or two), loop
    counts and int4 linears."""
    cfg = dgm.DiTConfig(B=B, loops=loops, bits=bits)
    w = _dit_weights(orc, cfg, seed=31 + B)
    x0 = orc.RNG(1000 + B).randn(cfg.B * cfg.T * cfg.C, 1.0)
    _check_block(gpu, dgm, orc, cfg, w, x0, 1e-5)


@pytest.mark.parametrize("bits,group", [(4, 32), (32, 32)])
def test_dit_block_other_widths(gpu, dgm, orc, bits, group):
    cfg = dgm.DiTConfig(B=2, T=16, C=64, F=128, H=4, D=16, loops=3, group=group, bits=bits)
    w = _dit_weights(orc, cfg, seed=7)
    x0 = orc.RNG(8).randn(cfg.B * cfg.T * cfg.C, 1.0)
    if bits == 32:
        import torch
        blk = dgm.DiTBlock(gpu, cfg, {k: to_dev(v) for k, v in w.items()})
        x = to_dev(x0)
        gpu.begin()
        blk.forward(x)
        gpu.end()
        # fp32 linears: the oracle's quantized forward does not apply; compare with
        # the float64 statement of the block on the fp32 weights.
        from test_oracle import _dit_float64
        W = {k: (v.reshape(cfg.linear_shapes()[k]) if k in cfg.linear_shapes() else v).astype(np.float64)
             for k, v in w.items()}
        ref = _dit_float64(cfg, W, x0.reshape(-1, cfg.C).astype(np.float64))
        assert rel_err(from_dev(x), ref.ravel()) <= 1e-5
        assert torch.isfinite(x).all()
    else:
        _check_block(gpu, dgm, orc, cfg, w, x0, 1e-5)


def test_dit_forward_separate_weight_buffers(gpu, dgm, orc):
    """Linears in unrelated allocations (not back to back): the projections run
    as separate GEMMs; the result still matches the oracle."""
    import torch
    cfg = dgm.DiTConfig(B=2, T=32, C=96, F=192, H=2, D=48, loops=2, group=32, bits=8)
    w = _dit_weights(orc, cfg, seed=11)
    x0 = orc.RNG(12).randn(cfg.B * cfg.T * cfg.C, 1.0)
    keep, lins, codes = [], {}, {}
    gpu.begin()
    for name in orc.DIT_LINEARS:
        N, K = cfg.linear_shapes()[name]
        pad = torch.zeros(4096, dtype=torch.uint8, device="cuda")     # keeps allocations apart
        q = torch.zeros(N * K, dtype=torch.int8, device="cuda")
        s = torch.zeros(N * (K // cfg.group), device="cuda")
        wd = to_dev(w[name])
        gpu.quantize(wd, q, s, N, K, 8, cfg.group)
        keep += [pad, q, s, wd]
        lins[name] = dgm.DiTLinear(None, q.data_ptr(), s.data_ptr())
    gpu.end()
    for name in orc.DIT_LINEARS:
        N, K = cfg.linear_shapes()[name]
        codes[name] = orc.quant(w[name], N, K, cfg.group, 8)
    norms = {n: to_dev(w[n]) for n in orc.DIT_NORMS}
    wts = dgm.DiTWeights(*[lins[n] for n in orc.DIT_LINEARS], *[norms[n].data_ptr() for n in orc.DIT_NORMS])
    c = cfg.c_cfg()
    cos, sin = dgm.rope_tables(cfg.T, cfg.D, cfg.theta)
    cd, sd = to_dev(cos), to_dev(sin)
    nws = gpu.dit_workspace_floats(c)
    ws = torch.zeros(nws, device="cuda")
    x = to_dev(x0)
    gpu.begin()
    gpu.dit_forward(c, wts, cd, sd, x, ws, nws)
    gpu.end()
    ref = _oracle_forward(orc, cfg, w, x0, codes)
    assert rel_err(from_dev(x), ref) <= 1e-5


def test_dit_forward_rejects_bad_config(gpu, dgm):
    import torch
    cfg = dgm.DiTConfig(B=1, T=4, C=30, F=32, H=4, D=8, group=8)   # C != H*D
    c = cfg.c_cfg()
    wts = dgm.DiTWeights()
    t = torch.zeros(1024, device="cuda")
    gpu.begin()
    with pytest.raises(dgm.DgmError) as e:
        gpu.dit_forward(c, wts, t, t, t, t, 1024)
    assert e.value.code == dgm.DGM_ERR_SHAPE
    with pytest.raises(dgm.DgmError):
        gpu.end()
