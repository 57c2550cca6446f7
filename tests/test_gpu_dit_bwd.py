"""GPU parity of the DiT block backward (src/DiT.swift:558-626) through the C ABI.

Per wrapper against the CPU oracle: attnBwd (metal/kernels.metal:508-612),
ropeBwd, sumHeads, acc, accScale bit-exact; rmsBwd (827-868, wave-reduced
row sums) <= 1e-5; swigluBwd (932-949, device expf) <= 2e-6. The block's
training forward and backward against orc_dit_train (itself pinned to float64
autograd): max relative error <= 1e-5 for xs[loops], dL/dxs[0] and every
parameter gradient, at c3 (int8 G=32) and small configs (fp32, int8, int4).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, rel_err, to_dev

pytestmark = pytest.mark.gpu


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(1, 8), (512, 192), (37, 100), (64, 1024)])
def test_rms_bwd(gpu, orc, rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal(rows * cols).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    dy = rng.standard_normal(rows * cols).astype(np.float32)
    _, rstd = orc.rmsnorm_fwd(x, w, rows, cols, 1e-6)
    dw0 = rng.standard_normal(cols).astype(np.float32)
    dxd, dwd = to_dev(np.zeros(rows * cols, np.float32)), to_dev(dw0)
    gpu.begin()
    gpu.rmsBwd(to_dev(x), to_dev(rstd), to_dev(w), to_dev(dy), dxd, dwd, rows, cols, 1e-6)
    gpu.end()
    rdx, rdw = orc.rms_bwd(x, rstd, w, dy, dw0, rows, cols)
    assert rel_err(from_dev(dxd), rdx) <= 1e-5
    assert rel_err(from_dev(dwd) - dw0, rdw.astype(np.float64) - dw0) <= 1e-5
    assert gpu.lastKernel == "rmsnorm_bwd"


# T % 8 == 0: the two-launch split kernels; T % 4 == 0 (12): the one-workgroup-
# per-head kernel; others: the five passes.
@pytest.mark.parametrize("B,T,H,D", [(8, 64, 4, 48), (2, 32, 2, 12), (2, 12, 3, 8), (2, 5, 3, 4), (1, 17, 2, 10)])
def test_attn_bwd_bitexact(gpu, orc, B, T, H, D):
    import torch
    rng = np.random.default_rng(B * T + H * D)
    n, tt = B * T * H * D, B * H * T * T
    q, k, v, dout = (rng.standard_normal(n).astype(np.float32) for _ in range(4))
    _, probs, _ = orc.attn_fwd(q, k, v, B, T, H, D, 0)
    outs = [torch.zeros(m, dtype=torch.float32, device="cuda") for m in (n, n, n, tt, tt)]
    gpu.begin()
    gpu.attnBwd(to_dev(q), to_dev(k), to_dev(v), to_dev(probs), to_dev(dout), *outs, B, T, H, D)
    gpu.end()
    refs = orc.attn_bwd(q, k, v, probs, dout, B, T, H, D)
    for name, got, ref in zip(("dq", "dk", "dv", "dprobs", "dscores"), outs, refs):
        assert _same(from_dev(got), ref), name


@pytest.mark.parametrize("B,T,H,D", [(8, 64, 4, 48), (8, 64, 1, 48), (3, 7, 2, 6)])
def test_rope_bwd_and_sum_heads_bitexact(gpu, orc, B, T, H, D):
    import torch
    cos, sin = orc.rope_tables(T, D, 1e4)
    rng = np.random.default_rng(T * D + H)
    dy = rng.standard_normal(B * T * H * D).astype(np.float32)
    dx = torch.zeros(B * T * H * D, dtype=torch.float32, device="cuda")
    s = torch.zeros(B * T * D, dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.ropeBwd(to_dev(dy), dx, to_dev(cos), to_dev(sin), B, T, H, D)
    gpu.sumHeads(to_dev(dy), s, B, T, H, D)
    gpu.end()
    assert _same(from_dev(dx), orc.rope_bwd(dy, cos, sin, B, T, H, D))
    assert _same(from_dev(s), orc.sum_heads(dy, B, T, H, D))


def test_swiglu_bwd_and_acc(gpu, orc):
    import torch
    rng = np.random.default_rng(3)
    n = 512 * 768 + 5
    gate = (3 * rng.standard_normal(n)).astype(np.float32)
    gate[:3] = [0.0, -0.0, 30.0]
    up, dy = (rng.standard_normal(n).astype(np.float32) for _ in range(2))
    dg, du = (torch.zeros(n, dtype=torch.float32, device="cuda") for _ in range(2))
    a, b = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    a1, a2 = to_dev(a), to_dev(a)
    gpu.begin()
    gpu.swigluBwd(to_dev(gate), to_dev(up), to_dev(dy), dg, du, n)
    gpu.acc(a1, to_dev(b), n)
    gpu.accScale(a2, to_dev(b), n, 0.5)
    gpu.end()
    rg, ru = orc.swiglu_bwd(gate, up, dy)
    assert rel_err(from_dev(dg), rg) <= 2e-6 and rel_err(from_dev(du), ru) <= 2e-6
    assert _same(from_dev(a1), a + b)
    assert _same(from_dev(a2), orc.acc_scale(a, b, 0.5))


def _block_case(dgm, orc, cfg, seed):
    shapes = cfg.linear_shapes()
    rng = orc.RNG(seed)
    masters = {n: rng.randn(shapes[n][0] * shapes[n][1], 0.02 if cfg.C >= 128 else 0.2) for n in dgm.DIT_LINEARS}
    norms = {n: (1.0 + 0.1 * rng.randn(cfg.C, 1.0)).astype(np.float32) for n in dgm.DIT_NORMS}
    x0 = rng.randn(cfg.B * cfg.T * cfg.C, 1.0)
    gy = rng.randn(cfg.B * cfg.T * cfg.C, 1e-2)
    return shapes, masters, norms, x0, gy


def _run_block(gpu, dgm, orc, cfg, seed):
    shapes, masters, norms, x0, gy = _block_case(dgm, orc, cfg, seed)
    blk = dgm.DiTBlock(gpu, cfg, {**{n: to_dev(v) for n, v in masters.items()},
                                  **{n: to_dev(v) for n, v in norms.items()}})
    blk.zero_grads()
    x, g = to_dev(x0), to_dev(gy)
    gpu.begin()
    blk.forward_train(x)
    blk.backward(g)
    gpu.end()
    ocfg = orc.DiTCfg(B=cfg.B, T=cfg.T, C=cfg.C, F=cfg.F, H=cfg.H, D=cfg.D, loops=cfg.loops, group=cfg.group,
                      bits=cfg.bits, eps=cfg.eps, theta=cfg.theta, mix=cfg.mix)
    if cfg.bits == 32:
        lin = masters
    else:
        lin = {n: (from_dev(blk.codes[n]).view(np.int8) if cfg.bits == 8 else from_dev(blk.codes[n]),
                   from_dev(blk.scales[n])) for n in dgm.DIT_LINEARS}
    xo, gx, gw, gn = orc.dit_train(ocfg, lin, norms, x0, gy)
    return blk, from_dev(x), from_dev(g), xo, gx, gw, gn, x0


def _check_block(blk, dgm, xg, gg, xo, gx, gw, gn, bar=1e-5):
    errs = {"x": rel_err(xg, xo), "gx": rel_err(gg, gx)}
    errs.update({n: rel_err(from_dev(blk.grads[n]), gw[n]) for n in dgm.DIT_LINEARS})
    errs.update({n: rel_err(from_dev(blk.grads[n]), gn[n]) for n in dgm.DIT_NORMS})
    bad = {k: v for k, v in errs.items() if not v <= bar}
    assert not bad, bad


def test_c3_block_backward(gpu, dgm, orc):
    """c3: B 8, T 64, C 192, F 768, H 4, D 48, 4 loops, int8 G=32 (STE backward)."""
    cfg = dgm.DiTConfig()
    blk, xg, gg, xo, gx, gw, gn, _ = _run_block(gpu, dgm, orc, cfg, 456)
    _check_block(blk, dgm, xg, gg, xo, gx, gw, gn)


@pytest.mark.parametrize("B,bits,loops", [(2, 4, 2), (3, 8, 1)])
def test_c3_shape_block_backward(gpu, dgm, orc, B, bits, loops):
    """The c3 block shape at other batch sizes, loop counts and int4 linears
    (the three-launch forward, the one-launch attention backward and the
    bf16-dX weight backward)."""
    cfg = dgm.DiTConfig(B=B, bits=bits, loops=loops)
    blk, xg, gg, xo, gx, gw, gn, _ = _run_block(gpu, dgm, orc, cfg, 600 + B)
    _check_block(blk, dgm, xg, gg, xo, gx, gw, gn)


@pytest.mark.parametrize("bits,group", [(32, 8), (8, 16), (4, 16), (8, 32), (4, 32)])
def test_small_block_backward(gpu, dgm, orc, bits, group):
    cfg = dgm.DiTConfig(B=2, T=16, C=64, F=128, H=4, D=16, loops=3, group=group, bits=bits)
    blk, xg, gg, xo, gx, gw, gn, _ = _run_block(gpu, dgm, orc, cfg, 900 + bits)
    _check_block(blk, dgm, xg, gg, xo, gx, gw, gn)


def test_block_backward_separate_grads(gpu, dgm, orc):
    """Linear gradients in separate buffers: the backward takes the per-linear
    path instead of the stacked [wq; wk; wv] / [wgate; wup] weight backwards."""
    import torch
    cfg = dgm.DiTConfig(B=2, T=16, C=64, F=128, H=4, D=16, loops=3, group=16, bits=8)
    shapes, masters, norms, x0, gy = _block_case(dgm, orc, cfg, 77)
    blk = dgm.DiTBlock(gpu, cfg, {**{n: to_dev(v) for n, v in masters.items()},
                                  **{n: to_dev(v) for n, v in norms.items()}})
    blk.zero_grads()
    for n in dgm.DIT_LINEARS:
        blk.grads[n] = torch.zeros_like(blk.grads[n]).clone()
    blk.c_grads = type(blk.c_grads)(*[blk.grads[n].data_ptr() for n in dgm.DIT_LINEARS],
                                    *[blk.grads[n].data_ptr() for n in dgm.DIT_NORMS])
    x, g = to_dev(x0), to_dev(gy)
    gpu.begin()
    blk.forward_train(x)
    blk.backward(g)
    gpu.end()
    ocfg = orc.DiTCfg(B=cfg.B, T=cfg.T, C=cfg.C, F=cfg.F, H=cfg.H, D=cfg.D, loops=cfg.loops, group=cfg.group,
                      bits=cfg.bits, eps=cfg.eps, theta=cfg.theta, mix=cfg.mix)
    lin = {n: (from_dev(blk.codes[n]).view(np.int8), from_dev(blk.scales[n])) for n in dgm.DIT_LINEARS}
    xo, gx, gw, gn = orc.dit_train(ocfg, lin, norms, x0, gy)
    _check_block(blk, dgm, from_dev(x), from_dev(g), xo, gx, gw, gn)


def test_block_backward_swiglu_wide_dx_tiles(gpu, dgm, orc):
    """int8 G=16 (no bf16-dX weight backward): wdown's backward runs the
    STE pair with the SwiGLU backward in its dX epilogue on 32-row dX tiles
    (C = 192, F = 1024, 512 rows)."""
    cfg = dgm.DiTConfig(B=8, T=64, C=192, F=1024, H=4, D=48, loops=1, group=16, bits=8)
    blk, xg, gg, xo, gx, gw, gn, _ = _run_block(gpu, dgm, orc, cfg, 41)
    _check_block(blk, dgm, xg, gg, xo, gx, gw, gn)


def test_wide_block_backward(gpu, dgm, orc):
    """C = 320 > 256: the RMSNorm backwards run one launch each (no chains)."""
    cfg = dgm.DiTConfig(B=2, T=16, C=320, F=128, H=4, D=80, loops=2, group=16, bits=8)
    blk, xg, gg, xo, gx, gw, gn, _ = _run_block(gpu, dgm, orc, cfg, 31)
    _check_block(blk, dgm, xg, gg, xo, gx, gw, gn)


def test_forward_train_matches_forward(gpu, dgm, orc):
    """The saving forward and the fused forward give the same xs[loops] (1e-5)."""
    cfg = dgm.DiTConfig()
    shapes, masters, norms, x0, _ = _block_case(dgm, orc, cfg, 7)
    blk = dgm.DiTBlock(gpu, cfg, {**{n: to_dev(v) for n, v in masters.items()},
                                  **{n: to_dev(v) for n, v in norms.items()}})
    x1, x2 = to_dev(x0), to_dev(x0)
    gpu.begin()
    blk.forward(x1)
    blk.forward_train(x2)
    gpu.end()
    assert rel_err(from_dev(x2), from_dev(x1).astype(np.float64)) <= 1e-5


def test_grads_accumulate_over_steps(gpu, dgm, orc):
    """Two backward passes add into the same gradients (gemmDWAcc and
    rmsnorm_bwd_dw are accumulating): twice one pass, within fp32 rounding."""
    cfg = dgm.DiTConfig(B=2, T=16, C=64, F=128, H=4, D=16, loops=2, group=16, bits=8)
    shapes, masters, norms, x0, gy = _block_case(dgm, orc, cfg, 31)
    blk = dgm.DiTBlock(gpu, cfg, {**{n: to_dev(v) for n, v in masters.items()},
                                  **{n: to_dev(v) for n, v in norms.items()}})
    blk.zero_grads()
    gpu.begin()
    for _ in range(2):
        x, g = to_dev(x0), to_dev(gy)
        blk.forward_train(x)
        blk.backward(g)
    gpu.end()
    twice = {n: from_dev(t).copy() for n, t in blk.grads.items()}
    blk.zero_grads()
    x, g = to_dev(x0), to_dev(gy)
    gpu.begin()
    blk.forward_train(x)
    blk.backward(g)
    gpu.end()
    for n, t in blk.grads.items():
        assert rel_err(twice[n], 2.0 * from_dev(t).astype(np.float64)) <= 1e-6, n


def test_block_backward_rejects(gpu, dgm):
    import torch
    cfg = dgm.DiTConfig(B=2, T=16, C=64, F=128, H=4, D=16, loops=1, group=16, bits=8)
    bad = cfg.c_cfg()
    bad.H = 3
    t = torch.zeros(16, device="cuda")
    with pytest.raises(dgm.DgmError) as e:
        gpu.begin()
        try:
            gpu.dit_backward(bad, dgm.DiTWeights(), dgm.DiTGrads(), t, t, t, 1 << 30, t, t, 1 << 30)
        finally:
            gpu.lib.dgm_end(gpu.h)
    assert e.value.code == dgm.DGM_ERR_SHAPE
