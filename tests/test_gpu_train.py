"""GPU parity of the training-step entry points through the C ABI.

adamw / adam_quantize (metal/kernels.metal:786-802 then 100-124; GPT.swift:
214-217, 441-447), zero/scale (770-784), embed_* (616-663), embed_bwd
(665-682), pos_bwd (684-697), bias_grad (285-295): bit-exact against the CPU
oracle. reduce_sumsq (749-768) sums in this library's own fixed order: max
relative error 1e-6 against float64, and bitwise repeatable.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-3, b1=0.9, b2=0.95, eps=1e-8, wd=0.1)


def _bc(step, b1=0.9, b2=0.95):
    f = np.float32
    return float(f(1) / (f(1) - f(b1) ** f(step))), float(f(1) / (f(1) - f(b2) ** f(step)))


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def _shifted(t, offset):
    """A copy of device tensor t starting `offset` floats into a fresh buffer."""
    import torch
    if not offset:
        return t
    raw = torch.zeros(t.numel() + offset, dtype=t.dtype, device="cuda")
    raw[offset:] = t
    return raw[offset:]


@pytest.mark.parametrize("n", [1, 7, 8, 9, 1000, 4099, (1 << 20) + 3])
@pytest.mark.parametrize("offset", [0, 1])
def test_adam_bitexact(gpu, orc, n, offset):
    rng = np.random.default_rng(n + offset)
    w = rng.standard_normal(n).astype(np.float32)
    m = (0.1 * rng.standard_normal(n)).astype(np.float32)
    v = np.abs(0.01 * rng.standard_normal(n)).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    bc1, bc2 = _bc(3)
    wd_, md, vd, gd = (_shifted(to_dev(a), offset) for a in (w, m, v, g))
    gpu.begin()
    gpu.adam(wd_, gd, md, vd, n, HP["lr"], HP["b1"], HP["b2"], HP["eps"], HP["wd"], bc1, bc2)
    gpu.end()
    rw, rm, rv = orc.adamw(w, g, m, v, HP["lr"], HP["b1"], HP["b2"], HP["eps"], HP["wd"], bc1, bc2)
    assert _same(from_dev(wd_), rw) and _same(from_dev(md), rm) and _same(from_dev(vd), rv)
    assert gpu.lastKernel == "adamw"


def test_adamw_kernel_entry_and_steps(gpu, dgm, orc):
    """Five steps through the kernel-level entry (AdamP block), no decay."""
    n = 3000
    rng = np.random.default_rng(11)
    w = rng.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    wd_, md, vd = to_dev(w), to_dev(m), to_dev(v)
    for step in range(1, 6):
        g = rng.standard_normal(n).astype(np.float32)
        bc1, bc2 = _bc(step)
        p = dgm.AdamP(n, 1e-2, 0.9, 0.95, 1e-8, 0.0, bc1, bc2)
        gpu.begin()
        gpu.adamw(wd_, to_dev(g), md, vd, p)
        gpu.end()
        w, m, v = orc.adamw(w, g, m, v, 1e-2, 0.9, 0.95, 1e-8, 0.0, bc1, bc2)
    assert _same(from_dev(wd_), w) and _same(from_dev(md), m) and _same(from_dev(vd), v)


# Fused shapes (power-of-two G in [8, 512], cols % G == 0) and shapes that run
# as adam + quantize: G 6 / 12 (not a power of two), cols not a multiple of G.
SHAPES = [(8, 64, 8), (5, 96, 16), (16, 192, 32), (7, 768, 64), (3, 4096, 128), (2, 1024, 256),
          (4, 2048, 512), (5, 36, 6), (3, 50, 12), (4, 100, 32)]


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("rows,cols,G", SHAPES)
def test_adam_quantize_bitexact(gpu, orc, bits, rows, cols, G):
    import torch
    rng = np.random.default_rng(rows * cols + G + bits)
    n = rows * cols
    w = (0.05 * rng.standard_normal(n)).astype(np.float32)
    m = (0.01 * rng.standard_normal(n)).astype(np.float32)
    v = np.abs(1e-4 * rng.standard_normal(n)).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    nq = n if bits == 8 else n // 2
    q0 = rng.integers(0, 256, nq).astype(np.uint8)          # tail codes must survive
    bc1, bc2 = _bc(2)
    wd_, md, vd, gd = to_dev(w), to_dev(m), to_dev(v), to_dev(g)
    qd = to_dev(q0)
    sd = torch.zeros(max(rows * (cols // G), 1), dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.adamQuantize(wd_, gd, md, vd, qd, sd, rows, cols, bits, G, HP["lr"], HP["b1"], HP["b2"], HP["eps"],
                     HP["wd"], bc1, bc2)
    gpu.end()
    init = q0.view(np.int8) if bits == 8 else q0
    rw, rm, rv, rq, rs = orc.adam_quantize(w, g, m, v, rows, cols, G, bits, HP["lr"], HP["b1"], HP["b2"],
                                           HP["eps"], HP["wd"], bc1, bc2, init=init)
    assert _same(from_dev(wd_), rw) and _same(from_dev(md), rm) and _same(from_dev(vd), rv)
    qh = from_dev(qd)
    assert np.array_equal(qh.view(np.int8) if bits == 8 else qh, rq)
    assert _same(from_dev(sd)[:rs.size], rs)
    fused = cols % G == 0 and G & (G - 1) == 0 and 8 <= G <= 512
    assert gpu.lastKernel == ("adam_quantize" if fused else ("quant_i4" if bits == 4 else "quant_i8"))


def test_adam_quantize_c4_shape(gpu, orc):
    """The c4/c5 weight (14336 x 4096, int4, G 128): bit-exact on a row slice,
    and the full-size result equals adam followed by quantize on the GPU."""
    import torch
    rows, cols, G = 14336, 4096, 128
    gen = torch.Generator(device="cuda").manual_seed(0)
    w = 0.02 * torch.randn(rows * cols, generator=gen, device="cuda")
    g = torch.randn(rows * cols, generator=gen, device="cuda")
    m = torch.zeros_like(w)
    v = torch.zeros_like(w)
    bc1, bc2 = _bc(1)
    w_init = w.clone()
    w2, m2, v2 = w.clone(), m.clone(), v.clone()
    q1 = torch.zeros(rows * cols // 2, dtype=torch.uint8, device="cuda")
    s1 = torch.zeros(rows * cols // G, dtype=torch.float32, device="cuda")
    q2, s2 = torch.zeros_like(q1), torch.zeros_like(s1)
    args = (HP["lr"], HP["b1"], HP["b2"], HP["eps"], HP["wd"], bc1, bc2)
    gpu.begin()
    gpu.adamQuantize(w, g, m, v, q1, s1, rows, cols, 4, G, *args)
    gpu.adam(w2, g, m2, v2, rows * cols, *args)
    gpu.quantize(w2, q2, s2, rows, cols, 4, G)
    gpu.end()
    assert torch.equal(w.view(torch.int32), w2.view(torch.int32))
    assert torch.equal(q1, q2) and torch.equal(s1.view(torch.int32), s2.view(torch.int32))
    r0, r1 = 1000, 1040
    sl = slice(r0 * cols, r1 * cols)
    z = np.zeros((r1 - r0) * cols, np.float32)
    rw, _, _, rq, rs = orc.adam_quantize(from_dev(w_init[sl].clone()), from_dev(g[sl].clone()), z, z,
                                         r1 - r0, cols, G, 4, *args)
    assert _same(from_dev(w[sl].clone()), rw)
    assert np.array_equal(from_dev(q1[r0 * cols // 2: r1 * cols // 2].clone()), rq)
    assert _same(from_dev(s1[r0 * cols // G: r1 * cols // G].clone()), rs)


@pytest.mark.parametrize("n", [0, 1, 255, 16384, 16385, 100003, 5_000_000])
def test_reduce_sumsq(gpu, orc, n):
    import torch
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    out = torch.full((4,), -1.0, dtype=torch.float32, device="cuda")
    xd = to_dev(x) if n else torch.zeros(1, device="cuda")
    gpu.begin()
    gpu.reduceSumsq(xd, out, n, 2)
    gpu.reduceSumsq(xd, out, n, 3)
    gpu.end()
    o = from_dev(out)
    assert o[0] == -1.0 and o[1] == -1.0
    ref = float(np.sum(x.astype(np.float64) ** 2))
    assert abs(float(o[2]) - ref) <= 1e-6 * max(ref, 1e-30)
    assert _same(o[2:3], o[3:4]), "repeatable"
    if n:
        assert abs(orc.reduce_sumsq(x) - ref) <= 1e-5 * ref


def test_reduce_sumsq_exact_integers(gpu, dgm):
    import torch
    x = ((np.arange(70000) % 17) - 8).astype(np.float32)
    out = torch.zeros(1, dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.reduce_sumsq(to_dev(x), out, dgm.ReduceP(x.size, 0, 0, 0))
    gpu.end()
    assert float(from_dev(out)[0]) == float(np.sum(x.astype(np.int64) ** 2))


def test_zero_and_scale(gpu, dgm):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(1001).astype(np.float32)
    xd = to_dev(x)
    gpu.begin()
    gpu.scale(xd, 1000, 0.37)
    gpu.end()
    got = from_dev(xd)
    assert _same(got[:1000], x[:1000] * np.float32(0.37)) and got[1000] == x[1000]
    gpu.begin()
    gpu.zero_f(xd, dgm.UnaryP(999, 0, 0, 0))
    gpu.zero(xd, 0)            # n == 0 dispatches nothing (src/GPU.swift:200-201)
    gpu.end()
    got = from_dev(xd)
    assert not got[:999].any() and got[999] == x[999] * np.float32(0.37)


def _embed_case(orc, B, T, C, V, G, bits, seed):
    rng = orc.RNG(seed)
    master = rng.randn(V * C, 0.4)
    wpe = rng.randn(T * C, 0.2)
    toks = np.array([(7 * i * i + 3 * i + seed) % V for i in range(B * T)], np.uint32)
    if bits == 32:
        q, s = None, None
    else:
        q, s = orc.quant(master, V, C, G, bits)
    return master, wpe, toks, q, s


@pytest.mark.parametrize("bits", [32, 8, 4])
@pytest.mark.parametrize("B,T,C,V,G", [(2, 3, 8, 4, 8), (4, 64, 192, 1000, 32), (3, 17, 130, 65, 10),
                                      (16, 64, 128, 65, 8)])
def test_embed_bitexact(gpu, orc, bits, B, T, C, V, G):
    import torch
    if bits == 4 and G % 2:
        pytest.skip("int4 needs an even group")
    master, wpe, toks, q, s = _embed_case(orc, B, T, C, V, G, bits, B + T + C)
    y = torch.zeros(B * T * C, dtype=torch.float32, device="cuda")
    td = torch.from_numpy(toks.view(np.int32).copy()).to("cuda")
    gpu.begin()
    gpu.embed(bits, td, to_dev(master) if bits == 32 else None, None if q is None else to_dev(q.view(np.uint8)),
              None if s is None else to_dev(s), to_dev(wpe), y, B, T, C, G)
    gpu.end()
    ref = orc.embed(toks, master, q, s, wpe, B, T, C, G, bits)
    assert _same(from_dev(y), ref)
    assert gpu.lastKernel == {32: "embed_f32", 8: "embed_i8", 4: "embed_i4"}[bits]


def test_embed_kernel_entries(gpu, dgm, orc):
    import torch
    B, T, C, V, G = 2, 5, 64, 11, 16
    for bits, fn in ((8, gpu.embed_i8), (4, gpu.embed_i4)):
        master, wpe, toks, q, s = _embed_case(orc, B, T, C, V, G, bits, 9)
        y = torch.zeros(B * T * C, dtype=torch.float32, device="cuda")
        gpu.begin()
        fn(torch.from_numpy(toks.view(np.int32).copy()).to("cuda"), to_dev(q.view(np.uint8)), to_dev(s),
           to_dev(wpe), y, dgm.EmbP(B, T, C, G))
        gpu.end()
        assert _same(from_dev(y), orc.embed(toks, None, q, s, wpe, B, T, C, G, bits))


def test_embed_rejects(gpu, dgm):
    import torch
    y = torch.zeros(64, device="cuda")
    t = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(dgm.DgmError) as e:
        gpu.begin()
        try:
            gpu.embed(4, t, None, y, y, y, y, 1, 8, 8, 3)
        finally:
            gpu.lib.dgm_end(gpu.h)
    assert e.value.code == dgm.DGM_ERR_SHAPE
    with pytest.raises(dgm.DgmError) as e:
        gpu.begin()
        try:
            gpu.embed(16, t, None, y, y, y, y, 1, 8, 8, 8)
        finally:
            gpu.lib.dgm_end(gpu.h)
    assert e.value.code == dgm.DGM_ERR_BITS
    with pytest.raises(dgm.DgmError) as e:
        gpu.embedBwd(t, y, y, 1, 8, 8, 1)       # outside begin/end
    assert e.value.code == dgm.DGM_ERR_NOT_BEGUN


@pytest.mark.parametrize("B,T,C,V,dist", [(2, 3, 8, 4, "check"), (16, 64, 128, 65, "zipf"),
                                         (4, 64, 300, 1000, "uniform"), (8, 64, 192, 7, "one"),
                                         (3, 50, 64, 5000, "uniform"), (1, 1, 17, 3, "uniform")])
def test_embed_bwd_bitexact(gpu, orc, B, T, C, V, dist):
    import torch
    rng = np.random.default_rng(B * T * C + V)
    BT = B * T
    if dist == "check":
        toks = np.array([1, 0, 3, 1, 2, 0], np.uint32)
    elif dist == "zipf":
        toks = (np.minimum(rng.zipf(1.3, BT), V) - 1).astype(np.uint32)
    elif dist == "one":
        toks = np.full(BT, 3, np.uint32)
    else:
        toks = rng.integers(0, V, BT).astype(np.uint32)
    dx = rng.standard_normal(BT * C).astype(np.float32)
    dwe = rng.standard_normal(V * C).astype(np.float32)
    dwe[::7] = -0.0                      # untouched rows still get "+= 0.0" (-0 -> +0)
    dd = to_dev(dwe)
    gpu.begin()
    gpu.embedBwd(torch.from_numpy(toks.view(np.int32).copy()).to("cuda"), to_dev(dx), dd, B, T, C, V)
    gpu.end()
    ref = orc.embed_bwd(toks, dx, dwe, B, T, C, V)
    assert _same(from_dev(dd), ref)
    assert gpu.lastKernel == "embed_bwd"


@pytest.mark.parametrize("B,T,C", [(1, 1, 1), (16, 64, 128), (5, 33, 70), (40, 8, 96)])
def test_pos_bwd_bitexact(gpu, dgm, orc, B, T, C):
    import torch
    rng = np.random.default_rng(B + T + C)
    dx = rng.standard_normal(B * T * C).astype(np.float32)
    out = torch.full((T * C,), 5.0, dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.posBwd(to_dev(dx), out, B, T, C)
    gpu.end()
    assert _same(from_dev(out), orc.pos_bwd(dx, B, T, C))
    out2 = torch.zeros_like(out)
    gpu.begin()
    gpu.pos_bwd(to_dev(dx), out2, dgm.PosP(B, T, C, 0))
    gpu.end()
    assert _same(from_dev(out2), orc.pos_bwd(dx, B, T, C))


@pytest.mark.parametrize("M,N", [(1, 1), (1024, 128), (1024, 512), (37, 300), (4096, 64)])
def test_bias_grad_bitexact(gpu, dgm, orc, M, N):
    import torch
    rng = np.random.default_rng(M + N)
    dy = rng.standard_normal(M * N).astype(np.float32)
    out = torch.full((N,), 3.0, dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.biasGrad(to_dev(dy), out, M, N)
    gpu.end()
    assert _same(from_dev(out), orc.bias_grad(dy, M, N))
    out2 = torch.zeros_like(out)
    gpu.begin()
    gpu.bias_grad(to_dev(dy), out2, dgm.BiasP(M, N, 0, 0))
    gpu.end()
    assert _same(from_dev(out2), orc.bias_grad(dy, M, N))


def _gpt_like_params(dgm, bits):
    """A few parameters shaped like the quantized GPT's (src/GPT.swift:118-160):
    quantized token table and linears, unquantized norms and biases."""
    G = 8
    spec = [("wte", 65, 128, True, True), ("wpe", 64, 128, False, True), ("ln1.g", 128, 1, False, False),
            ("wq", 128, 128, True, True), ("bq", 128, 1, False, False), ("fc", 512, 128, True, True),
            ("proj", 128, 512, True, True)]
    return [dgm.Param(n, r, c, q and bits != 32, d, bits, G) for n, r, c, q, d in spec]


@pytest.mark.parametrize("bits", [4, 8])
def test_optimizer_step_matches_reference_order(gpu, dgm, orc, bits):
    """GPT.step's update (src/GPT.swift:193-218): fused adam+quantize equals
    the literal adam-then-quantizeAll order bit for bit, and each parameter
    equals the oracle's clip-scale + adamw + quantize given the step's norm."""
    import torch
    runs = []
    for fused in (True, False):
        params = _gpt_like_params(dgm, bits)
        gen = torch.Generator(device="cpu").manual_seed(5)
        for p in params:
            p.w.copy_((0.02 * torch.randn(p.count, generator=gen)).to("cuda"))
            p.g.copy_((0.5 * torch.randn(p.count, generator=gen)).to("cuda"))
        init = [(from_dev(p.w.clone()), from_dev(p.g.clone())) for p in params]
        norms = [dgm.optimizer_step(gpu, params, 3e-3, 0.1, 1.0, 1, fused=fused)]
        # a second step from the updated state, without clipping
        norms.append(dgm.optimizer_step(gpu, params, 3e-3, 0.1, 0.0, 2, fused=fused))
        runs.append((params, norms, init))
    (pa, na, init), (pb, nb, _) = runs
    assert na == nb
    for a, b in zip(pa, pb):
        for f in ("w", "m", "v", "q", "scale"):
            ta, tb = getattr(a, f), getattr(b, f)
            if ta is not None:
                assert torch.equal(ta.view(torch.uint8), tb.view(torch.uint8)), (a.name, f)
    # Oracle check of the first step, with the norm the GPU step measured.
    norm0 = na[0]
    assert abs(norm0 - math_sqrt_sum(init)) <= 1e-5 * norm0
    params = _gpt_like_params(dgm, bits)
    gen = torch.Generator(device="cpu").manual_seed(5)
    for p in params:
        p.w.copy_((0.02 * torch.randn(p.count, generator=gen)).to("cuda"))
        p.g.copy_((0.5 * torch.randn(p.count, generator=gen)).to("cuda"))
    dgm.optimizer_step(gpu, params, 3e-3, 0.1, 1.0, 1)
    s = float(np.float32(1.0) / (np.float32(norm0) + np.float32(1e-6)))
    bc1, bc2 = dgm.bias_corrections(0.9, 0.95, 1)
    for p, (w0, g0) in zip(params, init):
        gs = orc.scale(g0, s)
        z = np.zeros_like(w0)
        rw, rm, rv = orc.adamw(w0, gs, z, z, 3e-3, 0.9, 0.95, 1e-8, 0.1 if p.decay else 0.0, bc1, bc2)
        assert _same(from_dev(p.w), rw) and _same(from_dev(p.m), rm), p.name
        if p.quantized:
            rq, rs = orc.quant(rw, p.rows, p.cols, 8, bits)
            qh = from_dev(p.q)
            assert np.array_equal(qh.view(np.int8) if bits == 8 else qh, rq), p.name
            assert _same(from_dev(p.scale), rs), p.name


def math_sqrt_sum(init):
    return float(np.sqrt(sum(float(np.sum(g.astype(np.float64) ** 2)) for _, g in init)))
