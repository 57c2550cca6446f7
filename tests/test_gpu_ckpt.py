"""GPU side of the checkpoint loaders: GPT.load's read-then-quantizeAll
(src/GPT.swift:283-324) and a DiT block built from a TDIT file
(src/DiT.swift:413-451). Files are written by this library's writers (the
reference's layout, pinned in test_ckpt_host.py). Bars: masters bitwise the
file, codes and scales bitwise the oracle's quantizer, the block forward
<= 1e-5 against the oracle."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, rel_err
from test_ckpt_host import GPT_H, _gpt_masters, _tdit_masters

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [8, 4])
def test_load_gpt_requantizes(gpu, dgm, orc, tmp_path, bits):
    h = dict(GPT_H, bits=bits)
    rng = np.random.default_rng(bits)
    shapes, masters = _gpt_masters(h, rng)
    path = tmp_path / "g.ckpt"
    dgm.save_tgmt(path, h, bytes(range(h["vocab"])), [0.05 * m for m in masters])
    hdr, itos, params = dgm.load_gpt(path, gpu)
    assert hdr == h and itos == bytes(range(h["vocab"]))
    for (name, r, c, q, _), m, p in zip(shapes, masters, params):
        w = (0.05 * m).astype(np.float32)
        assert np.array_equal(from_dev(p.w)[: r * c].view(np.uint32), w.view(np.uint32)), name
        assert p.quantized == q
        if q:
            rq, rs = orc.quant(w, r, c, h["qGroup"], bits)
            qh = from_dev(p.q)[: rq.size]
            assert np.array_equal(qh.view(np.int8) if bits == 8 else qh, rq), name
            assert np.array_equal(from_dev(p.scale)[: rs.size].view(np.uint32), rs.view(np.uint32)), name
        else:
            assert p.q is None and p.scale is None


def test_dit_block_from_checkpoint(gpu, dgm, orc, tmp_path):
    """A TDIT file at the c3 block shape (T = (128/16)^2 = 64 tokens, embd 192,
    4 heads, SwiGLU 768, 4 loops), weights ~N(0, 0.02), norms 1: the block
    loads, quantizes to int8 G=32 and runs the fused forward."""
    import torch
    h = dict(side=128, patch=16, names=14, loops=4, heads=4, kvHeads=1, embd=192, intermediate=768, freqDim=192,
             diffusionSteps=100, lastAlpha=1e-4, valueMix=0.5)
    rng = np.random.default_rng(12)
    shapes, masters = _tdit_masters(h, rng)
    masters = [np.ones_like(m) if n.startswith("n") and c == 1 else (0.02 * m).astype(np.float32)
               for (n, _, c), m in zip(shapes, masters)]
    path = tmp_path / "d.ckpt"
    dgm.save_tdit(path, h, masters)
    hdr, cfg, blk = dgm.load_dit_block(path, gpu, bits=8, group=32, batch=2)
    assert (cfg.T, cfg.C, cfg.F, cfg.H, cfg.D, cfg.loops, cfg.mix) == (64, 192, 768, 4, 48, 4, 0.5)
    x0 = np.random.default_rng(3).standard_normal(cfg.B * cfg.T * cfg.C).astype(np.float32)
    x = torch.from_numpy(x0.copy()).cuda()
    gpu.begin()
    blk.forward(x)
    gpu.end()
    by = {n: m for (n, _, _), m in zip(shapes, masters)}
    sh = cfg.linear_shapes()
    qw = {n: orc.quant(by[n], sh[n][0], sh[n][1], 32, 8) for n in dgm.DIT_LINEARS}
    qw.update({n: by[n] for n in dgm.DIT_NORMS})
    ocfg = orc.DiTCfg(B=cfg.B, T=cfg.T, C=cfg.C, F=cfg.F, H=cfg.H, D=cfg.D, loops=cfg.loops, group=32, bits=8,
                      eps=cfg.eps, theta=cfg.theta, mix=cfg.mix)
    ref = orc.dit_forward(ocfg, qw, x0)
    assert rel_err(from_dev(x), ref) <= 1e-5
