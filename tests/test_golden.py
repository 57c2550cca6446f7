"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) against their definition, on the CPU.

Each fixture freezes the inputs of one of the reference's runtime checks
(checkQuant, Check.swift:72-95; checkGemm, Check.swift:97-136) or a slice of
the reference's own photos-dit weights, with the expected outputs. These tests
pin the fixtures three ways:
  * the inputs are exactly the seeded draws the reference's checks make, in
    their order (RNG(bits*99); RNG(1000+bits) drawing x, w, bias, dy per case);
  * the expected arrays are what the oracle computes from those inputs today
    (a change to the oracle or to the files fails here);
  * the expected arrays satisfy what the mathematics fixes independently of the
    oracle: codes within +-qmax, every group's extreme weight at +-qmax, every
    weight within half a step of its dequantized value, and the GEMM outputs
    within 1e-5 (relative) of float64 products and within the reference's own
    2e-3 bar.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
REF_DIT = "/root/reference/build/photos-dit.ckpt"


def load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def groups_ok(w, q, s, rows, cols, g, bits, orc):
    """Independent checks of codes and scales (Check.swift:399-431 semantics)."""
    qmax = 127 if bits == 8 else 7
    deq = orc.dequant(q, s, rows, cols, g, bits).reshape(rows, cols).astype(np.float64)
    w2 = w.reshape(rows, cols).astype(np.float64)
    s2 = s.reshape(rows, cols // g).astype(np.float64)
    codes = np.rint(deq / np.repeat(s2, g, axis=1))
    assert np.all(np.abs(codes) <= qmax)
    for r in range(rows):
        for j in range(cols // g):
            blk = w2[r, j * g:(j + 1) * g]
            # the group's largest |w| codes to +-qmax; every w within half a step
            assert np.abs(codes[r, j * g + int(np.argmax(np.abs(blk)))]) == qmax
            assert np.all(np.abs(deq[r, j * g:(j + 1) * g] - blk) <= 0.5 * s2[r, j] * (1 + 1e-6))


@pytest.mark.parametrize("bits", [8, 4])
def test_checkquant_fixture(orc, bits):
    z = load(f"checkquant_b{bits}.npz")
    rows, cols, g, b = (int(v) for v in z["shape"])
    assert (rows, cols, g, b) == (5, 16, 8, bits)
    w = orc.RNG(bits * 99).randn(rows * cols, 0.3)
    assert np.array_equal(w.view(np.uint32), z["w"].view(np.uint32))
    q, s = orc.quant(w, rows, cols, g, bits)
    assert np.array_equal(q, z["q"]) and np.array_equal(s.view(np.uint32), z["s"].view(np.uint32))
    assert np.array_equal(orc.dequant(q, s, rows, cols, g, bits), z["deq"])
    groups_ok(w, z["q"], z["s"], rows, cols, g, bits, orc)


@pytest.mark.parametrize("bits", [32, 8, 4])
def test_checkgemm_fixture(orc, bits):
    z = load(f"checkgemm_b{bits}.npz")
    rng = orc.RNG(1000 + bits)
    cases = [(3, 5, 7), (17, 13, 16), (8, 24, 32)] if bits == 32 else [(3, 5, 8), (15, 13, 16), (8, 24, 32)]
    for i, (M, N, K) in enumerate(cases):
        p = f"c{i}_"
        assert tuple(int(v) for v in z[p + "shape"]) == (M, N, K, 8, bits)
        for name, n, std in (("x", M * K, 0.5), ("w", N * K, 0.5), ("bias", N, 0.1), ("dy", M * N, 0.2)):
            assert np.array_equal(rng.randn(n, std).view(np.uint32), z[p + name].view(np.uint32)), name
        x, w, bias, dy = z[p + "x"], z[p + "w"], z[p + "bias"], z[p + "dy"]
        if bits == 32:
            wd = w
        else:
            q, s = orc.quant(w, N, K, 8, bits)
            assert np.array_equal(q, z[p + "q"]) and np.array_equal(s, z[p + "s"])
            groups_ok(w, q, s, N, K, 8, bits, orc)
            wd = orc.dequant(q, s, N, K, 8, bits)
            assert np.array_equal(orc.gemm_nt_q(q, s, x, bias, M, N, K, 8, bits), z[p + "y_kernel"])
        assert np.array_equal(orc.gemm_nt(x, wd, bias, M, N, K), z[p + "y"])
        assert np.array_equal(orc.gemm_dx(dy, wd, M, N, K), z[p + "dx"])
        assert np.array_equal(orc.gemm_dw(dy, x, M, N, K), z[p + "dw"])
        x64, w64, dy64 = (a.astype(np.float64) for a in (x.reshape(M, K), wd.reshape(N, K), dy.reshape(M, N)))
        refs = {"y": x64 @ w64.T + bias.astype(np.float64), "dx": dy64 @ w64, "dw": dy64.T @ x64}
        if bits != 32:
            refs["y_kernel"] = refs["y"]
        for k, ref in refs.items():
            got = z[p + k].astype(np.float64).reshape(ref.shape)
            assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref)), k
            assert np.max(np.abs(got - ref)) < 2e-3, k


def test_photos_dit_wup_fixture(orc):
    z = load("photos_dit_wup.npz")
    M, rows, cols, g = (int(v) for v in z["shape"])
    assert (M, rows, cols, g) == (8, 64, 192, 32)
    w, x = z["w"], z["x"]
    assert np.array_equal(orc.RNG(1001).randn(M * cols, 1.0).view(np.uint32), x.view(np.uint32))
    # realistic trained weights, not N(0, s): the statistics of the reference's wup
    assert 0.05 < float(np.sqrt(np.mean(w.astype(np.float64) ** 2))) < 0.1
    x64 = x.reshape(M, cols).astype(np.float64)
    for bits in (8, 4):
        q, s = orc.quant(w, rows, cols, g, bits)
        assert np.array_equal(q, z[f"q{bits}"]) and np.array_equal(s, z[f"s{bits}"])
        groups_ok(w, q, s, rows, cols, g, bits, orc)
        y = orc.gemm_nt_q(q, s, x, None, M, rows, cols, g, bits)
        assert np.array_equal(y, z[f"y{bits}"])
        ref = x64 @ orc.dequant(q, s, rows, cols, g, bits).reshape(rows, cols).astype(np.float64).T
        assert np.max(np.abs(y.reshape(M, rows) - ref)) <= 1e-5 * np.max(np.abs(ref))


@pytest.mark.skipif(not os.path.exists(REF_DIT), reason="the reference's checkpoints are not on this machine")
def test_photos_dit_wup_fixture_matches_checkpoint(dgm):
    z = load("photos_dit_wup.npz")
    _, params = dgm.read_tdit(REF_DIT)
    wup = {p.name: p for p in params}["wup"]
    rows = int(z["shape"][1])
    assert np.array_equal(wup.data.reshape(wup.rows, wup.cols)[:rows].reshape(-1).view(np.uint32),
                          z["w"].view(np.uint32))
