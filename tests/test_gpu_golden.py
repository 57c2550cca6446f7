"""GPU parity on the committed golden fixtures (tests/golden/*.npz): the
reference's checkQuant and checkGemm cases (Check.swift:72-136) and a slice of
the reference's photos-dit `wup` weights, through the C ABI.

Bars: quantization codes and scales bit-exact; GEMM outputs within max
relative error 1e-5 of the stored oracle results (and the reference's own
max-abs bar 2e-3, Check.swift:135).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import from_dev, rel_err, to_dev

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def quantize(gpu, w, rows, cols, g, bits):
    import torch
    q = torch.zeros(rows * cols // (2 if bits == 4 else 1), dtype=torch.uint8 if bits == 4 else torch.int8,
                    device="cuda")
    s = torch.zeros(rows * (cols // g), dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.quantize(to_dev(w), q, s, rows, cols, bits, g)
    gpu.end()
    return q, s


@pytest.mark.parametrize("bits", [8, 4])
def test_gpu_checkquant_golden(gpu, bits):
    z = load(f"checkquant_b{bits}.npz")
    rows, cols, g, _ = (int(v) for v in z["shape"])
    q, s = quantize(gpu, z["w"], rows, cols, g, bits)
    assert np.array_equal(from_dev(q).view(z["q"].dtype), z["q"])
    assert np.array_equal(from_dev(s).view(np.uint32), z["s"].view(np.uint32))


@pytest.mark.parametrize("bits", [32, 8, 4])
def test_gpu_checkgemm_golden(gpu, bits):
    import torch
    z = load(f"checkgemm_b{bits}.npz")
    for i in range(3):
        p = f"c{i}_"
        M, N, K, G, _ = (int(v) for v in z[p + "shape"])
        x, w, bias, dy = (to_dev(z[p + k]) for k in ("x", "w", "bias", "dy"))
        q = s = None
        if bits != 32:
            q, s = quantize(gpu, z[p + "w"], N, K, G, bits)
            assert np.array_equal(from_dev(q).view(z[p + "q"].dtype), z[p + "q"])
            assert np.array_equal(from_dev(s), z[p + "s"])
        y = torch.zeros(M * N, device="cuda")
        dx = torch.zeros(M * K, device="cuda")
        dw = torch.zeros(N * K, device="cuda")
        gpu.begin()
        gpu.gemmNT(bits, w, q, s, x, bias, y, M, N, K, G)
        gpu.gemmDX(bits, w, q, s, dy, dx, M, N, K, G)
        gpu.gemmDW(dy, x, dw, M, N, K)
        gpu.end()
        for name, got in (("y", y), ("dx", dx), ("dw", dw)):
            got, ref = from_dev(got), z[p + name]
            assert rel_err(got, ref) <= 1e-5, (i, name)
            assert float(np.max(np.abs(got.astype(np.float64) - ref))) < 2e-3, (i, name)


def test_gpu_photos_dit_wup_golden(gpu):
    import torch
    z = load("photos_dit_wup.npz")
    M, rows, cols, g = (int(v) for v in z["shape"])
    for bits in (8, 4):
        q, s = quantize(gpu, z["w"], rows, cols, g, bits)
        assert np.array_equal(from_dev(q).view(z[f"q{bits}"].dtype), z[f"q{bits}"])
        assert np.array_equal(from_dev(s), z[f"s{bits}"])
        y = torch.zeros(M * rows, device="cuda")
        gpu.begin()
        gpu.gemmNT(bits, None, q, s, to_dev(z["x"]), None, y, M, rows, cols, g)
        gpu.end()
        assert rel_err(from_dev(y), z[f"y{bits}"]) <= 1e-5
