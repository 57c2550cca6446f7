"""Writes the golden fixtures in this directory (test data, not product code).

The reference keeps no stored vectors: its checks recompute expectations at run
time from a seeded RNG (src/Check.swift:27-136), and its code (Swift + Metal)
cannot run in this image. These fixtures freeze, as plain arrays:

  * checkquant_b{8,4}.npz — the reference's checkQuant case (Check.swift:72-95):
    rows 5, cols 16, group 8, RNG(bits * 99), weights ~ N(0, 0.3); expected
    codes and scales from the CPU oracle's restatement of cpuQuant
    (Check.swift:399-431).
  * checkgemm_b{32,8,4}.npz — the reference's checkGemm cases (Check.swift:97-136):
    shapes (3,5,7) (17,13,16) (8,24,32) for bits 32 and (3,5,8) (15,13,16)
    (8,24,32) otherwise, group 8, RNG(1000 + bits), draws x, w, bias, dy in the
    reference's order; expected codes/scales, Y (cpuGemmNT on the dequantized
    weights, bias first), Y in the Metal kernel's order (group partial, scale,
    bias last), dX and dW.
  * photos_dit_wup.npz — rows 0..63 of the `wup` matrix [768, 192] of the
    reference's own photos-dit checkpoint (build/photos-dit.ckpt, read with
    the TDIT parser), quantized int8 and int4 with group 32 (the c1/c3 layer
    of BASELINE's configs), plus Y = X deq(W)^T for X[8, 192] = RNG(1001)
    normals.

The input arrays are this library's SplitMix64 / Box-Muller draws (the
reference's normals go through Darwin's logf/cosf, whose last bits are not
reproducible here), so each fixture stores its inputs as bytes. Expected
outputs come from oracle/ (the CPU restatement pinned by tests/test_oracle.py);
tests/test_golden.py re-derives every array from the seeds and the oracle, and
tests/test_gpu_golden.py checks the HIP path against the stored arrays.

Usage: python tests/golden/make_golden.py   (needs oracle/liboracle.so; the
photos-dit fixture also needs /root/reference and libdgm_amd.so for the parser)
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
from oracle import oracle as orc  # noqa: E402

REF_DIT = "/root/reference/build/photos-dit.ckpt"
QGROUP = 8


def checkquant(bits: int) -> dict:
    rows, cols, g = 5, 16, 8
    rng = orc.RNG(bits * 99)
    w = rng.randn(rows * cols, 0.3)
    q, s = orc.quant(w, rows, cols, g, bits)
    return dict(shape=np.array([rows, cols, g, bits], dtype=np.int64), w=w, q=q, s=s,
                deq=orc.dequant(q, s, rows, cols, g, bits))


def gemm_cases(bits: int):
    return [(3, 5, 7), (17, 13, 16), (8, 24, 32)] if bits == 32 else [(3, 5, 8), (15, 13, 16), (8, 24, 32)]


def checkgemm(bits: int) -> dict:
    rng = orc.RNG(1000 + bits)
    out = {}
    for i, (M, N, K) in enumerate(gemm_cases(bits)):
        x = rng.randn(M * K, 0.5)
        w = rng.randn(N * K, 0.5)
        bias = rng.randn(N, 0.1)
        dy = rng.randn(M * N, 0.2)
        p = f"c{i}_"
        out[p + "shape"] = np.array([M, N, K, QGROUP, bits], dtype=np.int64)
        out[p + "x"], out[p + "w"], out[p + "bias"], out[p + "dy"] = x, w, bias, dy
        if bits == 32:
            wd = w
        else:
            q, s = orc.quant(w, N, K, QGROUP, bits)
            out[p + "q"], out[p + "s"] = q, s
            wd = orc.dequant(q, s, N, K, QGROUP, bits)
            out[p + "y_kernel"] = orc.gemm_nt_q(q, s, x, bias, M, N, K, QGROUP, bits)
        out[p + "y"] = orc.gemm_nt(x, wd, bias, M, N, K)
        out[p + "dx"] = orc.gemm_dx(dy, wd, M, N, K)
        out[p + "dw"] = orc.gemm_dw(dy, x, M, N, K)
    return out


def photos_dit_wup():
    if not os.path.exists(REF_DIT):
        return None
    spec = importlib.util.spec_from_file_location(
        "dgm_amd", os.path.join(REPO, "diffusion-gpt-metal_amd", "__init__.py"),
        submodule_search_locations=[os.path.join(REPO, "diffusion-gpt-metal_amd")])
    dgm = importlib.util.module_from_spec(spec)
    sys.modules["dgm_amd"] = dgm
    spec.loader.exec_module(dgm)
    _, params = dgm.read_tdit(REF_DIT)
    wup = {p.name: p for p in params}["wup"]
    rows, cols, g = 64, wup.cols, 32
    w = np.ascontiguousarray(wup.data.reshape(wup.rows, wup.cols)[:rows]).reshape(-1).astype(np.float32)
    x = orc.RNG(1001).randn(8 * cols, 1.0)
    out = dict(shape=np.array([8, rows, cols, g], dtype=np.int64), w=w, x=x)
    for bits in (8, 4):
        q, s = orc.quant(w, rows, cols, g, bits)
        out[f"q{bits}"], out[f"s{bits}"] = q, s
        out[f"y{bits}"] = orc.gemm_nt_q(q, s, x, None, 8, rows, cols, g, bits)
    return out


def main() -> None:
    for bits in (8, 4):
        np.savez(os.path.join(HERE, f"checkquant_b{bits}.npz"), **checkquant(bits))
    for bits in (32, 8, 4):
        np.savez(os.path.join(HERE, f"checkgemm_b{bits}.npz"), **checkgemm(bits))
    wup = photos_dit_wup()
    if wup is not None:
        np.savez(os.path.join(HERE, "photos_dit_wup.npz"), **wup)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
