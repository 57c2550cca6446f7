"""dgm_gemmNT_noalloc: dgm_gemmNT with its staging buffers in the library's
static device scratch, called through the C ABI.

* On each forward path that stages data (decode pieces at M <= 64 in both
  math modes, the K-sliced kernel's partial sums, the bf16 prefill path's
  bf16 copy of X) and on one that stages
  nothing (fp32 tiles), two calls in a row, the second with a smaller input,
  return exactly dgm_gemmNT's bytes.
* On a fresh context the call can be captured in a HIP graph (nothing to
  allocate) on the staging paths (M = 64 decode pieces, the K-sliced
  partial sums, bf16 prefill), and
  every replay, with eager work between replays, matches the eager result;
  under the same capture the regular entry point refuses.
* A call that needs more scratch than the library holds fails with
  DGM_ERR_UNSUPPORTED and leaves its output untouched.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _case(gpu, M, N, K, G, bits, seed):
    import torch
    rng = np.random.default_rng(seed)
    x = to_dev(rng.standard_normal(M * K).astype(np.float32))
    w = to_dev((rng.standard_normal(N * K) * 0.02).astype(np.float32))
    bias = to_dev(rng.standard_normal(N).astype(np.float32)) if seed % 2 else None
    q = torch.zeros(N * K // (2 if bits == 4 else 1), dtype=torch.uint8 if bits == 4 else torch.int8, device="cuda")
    s = torch.zeros(N * (K // G), device="cuda")
    gpu.begin()
    gpu.quantize(w, q, s, N, K, bits, G)
    gpu.end()
    return x, q, s, bias


def _both(gpu, dgm, math, bits, M, N, K, G, seed):
    import torch
    x, q, s, bias = _case(gpu, M, N, K, G, bits, seed)
    ya = torch.full((M * N,), float("nan"), device="cuda")
    yb = torch.full((M * N,), float("nan"), device="cuda")
    gpu.set_math(math)
    try:
        gpu.begin()
        gpu.gemmNT(bits, None, q, s, x, bias, ya, M, N, K, G)
        gpu.gemmNT_noalloc(bits, None, q, s, x, bias, yb, M, N, K, G)
        gpu.end()
    finally:
        gpu.set_math(dgm.DGM_MATH_FP32)
    return from_dev(ya), from_dev(yb)


# (math, bits, first shape, second shape): decode pieces (fused, prepared,
# tiled), bf16 prefill, fp32 tiles (no staging), K-sliced partial sums.
CASES = [
    ("fp32", 4, (16, 1024, 4096, 128), (3, 520, 2048, 128)),
    ("fp32", 8, (64, 700, 2048, 64), (7, 300, 1024, 64)),
    ("bf16", 4, (64, 900, 4096, 128), (16, 256, 1024, 128)),
    ("bf16", 4, (1024, 768, 2048, 128), (300, 500, 1024, 32)),
    ("bf16", 8, (512, 512, 1024, 64), (130, 260, 512, 32)),
    ("fp32", 4, (512, 192, 768, 32), (100, 64, 256, 32)),
    ("fp32", 4, (16, 3600, 4096, 128), (5, 7200, 2048, 128)),
    ("bf16", 8, (8, 3600, 2048, 64), (4, 3600, 2048, 128)),
]


@pytest.mark.parametrize("math,bits,first,second", CASES)
def test_matches_gemmNT_twice(gpu, dgm, math, bits, first, second):
    mode = dgm.DGM_MATH_FP32 if math == "fp32" else dgm.DGM_MATH_BF16
    for i, (M, N, K, G) in enumerate((first, second)):
        ya, yb = _both(gpu, dgm, mode, bits, M, N, K, G, 17 * i + M)
        assert np.all(np.isfinite(ya))
        assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), (math, bits, M, N, K, G)


# Shapes whose forward stages data: the decode kernels' prepared activation
# pieces (16 < M <= 64), the K-sliced kernel's partial sums (two launches)
# and the bf16 prefill path's bf16 copy of X.
CAPTURED = [
    ("fp32", 4, (64, 512, 2048, 128)),
    ("fp32", 4, (16, 3600, 4096, 128)),
    ("bf16", 4, (512, 512, 1024, 128)),
]


@pytest.mark.parametrize("math,bits,shape", CAPTURED)
def test_captured_on_a_fresh_context(dgm, orc, torch_cuda, math, bits, shape):
    """On a fresh context (empty workspace) the call is captured in a HIP
    graph and every replay, with eager work between replays, matches the
    eager dgm_gemmNT result bitwise; under the same capture, dgm_gemmNT on a
    second fresh context refuses (its workspace would have to grow), which is
    what the static scratch makes unnecessary."""
    torch = torch_cuda
    mode = dgm.DGM_MATH_FP32 if math == "fp32" else dgm.DGM_MATH_BF16
    M, N, K, G = shape
    stream = torch.cuda.Stream()
    g = dgm.GPU(stream=stream)
    g2 = dgm.GPU(stream=stream)
    ref_ctx = dgm.GPU(stream=stream)
    try:
        for c in (g, g2, ref_ctx):
            c.set_math(mode)
        x, q, s, bias = _case(ref_ctx, M, N, K, G, bits, 5)
        y = torch.zeros(M * N, device="cuda")
        ref = torch.zeros(M * N, device="cuda")
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            g.begin()
            g.gemmNT_noalloc(bits, None, q, s, x, bias, y, M, N, K, G)
            g2.begin()
            with pytest.raises(dgm.DgmError) as e:
                g2.gemmNT(bits, None, q, s, x, bias, y, M, N, K, G)
            assert e.value.code == dgm.DGM_ERR_UNSUPPORTED
        with torch.cuda.stream(stream):
            ref_ctx.begin()
            ref_ctx.gemmNT(bits, None, q, s, x, bias, ref, M, N, K, G)
            ref_ctx.end()
        want = from_dev(ref)
        assert np.all(np.isfinite(want))
        for _ in range(3):
            y.fill_(float("nan"))
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                graph.replay()
            stream.synchronize()
            assert np.array_equal(from_dev(y).view(np.uint32), want.view(np.uint32))
        del graph
    finally:
        torch.cuda.synchronize()
        for c in (g, g2, ref_ctx):
            c.close()


def test_too_large_is_refused(gpu, dgm):
    import torch
    # bf16 prefill: its bf16 copy of X needs 2*M*K bytes > the scratch.
    M, N, K, G = 2048, 256, 4096, 128
    assert 2 * M * K > dgm.DGM_NOALLOC_SCRATCH_BYTES
    x, q, s, _ = _case(gpu, M, N, K, G, 4, 9)
    y = torch.full((M * N,), 7.0, device="cuda")
    gpu.set_math(dgm.DGM_MATH_BF16)
    try:
        gpu.begin()
        with pytest.raises(dgm.DgmError) as e:
            gpu.gemmNT_noalloc(4, None, q, s, x, None, y, M, N, K, G)
        assert e.value.code == dgm.DGM_ERR_UNSUPPORTED
        gpu.begin()
        gpu.end()
    finally:
        gpu.set_math(dgm.DGM_MATH_FP32)
    assert np.all(from_dev(y) == 7.0)
