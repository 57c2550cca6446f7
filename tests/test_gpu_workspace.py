"""The context's grow-only workspace (staging for the decode kernels'
activation pieces) under HIP graph capture.

* A graph captured while the workspace is small keeps writing that buffer
  when replayed after a larger call has grown the workspace: the retired
  buffer stays allocated until the context is destroyed, so the replay is
  still correct.
* A call that would have to grow the workspace while its stream is being
  captured returns DGM_ERR_UNSUPPORTED and launches nothing.
* dgm_gpu_reserve / dgm_gemmNT_workspace_bound (no counterpart in the
  reference, whose buffers are all allocated at setup, src/GPU.swift:31-88):
  on a fresh context, reserving dgm_gemmNT_workspace_bound(M, N, K) makes
  every dgm_gemmNT call of that shape run without growing the workspace, on
  each forward path that stages data (the K-sliced kernel's partial sums, the
  decode kernels' activation pieces in both math modes, the int8 skinny
  kernel's pieces, the bf16 prefill path's bf16 copy of X) and on paths that
  stage nothing; the results are bitwise those of a context that grew its
  workspace on first use. A reserve is refused under graph capture and is a
  no-op when the workspace is already large enough.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, rel_err, to_dev

pytestmark = pytest.mark.gpu


def _setup(gpu, orc, M, N, K, G, seed):
    import torch
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q = torch.zeros(N * K // 2, dtype=torch.uint8, device="cuda")
    s = torch.zeros(N * (K // G), device="cuda")
    gpu.begin()
    gpu.quantize(to_dev(w), q, s, N, K, 4, G)
    gpu.end()
    wd = orc.dequant(from_dev(q), from_dev(s), N, K, G, 4).reshape(N, K).astype(np.float64)
    ref = (x.reshape(M, K).astype(np.float64) @ wd.T).ravel()
    return to_dev(x), q, s, ref


def test_graph_survives_workspace_growth(dgm, orc, torch_cuda):
    torch = torch_cuda
    stream = torch.cuda.Stream()
    gpu = dgm.GPU(stream=stream)
    try:
        # M = 32 and 64: the decode path that stages prepared activation
        # pieces in the workspace (M <= 16 converts them inside the kernel).
        N, K, G = 512, 2048, 128
        xs, qs, ss, refs = _setup(gpu, orc, 32, N, K, G, 1)
        xl, ql, sl, refl = _setup(gpu, orc, 64, N, K * 4, G, 2)
        ys = torch.zeros(32 * N, device="cuda")
        yl = torch.zeros(64 * N, device="cuda")
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            gpu.begin()
            gpu.gemmNT(4, None, qs, ss, xs, None, ys, 32, N, K, G)   # sizes the workspace
            gpu.end()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            gpu.begin()
            gpu.gemmNT(4, None, qs, ss, xs, None, ys, 32, N, K, G)
        gpu.begin()
        # A larger call grows the workspace (4x the pieces).
        with torch.cuda.stream(stream):
            gpu.gemmNT(4, None, ql, sl, xl, None, yl, 64, N, K * 4, G)
            gpu.end()
        assert rel_err(from_dev(yl), refl) <= 1e-5
        for _ in range(3):
            ys.fill_(float("nan"))
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                graph.replay()
            stream.synchronize()
            assert rel_err(from_dev(ys), refs) <= 1e-5
        del graph
    finally:
        torch.cuda.synchronize()
        gpu.close()


def test_growth_during_capture_is_refused(dgm, orc, torch_cuda):
    torch = torch_cuda
    stream = torch.cuda.Stream()
    gpu = dgm.GPU(stream=stream)   # a fresh context: empty workspace
    try:
        # M = 64: the decode path that stages prepared activation pieces in
        # the workspace (M <= 16 converts them inside the kernel instead).
        M, N, K, G = 64, 256, 1024, 128
        x, q, s, ref = _setup(gpu, orc, M, N, K, G, 3)
        y = torch.zeros(M * N, device="cuda")
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        err = None
        with torch.cuda.graph(graph, stream=stream):
            gpu.begin()
            try:
                gpu.gemmNT(4, None, q, s, x, None, y, M, N, K, G)
            except dgm.DgmError as e:
                err = e
        assert err is not None and err.code == dgm.DGM_ERR_UNSUPPORTED, err
        del graph
        # Outside capture the same call sizes the workspace and succeeds.
        with torch.cuda.stream(stream):
            gpu.begin()
            gpu.gemmNT(4, None, q, s, x, None, y, M, N, K, G)
            gpu.end()
        assert rel_err(from_dev(y), ref) <= 1e-5
    finally:
        torch.cuda.synchronize()
        gpu.close()


# (math, bits, (M, N, K, G)): stream (M = 1), K-sliced (fp32 M = 16, int4 and int8), one-launch
# decode (reduced M = 16), decode pieces (M = 64 both modes, M = 33), int8
# skinny (M = 24 int8 fp32), bf16 prefill (M = 256 reduced), fp32 tiles (M = 256).
CASES = [
    ("fp32", 4, (1, 14336, 4096, 128)),
    ("fp32", 4, (16, 14336, 4096, 128)),
    ("fp32", 8, (16, 8192, 4096, 128)),      # int8 K-sliced: 16 slices, partial sums exactly 8 MiB
    ("bf16", 4, (16, 14336, 4096, 128)),
    ("fp32", 4, (64, 14336, 4096, 128)),
    ("bf16", 4, (64, 14336, 4096, 128)),
    ("fp32", 8, (33, 4096, 2048, 64)),
    ("fp32", 8, (24, 4096, 2048, 64)),
    ("bf16", 4, (256, 2048, 1024, 128)),
    ("fp32", 4, (256, 2048, 1024, 128)),
]


def _case(gpu, M, N, K, G, bits, seed):
    import torch
    rng = np.random.default_rng(seed)
    x = to_dev(rng.standard_normal(M * K).astype(np.float32))
    w = to_dev((rng.standard_normal(N * K) * 0.02).astype(np.float32))
    q = torch.zeros(N * K // (2 if bits == 4 else 1), dtype=torch.uint8 if bits == 4 else torch.int8, device="cuda")
    s = torch.zeros(N * (K // G), device="cuda")
    gpu.begin()
    gpu.quantize(w, q, s, N, K, bits, G)
    gpu.end()
    return x, q, s


def _forward(g, dgm, math, bits, q, s, x, M, N, K, G):
    import torch
    y = torch.full((M * N,), float("nan"), device="cuda")
    g.set_math(dgm.DGM_MATH_FP32 if math == "fp32" else dgm.DGM_MATH_BF16)
    g.begin()
    g.gemmNT(bits, None, q, s, x, None, y, M, N, K, G)
    g.end()
    return from_dev(y)


@pytest.mark.parametrize("math,bits,shape", CASES)
def test_reserve_covers_the_call(dgm, torch_cuda, gpu, math, bits, shape):
    M, N, K, G = shape
    x, q, s = _case(gpu, M, N, K, G, bits, M + K)
    bound = gpu.gemmNT_workspace_bound(M, N, K)
    assert bound > 0
    # A context that allocates on first use, then one that reserved the bound.
    lazy = dgm.GPU(stream=torch_cuda.cuda.current_stream())
    eager = dgm.GPU(stream=torch_cuda.cuda.current_stream())
    try:
        assert lazy.workspaceBytes() == 0 and eager.workspaceBytes() == 0
        y0 = _forward(lazy, dgm, math, bits, q, s, x, M, N, K, G)
        eager.reserve(bound)
        held = eager.workspaceBytes()
        assert held >= bound
        y1 = _forward(eager, dgm, math, bits, q, s, x, M, N, K, G)
        y2 = _forward(eager, dgm, math, bits, q, s, x, M, N, K, G)
        assert eager.workspaceBytes() == held          # nothing was allocated by the calls
        assert lazy.workspaceBytes() <= max(held, 1 << 20)
        assert np.all(np.isfinite(y0))
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    finally:
        lazy.close()
        eager.close()


def test_reserve_is_monotone_and_refused_under_capture(dgm, torch_cuda):
    torch = torch_cuda
    st = torch.cuda.Stream()
    g = dgm.GPU(stream=st)
    try:
        g.reserve(3 << 20)
        held = g.workspaceBytes()
        assert held >= 3 << 20
        g.reserve(1 << 20)                            # smaller: nothing changes
        g.reserve(0)
        assert g.workspaceBytes() == held
        t = torch.zeros(16, device="cuda")
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=st):
            t.add_(1.0)
            with pytest.raises(dgm.DgmError) as err:
                g.reserve(4 * held)
            assert err.value.code == dgm.DGM_ERR_UNSUPPORTED
        assert g.workspaceBytes() == held
        with torch.cuda.stream(st):
            graph.replay()
        st.synchronize()
        assert np.all(from_dev(t) == 1.0)
        del graph
        with pytest.raises(dgm.DgmError) as err:
            g.reserve(-1)
        assert err.value.code == dgm.DGM_ERR_ARG
    finally:
        g.close()
