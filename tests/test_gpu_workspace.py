"""The context's grow-only workspace (staging for the decode kernels'
activation pieces) under HIP graph capture.

* A graph captured while the workspace is small keeps writing that buffer
  when replayed after a larger call has grown the workspace: the retired
  buffer stays allocated until the context is destroyed, so the replay is
  still correct.
* A call that would have to grow the workspace while its stream is being
  captured returns DGM_ERR_UNSUPPORTED and launches nothing.
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
