"""The measurement probes (no counterpart in the reference): the VALU GEMV the
decode kernels are compared against gives the dequantized product (fp32 FMAs:
max relative error 1e-5 against float64), and the register read probe stores
the fold of each workgroup's first thread."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, rel_err, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K,G", [(1, 14336, 4096, 128), (16, 1000, 4096, 128), (1, 37, 512, 32),
                                     (16, 70, 1024, 256)])
def test_valu_gemv_matches_dequant_product(gpu, dgm, orc, M, N, K, G):
    import torch
    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q = torch.zeros(N * K // 2, dtype=torch.uint8, device="cuda")
    s = torch.zeros(N * (K // G), device="cuda")
    y = torch.full((M * N,), float("nan"), device="cuda")
    gpu.begin()
    gpu.quantize(to_dev(w), q, s, N, K, 4, G)
    gpu.probeGemvValu(q, s, to_dev(x.ravel()), y, M, N, K, G)
    gpu.end()
    wd = orc.dequant(from_dev(q), from_dev(s), N, K, G, 4).reshape(N, K)
    ref = x.astype(np.float64) @ wd.astype(np.float64).T
    assert rel_err(from_dev(y).reshape(M, N), ref) <= 1e-5


def test_valu_gemv_rejects_other_m(gpu, dgm):
    import torch
    q = torch.zeros(64 * 32, dtype=torch.uint8, device="cuda")
    s = torch.ones(64, device="cuda")
    x = torch.zeros(4 * 64, device="cuda")
    y = torch.zeros(4 * 64, device="cuda")
    gpu.begin()
    with pytest.raises(dgm.DgmError) as e:
        gpu.probeGemvValu(q, s, x, y, 4, 64, 64, 64)
    assert e.value.code == dgm.DGM_ERR_UNSUPPORTED
    gpu.begin()
    gpu.end()


def _reg_probe_fold(words: np.ndarray, grid: int) -> np.ndarray:
    """What probe mode 0 stores per workgroup: thread 0's XOR over its 16-byte
    units i, i + 256, ... i + 7 * 256 of each pass (units past its share
    re-read unit i), passes 2048 units apart."""
    u = words.view(np.uint32).reshape(-1, 4)
    n16 = u.shape[0]
    per = -(-n16 // grid)
    out = np.zeros(grid, dtype=np.uint32)
    for blk in range(grid):
        b, e = blk * per, min(blk * per + per, n16)
        acc = np.uint32(0)
        for i in range(b, e, 2048):
            for k in range(8):
                j = i + 256 * k
                v = u[j if j < e else i]
                acc ^= v[0] ^ v[1] ^ v[2] ^ v[3]
        out[blk] = acc
    return out


def test_read_probe(gpu, dgm):
    import torch
    n = 1 << 18
    words = (np.arange(n, dtype=np.int64) * 2654435761 % (1 << 31)).astype(np.int32)
    src = to_dev(words)
    sink = torch.zeros(8, dtype=torch.int32, device="cuda")
    gpu.begin()
    gpu.probeRead(src, n * 4, 0, 8, sink)
    gpu.probeRead(src, n * 4, 1, 8, sink)   # direct-to-LDS: the launch succeeds
    gpu.end()
    sink0 = torch.zeros(8, dtype=torch.int32, device="cuda")
    gpu.begin()
    gpu.probeRead(src, n * 4, 0, 8, sink0)
    gpu.end()
    want = _reg_probe_fold(words, 8)
    assert np.array_equal(from_dev(sink0).view(np.uint32), want)
