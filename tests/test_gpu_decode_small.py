"""The one-launch decode kernel (M <= 16, a multiple of four scale groups per
row): activations converted inside every workgroup, no prepare pass. Against
the float64 product of the oracle's dequantized weights (the forward of
metal/kernels.metal:152-209, Check.swift:433-458), both math modes, ragged N, bias, rows of very different
magnitude, and int4/int8 group shapes up to the kernel's 64-group limit."""
import numpy as np
import pytest

from conftest import rel_err, to_dev
from test_gpu_skinny import _forward, _quantize, _ref

pytestmark = pytest.mark.gpu

SHAPES = [(4, 128, 512), (4, 128, 4096), (4, 256, 2048), (4, 512, 4096),
          (8, 64, 4096), (8, 128, 2048), (8, 64, 256)]


@pytest.mark.parametrize("bits,G,K", SHAPES)
@pytest.mark.parametrize("M,N", [(1, 64), (3, 100), (8, 257), (16, 300)])
def test_one_launch_decode(gpu, dgm, orc, bits, G, K, M, N):
    rng = np.random.default_rng(bits * 7919 + G + K + M * 31 + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0] *= np.float32(1e-3)                      # one row far below the others
    if M > 2:
        x[2, K // 3] = np.float32(3e3)            # an outlier inside one block
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if M % 2 else None
    q, s = _quantize(gpu, to_dev(w), N, K, G, bits)
    ref = _ref(orc, q, s, x.ravel(), bias, M, N, K, G, bits).reshape(M, N)
    for mode, bar in ((dgm.DGM_MATH_FP32, 1e-5), (dgm.DGM_MATH_BF16, 1e-2)):
        y = _forward(gpu, dgm, bits, q, s, x.ravel(), bias, M, N, K, G, mode).reshape(M, N)
        worst = max(rel_err(y[m], ref[m]) for m in range(M))
        assert worst <= bar, (mode, worst)


def test_one_launch_repeatable(gpu, dgm, orc):
    """Same inputs, same bits: the partials are summed in a fixed order."""
    M, N, K, G = 16, 512, 4096, 128
    rng = np.random.default_rng(5)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q, s = _quantize(gpu, to_dev(w), N, K, G, 4)
    y0 = _forward(gpu, dgm, 4, q, s, x, None, M, N, K, G, dgm.DGM_MATH_FP32)
    for _ in range(3):
        y1 = _forward(gpu, dgm, 4, q, s, x, None, M, N, K, G, dgm.DGM_MATH_FP32)
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))


def test_wait_give_up_is_reported(gpu, dgm, orc):
    """A bounded in-workgroup hand-over wait that gives up (forced by the test
    hook: one round per wait) makes dgm_end fail instead of handing back
    invalid results as if they were good; the kernel itself still ends. With
    the default bound restored the same call is exact again and dgm_end
    succeeds (the device flag was cleared by the failing end)."""
    # A shape the one-launch kernel takes (40 workgroups: too few for the
    # K-sliced kernel).
    M, N, K, G = 16, 4096, 2048, 128
    rng = np.random.default_rng(11)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q, s = _quantize(gpu, to_dev(w), N, K, G, 4)
    ref = _ref(orc, q, s, x, None, M, N, K, G, 4)
    lib = dgm.load_library()
    reported = False
    try:
        assert lib.dgm_debug_wait_limit(1) == dgm.DGM_OK
        for _ in range(5):   # one round per wait: some wait gives up in practice on the first call
            try:
                _forward(gpu, dgm, 4, q, s, x, None, M, N, K, G, dgm.DGM_MATH_FP32)
            except dgm.DgmError as e:
                assert e.code == dgm.DGM_ERR_HIP
                assert "gave up" in gpu.lastError
                reported = True
                break
    finally:
        assert lib.dgm_debug_wait_limit(0) == dgm.DGM_OK
    assert reported
    y = _forward(gpu, dgm, 4, q, s, x, None, M, N, K, G, dgm.DGM_MATH_FP32)
    assert rel_err(y, ref) <= 1e-5
