"""GPU parity of quant_i8 / quant_i4 (metal/kernels.metal:79-124) through the C ABI.

Bar: bit-exact scales, int8 codes and int4 packed bytes against the CPU oracle
(src/Check.swift:399-431 restated), on the reference's own check
(Check.swift:72-95: rows 5, cols 16, G 8, RNG(bits*99), std 0.3), the known
answers, every group-size code path, and the configs' full weight shapes.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu


def run_quant(gpu, dgm, w, rows, cols, group, bits, offset=0):
    import torch
    wd = to_dev(np.ascontiguousarray(w, np.float32).reshape(-1))
    nq = rows * cols if bits == 8 else rows * cols // 2
    # `offset` shifts the buffers off their natural alignment to exercise the
    # scalar path.
    qraw = torch.zeros(nq + 16, dtype=torch.uint8, device="cuda")
    sraw = torch.zeros(rows * (cols // group) + 4, dtype=torch.float32, device="cuda")
    if offset:
        wsrc = torch.zeros(rows * cols + 1, dtype=torch.float32, device="cuda")
        wsrc[1:] = wd
        wd = wsrc[1:]
    q = qraw[offset: offset + nq]
    s = sraw[:rows * (cols // group)]
    gpu.begin()
    gpu.quantize(wd, q, s, rows, cols, bits, group)
    gpu.end()
    qh = from_dev(q)
    return (qh.view(np.int8) if bits == 8 else qh), from_dev(s)


@pytest.mark.parametrize("bits", [8, 4])
def test_reference_check_quant(gpu, dgm, orc, bits):
    rows, cols, g = 5, 16, 8
    w = orc.RNG(bits * 99).randn(rows * cols, 0.3)
    q, s = run_quant(gpu, dgm, w, rows, cols, g, bits)
    qr, sr = orc.quant(w, rows, cols, g, bits)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32)), "scales exact"
    assert np.array_equal(q, qr), "codes exact"
    assert gpu.lastKernel == ("quant_i4" if bits == 4 else "quant_i8")


def test_known_answers(gpu, dgm):
    u = 2.0 ** -10
    w = (np.array([127, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5]) * u).astype(np.float32)
    q, s = run_quant(gpu, dgm, w, 1, 8, 8, 8)
    assert s[0] == np.float32(u) and q.tolist() == [127, 2, 4, -2, -4, 0, 0, 2]
    u = 2.0 ** -4
    w = (np.array([7, 2.5, 3.5, -2.5, -3.5, 0.5, -1.5, -7]) * u).astype(np.float32)
    q, s = run_quant(gpu, dgm, w, 1, 8, 8, 4)
    assert s[0] == np.float32(u) and q.tolist() == [0x27, 0xE4, 0x0C, 0x9E]
    q, s = run_quant(gpu, dgm, np.zeros(16, np.float32), 1, 16, 8, 4)
    assert s.tolist() == [np.float32(1e-8)] * 2 and not q.any()
    w = np.array([1e-7, -2.6e-8, 0.0, 4e-9, 0, 0, 0, 0], np.float32)
    q, s = run_quant(gpu, dgm, w, 1, 8, 8, 8)
    assert s[0] == np.float32(1e-8) and q.tolist()[:4] == [10, -3, 0, 0]


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group,rows,cols", [
    (2, 7, 10), (6, 5, 36), (8, 9, 64), (16, 33, 96), (32, 768, 192), (64, 17, 320),
    (128, 40, 4096), (256, 6, 512), (512, 3, 1536), (1024, 2, 2048), (12, 4, 48)])
def test_random_all_paths(gpu, dgm, orc, bits, group, rows, cols):
    rng = np.random.default_rng(rows * 31 + group + bits)
    scale = rng.choice([0.02, 0.3, 5.0])
    w = (rng.standard_normal(rows * cols) * scale).astype(np.float32)
    w[::7] *= 1e-3   # small values near the rounding boundary
    q, s = run_quant(gpu, dgm, w, rows, cols, group, bits)
    qr, sr = orc.quant(w, rows, cols, group, bits)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))
    assert np.array_equal(q, qr)


@pytest.mark.parametrize("bits", [8, 4])
def test_unaligned_buffers_take_scalar_path(gpu, dgm, orc, bits):
    rows, cols, group = 6, 64, 32
    w = orc.RNG(11).randn(rows * cols, 0.5)
    q, s = run_quant(gpu, dgm, w, rows, cols, group, bits, offset=1)
    qr, sr = orc.quant(w, rows, cols, group, bits)
    assert np.array_equal(s, sr) and np.array_equal(q, qr)


def test_exact_ties_at_scale(gpu, dgm, orc):
    # Every weight sits exactly on a half step of a power-of-two scale.
    rows, cols, group = 64, 256, 32
    rng = np.random.default_rng(9)
    half = rng.integers(-253, 254, size=(rows, cols)).astype(np.float64) / 2.0
    half[:, ::group] = 127.0
    w = (half * 2.0 ** -12).astype(np.float32)
    q, s = run_quant(gpu, dgm, w, rows, cols, group, 8)
    qr, sr = orc.quant(w, rows, cols, group, 8)
    assert np.all(s == np.float32(2.0 ** -12))
    assert np.array_equal(q, qr)


@pytest.mark.parametrize("name,rows,cols,group,bits", [
    ("c1 wup int8", 768, 192, 32, 8),
    ("c2 wdown int4", 192, 768, 32, 4),
    ("c4/c5 int4", 14336, 4096, 128, 4),
    ("c5 int8", 14336, 4096, 128, 8)])
def test_config_weights(gpu, dgm, orc, name, rows, cols, group, bits):
    rng = np.random.default_rng(rows + bits)
    w = (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.02))
    q, s = run_quant(gpu, dgm, w, rows, cols, group, bits)
    qr, sr = orc.quant(w, rows, cols, group, bits)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32)), name
    assert np.array_equal(q, qr), name


def test_kernel_level_entry_and_qmax_from_params(gpu, dgm, orc):
    rows, cols, group = 4, 64, 16
    w = orc.RNG(3).randn(rows * cols, 1.0)
    import torch
    wd = to_dev(w)
    q = torch.zeros(rows * cols, dtype=torch.int8, device="cuda")
    s = torch.zeros(rows * cols // group, dtype=torch.float32, device="cuda")
    gpu.begin()
    gpu.quant_i8(wd, q, s, dgm.QuantP(rows, cols, 127.0, group))
    gpu.end()
    qr, sr = orc.quant(w, rows, cols, group, 8)
    assert np.array_equal(from_dev(q), qr) and np.array_equal(from_dev(s), sr)


def test_error_paths(gpu, dgm):
    import torch
    w = torch.zeros(64, device="cuda")
    q = torch.zeros(64, dtype=torch.uint8, device="cuda")
    s = torch.zeros(64, device="cuda")
    with pytest.raises(dgm.DgmError) as e:       # dispatch outside begin/end
        gpu.quantize(w, q, s, 2, 32, 8, 8)
    assert e.value.code == dgm.DGM_ERR_NOT_BEGUN
    gpu.begin()
    with pytest.raises(dgm.DgmError) as e:       # odd group for int4 (Params.swift:171)
        gpu.quantize(w, q, s, 2, 30, 4, 3)
    assert e.value.code == dgm.DGM_ERR_SHAPE
    gpu.begin()
    with pytest.raises(dgm.DgmError) as e:
        gpu.quantize(w, q, s, 2, 32, 16, 8)
    assert e.value.code == dgm.DGM_ERR_BITS
    gpu.begin()
    gpu.quantize(w, q, s, 0, 32, 8, 8)           # empty: no work, no error
    gpu.end()


@pytest.mark.parametrize("bits", [8, 4])
def test_partial_last_group_left_alone(gpu, dgm, orc, bits):
    """cols % G != 0: floor(cols/G) groups per row, tail codes untouched,
    scales strided by floor(cols/G) (Check.swift:399-424, kernels.metal:86-98)."""
    import torch
    rows, cols, group = 5, 52, 8          # 6 groups + 4 tail columns per row
    w = orc.RNG(77).randn(rows * cols, 0.4)
    nq = rows * cols if bits == 8 else rows * cols // 2
    prior = (np.arange(nq) % 251).astype(np.uint8)
    q = torch.from_numpy(prior.copy()).to("cuda")
    s = torch.zeros(rows * (cols // group), device="cuda")
    gpu.begin()
    gpu.quantize(to_dev(w), q, s, rows, cols, bits, group)
    gpu.end()
    qr, sr = orc.quant(w, rows, cols, group, bits, init=prior.view(np.int8) if bits == 8 else prior)
    assert np.array_equal(from_dev(s), sr)
    assert np.array_equal(from_dev(q), qr.view(np.uint8))
