"""Checkpoint layouts (CPU): TGMT (src/GPT.swift:265-324) and TDIT
(src/DiT.swift:396-451) through the library's parsers.

Pinned by: our writer's files round-trip; the parameter order, shapes and
flags restate GPT.init / Block.init / DiT.init's make() calls; every file the
reference would reject (magic, version, configuration, length) is rejected;
and the reference's own photos-dit checkpoint (when /root/reference is
present) parses to the header the DiT config implies, with the block's wup
statistics (768 x 192, max |w| 0.43, rms 0.072) that the survey of the
checkpoint recorded.
"""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

REF_DIT = "/root/reference/build/photos-dit.ckpt"


def _gpt_masters(h, rng):
    C, V, Tb, F = h["embd"], h["vocab"], h["block"], 4 * h["embd"]
    shapes = [("wte", V, C, True, True), ("wpe", Tb, C, False, True)]
    for l in range(h["layers"]):
        for name, r, c, q, d in [("ln1.g", C, 1, False, False), ("ln1.b", C, 1, False, False),
                                 ("wq", C, C, True, True), ("bq", C, 1, False, False),
                                 ("wk", C, C, True, True), ("bk", C, 1, False, False),
                                 ("wv", C, C, True, True), ("bv", C, 1, False, False),
                                 ("wo", C, C, True, True), ("bo", C, 1, False, False),
                                 ("ln2.g", C, 1, False, False), ("ln2.b", C, 1, False, False),
                                 ("fc", F, C, True, True), ("fc.b", F, 1, False, False),
                                 ("proj", C, F, True, True), ("proj.b", C, 1, False, False)]:
            shapes.append((f"b{l}.{name}", r, c, q, d))
    shapes += [("ln_f.g", C, 1, False, False), ("ln_f.b", C, 1, False, False)]
    return shapes, [rng.standard_normal(r * c).astype(np.float32) for _, r, c, _, _ in shapes]


GPT_H = dict(version=1, bits=4, vocab=11, block=8, layers=2, heads=2, embd=16, qGroup=8)


def test_tgmt_round_trip(dgm, tmp_path):
    rng = np.random.default_rng(0)
    shapes, masters = _gpt_masters(GPT_H, rng)
    itos = bytes(range(65, 65 + GPT_H["vocab"]))
    path = tmp_path / "m.ckpt"
    dgm.save_tgmt(path, GPT_H, itos, masters)
    h, it, params = dgm.read_tgmt(path)
    assert h == GPT_H and it == itos
    assert len(params) == 2 + 16 * GPT_H["layers"] + 2
    for (name, r, c, q, d), m, p in zip(shapes, masters, params):
        assert (p.name, p.rows, p.cols, p.quantized, p.decay) == (name, r, c, q and GPT_H["bits"] != 32, d)
        assert np.array_equal(p.data, m)
    assert os.path.getsize(path) == 36 + GPT_H["vocab"] + 4 * sum(m.size for m in masters)


def test_tgmt_rejects(dgm, tmp_path):
    rng = np.random.default_rng(1)
    _, masters = _gpt_masters(GPT_H, rng)
    good = tmp_path / "good.ckpt"
    dgm.save_tgmt(good, GPT_H, bytes(GPT_H["vocab"]), masters)
    raw = good.read_bytes()
    cases = {"short": raw[:-4], "long": raw + b"\0\0\0\0", "magic": b"TGMX" + raw[4:],
             "version": raw[:4] + struct.pack("<I", 2) + raw[8:]}
    for name, h in (("heads", dict(GPT_H, heads=3)), ("odd group", dict(GPT_H, qGroup=5)),
                    ("bits", dict(GPT_H, bits=16))):
        p = tmp_path / f"{name}.ckpt"
        dgm.save_tgmt(p, h, bytes(h["vocab"]), masters)
        cases[name] = p.read_bytes()
    for name, data in cases.items():
        p = tmp_path / f"bad_{name.replace(' ', '_')}.ckpt"
        p.write_bytes(data)
        with pytest.raises(dgm.DgmError) as e:
            dgm.read_tgmt(p)
        assert e.value.code == dgm.DGM_ERR_SHAPE, name


TDIT_H = dict(side=16, patch=4, names=3, loops=2, heads=2, kvHeads=1, embd=16, intermediate=32, freqDim=8,
              diffusionSteps=10, lastAlpha=0.02, valueMix=0.5)


def _tdit_masters(h, rng):
    C, F, P, KV = h["embd"], h["intermediate"], h["patch"] ** 2 * 3, h["embd"] // h["heads"]
    shapes = [("wpatch", C, P), ("whead", P, C), ("wname", h["names"], C), ("wtime1", C, h["freqDim"]),
              ("wtime2", C, C), ("wq", C, C), ("wk", KV, C), ("wv", KV, C), ("wo", C, C), ("wgate", F, C),
              ("wup", F, C), ("wdown", C, F)] + [(n, C, 1) for n in ("n1", "n1b", "n2", "n2b", "nf")]
    return shapes, [rng.standard_normal(r * c).astype(np.float32) for _, r, c in shapes]


@pytest.mark.parametrize("version", [1, 2])
def test_tdit_round_trip(dgm, tmp_path, version):
    rng = np.random.default_rng(version)
    shapes, masters = _tdit_masters(TDIT_H, rng)
    path = tmp_path / "d.ckpt"
    dgm.save_tdit(path, TDIT_H, masters, version=version)
    h, params = dgm.read_tdit(path)
    assert h["version"] == version and h["valueMix"] == 0.5
    assert h["lastAlpha"] == (np.float32(0.02) if version == 2 else np.float32(0.01))   # DiT.load's v1 default
    for (name, r, c), m, p in zip(shapes, masters, params):
        assert (p.name, p.rows, p.cols, p.quantized, p.decay) == (name, r, c, False, name == "wname")
        assert np.array_equal(p.data, m)
    bad = tmp_path / "bad.ckpt"
    bad.write_bytes(path.read_bytes()[:-1])
    with pytest.raises(dgm.DgmError):
        dgm.read_tdit(bad)
    two_kv = tmp_path / "kv.ckpt"
    dgm.save_tdit(two_kv, dict(TDIT_H, kvHeads=2), masters)     # this build repeats a single KV head
    with pytest.raises(dgm.DgmError):
        dgm.read_tdit(two_kv)


@pytest.mark.skipif(not os.path.exists(REF_DIT), reason="the reference's checkpoints are not on this machine")
def test_reference_photos_dit_checkpoint(dgm):
    h, params = dgm.read_tdit(REF_DIT)
    assert {k: h[k] for k in ("side", "patch", "names", "loops", "heads", "kvHeads", "embd", "intermediate",
                              "freqDim", "diffusionSteps")} == dict(
        side=128, patch=16, names=14, loops=4, heads=4, kvHeads=1, embd=192, intermediate=768, freqDim=192,
        diffusionSteps=100)
    assert h["valueMix"] == 0.5
    by = {p.name: p for p in params}
    assert [p.name for p in params][5:12] == ["wq", "wk", "wv", "wo", "wgate", "wup", "wdown"]
    for p in params:
        assert np.all(np.isfinite(p.data))
    wup = by["wup"]
    assert (wup.rows, wup.cols) == (768, 192)
    assert abs(float(np.max(np.abs(wup.data))) - 0.43) < 0.01
    assert abs(float(np.sqrt(np.mean(wup.data.astype(np.float64) ** 2))) - 0.072) < 0.002
