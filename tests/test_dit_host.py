"""CPU checks of the DiT block's host side: RoPE tables, config plumbing and
workspace sizing (no GPU calls)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest


@pytest.mark.parametrize("T,D,theta", [(64, 48, 1e4), (1, 2, 1e4), (17, 10, 500.0), (128, 64, 1e4)])
def test_rope_tables_match_oracle_bit_for_bit(dgm, orc, T, D, theta):
    c, s = dgm.rope_tables(T, D, theta)
    oc, os_ = orc.rope_tables(T, D, theta)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)
    # Row 0 is the identity rotation; both halves repeat.
    assert np.all(c.reshape(T, D)[0] == 1.0) and np.all(s.reshape(T, D)[0] == 0.0)
    assert np.array_equal(c.reshape(T, D)[:, : D // 2], c.reshape(T, D)[:, D // 2:])


def test_rope_tables_reject_odd_dim(dgm):
    with pytest.raises(dgm.DgmError):
        dgm.rope_tables(4, 3, 1e4)


def test_config_struct_and_shapes(dgm):
    cfg = dgm.DiTConfig()
    c = cfg.c_cfg()
    assert ctypes.sizeof(dgm.DiTCfg) == 48
    assert (c.B, c.T, c.C, c.F, c.H, c.D, c.loops, c.group, c.bits) == (8, 64, 192, 768, 4, 48, 4, 32, 8)
    shapes = cfg.linear_shapes()
    # src/DiT.swift:242-248, KV = one head of D.
    assert shapes == {"wq": (192, 192), "wk": (48, 192), "wv": (48, 192), "wo": (192, 192),
                      "wgate": (768, 192), "wup": (768, 192), "wdown": (192, 768)}
    assert ctypes.sizeof(dgm.DiTWeights) == 7 * 3 * 8 + 5 * 8


def test_workspace_size_matches_host_layout(dgm):
    from dgm_amd.dit import _ws_sizes
    lib = dgm.load_library()
    for cfg in (dgm.DiTConfig(), dgm.DiTConfig(B=2, T=16, C=64, F=128, H=4, D=16)):
        c = cfg.c_cfg()
        n = lib.dgm_dit_workspace_floats(ctypes.byref(c))
        assert n == sum((sz + 63) & ~63 for _, sz in _ws_sizes(cfg))
    assert lib.dgm_dit_workspace_floats(None) == -1
