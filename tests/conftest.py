"""Shared fixtures. GPU tests are marked @pytest.mark.gpu; everything else runs
on the CPU. The product package is loaded from its in-tree directory; the
oracle (test infrastructure) from oracle/."""
from __future__ import annotations

import importlib.util
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "diffusion-gpt-metal_amd")
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def load_package():
    """Imports diffusion-gpt-metal_amd/ as module `dgm_amd`."""
    if "dgm_amd" in sys.modules:
        return sys.modules["dgm_amd"]
    spec = importlib.util.spec_from_file_location(
        "dgm_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["dgm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def dgm():
    return load_package()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as orc_mod
    orc_mod.lib()
    return orc_mod


@pytest.fixture(scope="session")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    return torch


@pytest.fixture(scope="session")
def gpu(dgm, torch_cuda):
    # Launch on torch's current stream: the buffers are torch tensors filled on it.
    g = dgm.GPU(stream=torch_cuda.cuda.current_stream())
    yield g
    g.close()


def to_dev(a):
    """numpy array -> device tensor (bitwise copy)."""
    import torch
    return torch.from_numpy(a.copy()).to("cuda")


def from_dev(t):
    return t.detach().cpu().numpy()


def rel_err(got, ref):
    """max |got - ref| / max |ref|, ref in float64 (the accuracy metric)."""
    import numpy as np
    ref = np.asarray(ref, dtype=np.float64)
    den = max(float(np.max(np.abs(ref))), 1e-30) if ref.size else 1.0
    return float(np.max(np.abs(np.asarray(got, dtype=np.float64) - ref))) / den if ref.size else 0.0
