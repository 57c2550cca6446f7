"""MI355X (gfx950) group-quantized linear path: host side of libdgm_amd.so.

The directory name is not a Python identifier, so load it with
    importlib.util.spec_from_file_location("dgm_amd", ".../__init__.py",
        submodule_search_locations=[".../diffusion-gpt-metal_amd"])
(see load_package() in tests/conftest.py and bench.py).
"""
from .abi import (DGM_ERR_ARG, DGM_ERR_BITS, DGM_ERR_HIP, DGM_ERR_NOT_BEGUN,
                  DGM_ERR_SHAPE, DGM_ERR_UNSUPPORTED, DGM_MATH_BF16,
                  DGM_MATH_FP32, DGM_NOALLOC_SCRATCH_BYTES, DGM_OK, HEADER, LIB_PATH, PROTOTYPES,
                  DIT_LINEARS, DIT_NORMS, DgmError, DiTCfg, DiTLinear,
                  DiTWeights, GemmP, QuantP, AdamP, EmbP, EmbBwdP, PosP, BiasP,
                  ReduceP, ScaleP, UnaryP, DiTGrads, load_library)
from .gpu import GPU, Buf, RawBuf
from .dit import DiTBlock, DiTConfig, rope_tables
from .train import Param, bias_corrections, grad_norm, optimizer_step, zero_grads
from .ckpt import load_dit_block, load_gpt, read_tdit, read_tgmt, save_tdit, save_tgmt

__all__ = [
    "GPU", "Buf", "RawBuf", "GemmP", "QuantP", "DgmError", "load_library",
    "LIB_PATH", "HEADER", "PROTOTYPES", "DGM_OK", "DGM_ERR_ARG", "DGM_ERR_SHAPE",
    "DGM_ERR_NOT_BEGUN", "DGM_ERR_HIP", "DGM_ERR_BITS", "DGM_ERR_UNSUPPORTED",
    "DGM_MATH_FP32", "DGM_MATH_BF16", "DGM_NOALLOC_SCRATCH_BYTES", "DiTBlock", "DiTConfig", "DiTCfg", "DiTLinear",
    "DiTWeights", "DIT_LINEARS", "DIT_NORMS", "rope_tables", "AdamP", "EmbP", "EmbBwdP",
    "PosP", "BiasP", "ReduceP", "ScaleP", "UnaryP", "Param", "bias_corrections", "grad_norm",
    "optimizer_step", "zero_grads", "DiTGrads", "load_dit_block", "load_gpt", "read_tdit", "read_tgmt",
    "save_tdit", "save_tgmt",
]
