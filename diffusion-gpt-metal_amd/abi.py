"""ctypes binding of include/dgm_quant.h (libdgm_amd.so).

Only plumbing: prototypes, the parameter-block structs and the status
codes. The HIP library is required; there is no fallback of any kind, and a
missing library raises at load time.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libdgm_amd.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "dgm_quant.h")

DGM_OK = 0
DGM_ERR_ARG = 1
DGM_ERR_SHAPE = 2
DGM_ERR_NOT_BEGUN = 3
DGM_ERR_HIP = 4
DGM_ERR_BITS = 5
DGM_ERR_UNSUPPORTED = 6

DGM_MATH_FP32 = 0
DGM_MATH_BF16 = 1
DGM_NOALLOC_SCRATCH_BYTES = 8 << 20   # static scratch of dgm_gemmNT_noalloc (include/dgm_quant.h)


class GemmP(ctypes.Structure):
    """src/Params.swift:7-16 — eight u32, 32 bytes."""
    _fields_ = [(n, ctypes.c_uint32) for n in ("M", "N", "K", "hasBias", "qGroup", "pad0", "pad1", "pad2")]


class QuantP(ctypes.Structure):
    """src/Params.swift:18-23 — rows, cols, qmax (f32), qGroup; 16 bytes."""
    _fields_ = [("rows", ctypes.c_uint32), ("cols", ctypes.c_uint32),
                ("qmax", ctypes.c_float), ("qGroup", ctypes.c_uint32)]


assert ctypes.sizeof(GemmP) == 32 and ctypes.sizeof(QuantP) == 16


class DiTCfg(ctypes.Structure):
    """dgm_dit_cfg: the DiTConfig fields the loop body reads (src/DiT.swift:9-41)."""
    _fields_ = ([(n, ctypes.c_int32) for n in ("B", "T", "C", "F", "H", "D", "loops", "group", "bits")]
                + [("eps", ctypes.c_float), ("mix", ctypes.c_float), ("pad", ctypes.c_int32)])


class DiTLinear(ctypes.Structure):
    """dgm_dit_linear: fp32 weight (bits 32) or codes + scales (bits 8 / 4)."""
    _fields_ = [("w", ctypes.c_void_p), ("q", ctypes.c_void_p), ("scale", ctypes.c_void_p)]


DIT_LINEARS = ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")
DIT_NORMS = ("n1", "n1b", "n2", "n2b", "nf")


class DiTWeights(ctypes.Structure):
    """dgm_dit_weights: the block's parameters (src/DiT.swift:242-253)."""
    _fields_ = [(n, DiTLinear) for n in DIT_LINEARS] + [(n, ctypes.c_void_p) for n in DIT_NORMS]


class DiTGrads(ctypes.Structure):
    """dgm_dit_grads: fp32 gradients (+=) of the seven linears and five norms."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")] + \
               [(n, ctypes.c_void_p) for n in ("n1", "n1b", "n2", "n2b", "nf")]


class TgmtHeader(ctypes.Structure):
    """dgm_tgmt_header: GPT.save's header fields (src/GPT.swift:265-281)."""
    _fields_ = [(n, ctypes.c_uint32) for n in ("version", "bits", "vocab", "block", "layers", "heads", "embd",
                                               "qGroup")]


class TditHeader(ctypes.Structure):
    """dgm_tdit_header: DiT.save's header fields (src/DiT.swift:396-411)."""
    _fields_ = [(n, ctypes.c_uint32) for n in ("version", "side", "patch", "names", "loops", "heads", "kvHeads",
                                               "embd", "intermediate", "freqDim", "diffusionSteps")] + \
               [("lastAlpha", ctypes.c_float), ("valueMix", ctypes.c_float), ("header_bytes", ctypes.c_uint32)]


class ParamInfo(ctypes.Structure):
    """dgm_param_info: one parameter of a checkpoint."""
    _fields_ = [("name", ctypes.c_char * 32), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                ("quantized", ctypes.c_int32), ("decay", ctypes.c_int32), ("offset", ctypes.c_int64)]


def _u32s(*names):
    return [(n, ctypes.c_uint32) for n in names]


class AdamP(ctypes.Structure):
    """src/Params.swift:138-147 — n (u32) and seven f32; 32 bytes."""
    _fields_ = [("n", ctypes.c_uint32)] + [(n, ctypes.c_float) for n in
                                          ("lr", "b1", "b2", "eps", "wd", "invBC1", "invBC2")]


class EmbP(ctypes.Structure):
    """src/Params.swift:78-83."""
    _fields_ = _u32s("B", "T", "C", "qGroup")


class EmbBwdP(ctypes.Structure):
    """src/Params.swift:85-90."""
    _fields_ = _u32s("B", "T", "C", "V")


class PosP(ctypes.Structure):
    """src/Params.swift:92-97."""
    _fields_ = _u32s("B", "T", "C", "pad")


class BiasP(ctypes.Structure):
    """src/Params.swift:46-51."""
    _fields_ = _u32s("M", "N", "pad0", "pad1")


class ReduceP(ctypes.Structure):
    """src/Params.swift:106-111."""
    _fields_ = _u32s("n", "slot", "pad0", "pad1")


class ScaleP(ctypes.Structure):
    """src/Params.swift:39-44."""
    _fields_ = [("n", ctypes.c_uint32), ("s", ctypes.c_float), ("pad0", ctypes.c_uint32), ("pad1", ctypes.c_uint32)]


class UnaryP(ctypes.Structure):
    """src/Params.swift:32-37."""
    _fields_ = _u32s("n", "pad0", "pad1", "pad2")


assert ctypes.sizeof(AdamP) == 32
assert all(ctypes.sizeof(t) == 16 for t in (EmbP, EmbBwdP, PosP, BiasP, ReduceP, ScaleP, UnaryP))

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_GP = ctypes.POINTER(GemmP)
_QP = ctypes.POINTER(QuantP)

# name -> (restype, argtypes); every function of include/dgm_quant.h.
PROTOTYPES = {
    "dgm_gpu_create": (_I, [ctypes.POINTER(_P)]),
    "dgm_gpu_destroy": (None, [_P]),
    "dgm_gpu_set_stream": (_I, [_P, _P]),
    "dgm_gpu_stream": (_P, [_P]),
    "dgm_set_math": (_I, [_P, _I]),
    "dgm_get_math": (_I, [_P]),
    "dgm_begin": (_I, [_P]),
    "dgm_end": (_I, [_P]),
    "dgm_last_kernel": (ctypes.c_char_p, [_P]),
    "dgm_last_error": (ctypes.c_char_p, [_P]),
    "dgm_quant_i8": (_I, [_P, _P, _P, _P, _QP]),
    "dgm_quant_i4": (_I, [_P, _P, _P, _P, _QP]),
    "dgm_gemm_nt_f32": (_I, [_P, _P, _P, _P, _P, _GP]),
    "dgm_gemm_nt_i8": (_I, [_P, _P, _P, _P, _P, _P, _GP]),
    "dgm_gemm_nt_i4": (_I, [_P, _P, _P, _P, _P, _P, _GP]),
    "dgm_gemm_dx_f32": (_I, [_P, _P, _P, _P, _GP]),
    "dgm_gemm_dx_i8": (_I, [_P, _P, _P, _P, _P, _GP]),
    "dgm_gemm_dx_i4": (_I, [_P, _P, _P, _P, _P, _GP]),
    "dgm_gemm_dw": (_I, [_P, _P, _P, _P, _GP]),
    "dgm_gemm_dw_acc": (_I, [_P, _P, _P, _P, _GP]),
    "dgm_quantize": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_gemmNT": (_I, [_P, _I64, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_gemmNT_noalloc": (_I, [_P, _I64, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_gemmNT_workspace_bound": (_I64, [_I64, _I64, _I64]),
    "dgm_gpu_reserve": (_I, [_P, _I64]),
    "dgm_gpu_workspace_bytes": (_I64, [_P]),
    "dgm_probe_read": (_I, [_P, _P, _I64, _I64, _I64, _P]),
    "dgm_probe_gemv_valu": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_debug_wait_limit": (_I, [_I64]),
    "dgm_gemmDX": (_I, [_P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_gemmDW": (_I, [_P, _P, _P, _P, _I64, _I64, _I64]),
    "dgm_gemmDWAcc": (_I, [_P, _P, _P, _P, _I64, _I64, _I64]),
    "dgm_gemmBwd": (_I, [_P, _I64, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I]),
    "dgm_rmsFwd": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _F]),
    "dgm_ropeFwd": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_repeatHeads": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_attnFwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I]),
    "dgm_swigluFwd": (_I, [_P, _P, _P, _P, _I64]),
    "dgm_add": (_I, [_P, _P, _P, _P, _I64]),
    "dgm_mix": (_I, [_P, _P, _P, _P, _I64, _F, _F]),
    "dgm_copy": (_I, [_P, _P, _P, _I64]),
    "dgm_ropeTables": (_I, [_I64, _I64, _F, _P, _P]),
    "dgm_dit_workspace_floats": (_I64, [ctypes.POINTER(DiTCfg)]),
    "dgm_dit_forward": (_I, [_P, ctypes.POINTER(DiTCfg), ctypes.POINTER(DiTWeights), _P, _P, _P, _P, _I64]),
    "dgm_tgmt_parse": (_I, [_P, _I64, ctypes.POINTER(TgmtHeader), ctypes.POINTER(_I64), ctypes.POINTER(_I64)]),
    "dgm_tgmt_param": (_I, [ctypes.POINTER(TgmtHeader), _I64, ctypes.POINTER(ParamInfo)]),
    "dgm_tdit_parse": (_I, [_P, _I64, ctypes.POINTER(TditHeader), ctypes.POINTER(_I64)]),
    "dgm_tdit_param": (_I, [ctypes.POINTER(TditHeader), _I64, ctypes.POINTER(ParamInfo)]),
    "dgm_rmsBwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _F]),
    "dgm_attnBwd": (_I, [_P] * 11 + [_I64] * 4),
    "dgm_ropeBwd": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_swigluBwd": (_I, [_P, _P, _P, _P, _P, _P, _I64]),
    "dgm_sumHeads": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_acc": (_I, [_P, _P, _P, _I64]),
    "dgm_accScale": (_I, [_P, _P, _P, _I64, _F]),
    "dgm_dit_acts_floats": (_I64, [ctypes.POINTER(DiTCfg)]),
    "dgm_dit_backward_ws_floats": (_I64, [ctypes.POINTER(DiTCfg)]),
    "dgm_dit_forward_train": (_I, [_P, ctypes.POINTER(DiTCfg), ctypes.POINTER(DiTWeights), _P, _P, _P, _P, _I64]),
    "dgm_dit_backward": (_I, [_P, ctypes.POINTER(DiTCfg), ctypes.POINTER(DiTWeights), ctypes.POINTER(DiTGrads),
                              _P, _P, _P, _I64, _P, _P, _I64]),
    "dgm_adamw": (_I, [_P, _P, _P, _P, _P, ctypes.POINTER(AdamP)]),
    "dgm_adam": (_I, [_P, _P, _P, _P, _P, _I64] + [_F] * 7),
    "dgm_adam_quantize": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64] + [_F] * 7),
    "dgm_reduce_sumsq": (_I, [_P, _P, _P, ctypes.POINTER(ReduceP)]),
    "dgm_reduceSumsq": (_I, [_P, _P, _P, _I64, _I64]),
    "dgm_zero_f": (_I, [_P, _P, ctypes.POINTER(UnaryP)]),
    "dgm_scale_f": (_I, [_P, _P, ctypes.POINTER(ScaleP)]),
    "dgm_zero": (_I, [_P, _P, _I64]),
    "dgm_scale": (_I, [_P, _P, _I64, _F]),
    "dgm_embed_f32": (_I, [_P, _P, _P, _P, _P, ctypes.POINTER(EmbP)]),
    "dgm_embed_i8": (_I, [_P, _P, _P, _P, _P, _P, ctypes.POINTER(EmbP)]),
    "dgm_embed_i4": (_I, [_P, _P, _P, _P, _P, _P, ctypes.POINTER(EmbP)]),
    "dgm_embed": (_I, [_P, _I64, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_embed_bwd": (_I, [_P, _P, _P, _P, ctypes.POINTER(EmbBwdP)]),
    "dgm_embedBwd": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64]),
    "dgm_pos_bwd": (_I, [_P, _P, _P, ctypes.POINTER(PosP)]),
    "dgm_posBwd": (_I, [_P, _P, _P, _I64, _I64, _I64]),
    "dgm_bias_grad": (_I, [_P, _P, _P, ctypes.POINTER(BiasP)]),
    "dgm_biasGrad": (_I, [_P, _P, _P, _I64, _I64]),
}


class DgmError(RuntimeError):
    """A nonzero status from the C ABI (the reference's fatalError/exit path)."""

    def __init__(self, code: int, message: str, kernel: str = ""):
        super().__init__(f"dgm status {code} ({kernel}): {message}")
        self.code = code
        self.message = message
        self.kernel = kernel


_LIB = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads libdgm_amd.so and installs prototypes. Raises if it is not built."""
    global _LIB
    if _LIB is not None and path == LIB_PATH:
        return _LIB
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is not built; run python diffusion-gpt-metal_amd/build.py "
            "(or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path == LIB_PATH:
        _LIB = lib
    return lib
