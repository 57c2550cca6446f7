"""numpy binding of the CPU oracle (liboracle.so) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker or the timed CPU baseline. The product
library never uses it.

Each function names the reference routine it restates (paths relative to the
reference root); the C source (oracle.c) carries the same citations.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f = ctypes.POINTER(ctypes.c_float)
_P = ctypes.c_void_p
_i64 = ctypes.c_int64
_i = ctypes.c_int
_u64 = ctypes.c_uint64

_lib = None


class _Rng(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint64)]


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing; run oracle/build.sh")
        L = ctypes.CDLL(LIB_PATH)
        R = ctypes.POINTER(_Rng)
        protos = {
            "orc_rng_init": (None, [R, _u64]),
            "orc_rng_next": (_u64, [R]),
            "orc_rng_uniform": (ctypes.c_float, [R]),
            "orc_rng_normal": (ctypes.c_float, [R]),
            "orc_normal_stream": (_u64, [_u64, _P, _i64, ctypes.c_float]),
            "orc_quant_code": (_i, [ctypes.c_float, ctypes.c_float, _i]),
            "orc_quant": (_i, [_P, _i64, _i64, _i, _i, _P, _P, _P]),
            "orc_dequant": (_i, [_P, _P, _i64, _i64, _i, _i, _P]),
            "orc_gemm_nt": (None, [_P, _P, _P, _P, _i64, _i64, _i64]),
            "orc_gemm_dx": (None, [_P, _P, _P, _i64, _i64, _i64]),
            "orc_gemm_dw": (None, [_P, _P, _P, _i64, _i64, _i64, _i]),
            "orc_gemm_nt_q": (_i, [_P, _P, _P, _P, _P, _i64, _i64, _i64, _i, _i]),
            "orc_gemm_dx_q": (_i, [_P, _P, _P, _P, _i64, _i64, _i64, _i, _i]),
            "orc_rmsnorm_fwd": (None, [_P, _P, _P, _P, _i64, _i64, ctypes.c_float]),
            "orc_rope_tables": (None, [_i, _i, ctypes.c_float, _P, _P]),
            "orc_rope_fwd": (None, [_P, _P, _P, _P, _i, _i, _i, _i]),
            "orc_repeat_heads": (None, [_P, _P, _i, _i, _i, _i]),
            "orc_attn_fwd": (None, [_P, _P, _P, _P, _P, _P, _i, _i, _i, _i, _i]),
            "orc_swiglu_fwd": (None, [_P, _P, _P, _i64]),
            "orc_add": (None, [_P, _P, _P, _i64]),
            "orc_mix": (None, [_P, _P, _P, _i64, ctypes.c_float, ctypes.c_float]),
            "orc_dit_workspace_floats": (_i64, [_P]),
            "orc_dit_forward": (_i, [_P] + [_P] * 14 + [_P] * 5 + [_P, _P]),
            "orc_adamw": (None, [_P, _P, _P, _P, _i64] + [ctypes.c_float] * 7),
            "orc_reduce_sumsq": (ctypes.c_float, [_P, _i64]),
            "orc_scale": (None, [_P, _i64, ctypes.c_float]),
            "orc_embed": (_i, [_P, _P, _P, _P, _P, _P, _i, _i, _i, _i, _i]),
            "orc_embed_bwd": (None, [_P, _P, _P, _i, _i, _i, _i]),
            "orc_pos_bwd": (None, [_P, _P, _i, _i, _i]),
            "orc_bias_grad": (None, [_P, _P, _i64, _i64]),
            "orc_rms_bwd": (None, [_P, _P, _P, _P, _P, _P, _i64, _i64]),
            "orc_attn_bwd": (None, [_P] * 10 + [_i, _i, _i, _i]),
            "orc_rope_bwd": (None, [_P, _P, _P, _P, _i, _i, _i, _i]),
            "orc_swiglu_bwd": (None, [_P, _P, _P, _P, _P, _i64]),
            "orc_sum_heads": (None, [_P, _P, _i, _i, _i, _i]),
            "orc_acc_scale": (None, [_P, _P, _i64, ctypes.c_float]),
            "orc_dit_train_floats": (_i64, [_P]),
            "orc_dit_train": (_i, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
        }
        for name, (res, args) in protos.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- RNG: src/GPU.swift:4-29 ---------------------------------------------

class RNG:
    """SplitMix64 + Box-Muller, src/GPU.swift:4-29."""

    def __init__(self, seed: int):
        self._s = _Rng()
        lib().orc_rng_init(ctypes.byref(self._s), seed)

    @property
    def state(self) -> int:
        return self._s.state

    def next(self) -> int:
        return lib().orc_rng_next(ctypes.byref(self._s))

    def uniform(self) -> float:
        return lib().orc_rng_uniform(ctypes.byref(self._s))

    def normal(self) -> float:
        return lib().orc_rng_normal(ctypes.byref(self._s))

    def randn(self, n: int, std: float) -> np.ndarray:
        """n draws of normal() * std (Check.swift randn / GPT.swift fillNormal)."""
        out = np.empty(n, dtype=np.float32)
        self._s.state = lib().orc_normal_stream(self._s.state, _p(out), n, std)
        return out


# ---- quantize / dequant: Check.swift:399-458 -------------------------------

def quant(w: np.ndarray, rows: int, cols: int, group: int, bits: int, init=None):
    """cpuQuant (Check.swift:399-424). Returns (codes, scales); codes are
    int8 [rows*cols] for bits 8 and packed uint8 [rows*cols/2] for bits 4.
    `init` gives the codes' prior contents (tail columns of a row that is not
    a whole number of groups keep them; zeros by default)."""
    w = _f32(w).reshape(-1)
    assert w.size == rows * cols
    scale = np.zeros(rows * (cols // group), dtype=np.float32)
    if bits == 8:
        q = np.zeros(rows * cols, dtype=np.int8) if init is None else np.array(init, dtype=np.int8)
        rc = lib().orc_quant(_p(w), rows, cols, group, 8, _p(q), None, _p(scale))
    else:
        q = np.zeros(rows * cols // 2, dtype=np.uint8) if init is None else np.array(init, dtype=np.uint8)
        rc = lib().orc_quant(_p(w), rows, cols, group, 4, None, _p(q), _p(scale))
    if rc != 0:
        raise ValueError("oracle rejected the quantization shape")
    return q, scale


def quant_code(w: float, s: float, lim: int) -> int:
    return lib().orc_quant_code(w, s, lim)


def dequant(q: np.ndarray, scale: np.ndarray, rows: int, cols: int, group: int, bits: int) -> np.ndarray:
    """dequant (Check.swift:433-458) for any group size."""
    out = np.zeros(rows * cols, dtype=np.float32)
    q = np.ascontiguousarray(q)
    scale = _f32(scale)
    if lib().orc_dequant(_p(q), _p(scale), rows, cols, group, bits, _p(out)) != 0:
        raise ValueError("oracle rejected the dequant shape")
    return out


# ---- GEMMs: Check.swift:460-494, kernels.metal:152-283 ---------------------

def gemm_nt(x, w, bias, M, N, K):
    x, w = _f32(x), _f32(w)
    b = None if bias is None else _f32(bias)
    y = np.zeros(M * N, dtype=np.float32)
    lib().orc_gemm_nt(_p(x), _p(w), _p(b), _p(y), M, N, K)
    return y


def gemm_dx(dy, w, M, N, K):
    dy, w = _f32(dy), _f32(w)
    dx = np.zeros(M * K, dtype=np.float32)
    lib().orc_gemm_dx(_p(dy), _p(w), _p(dx), M, N, K)
    return dx


def gemm_dw(dy, x, M, N, K, dw=None):
    dy, x = _f32(dy), _f32(x)
    acc = dw is not None
    out = np.array(dw, dtype=np.float32, copy=True) if acc else np.zeros(N * K, dtype=np.float32)
    lib().orc_gemm_dw(_p(dy), _p(x), _p(out), M, N, K, 1 if acc else 0)
    return out


def gemm_nt_q(q, scale, x, bias, M, N, K, group, bits):
    q = np.ascontiguousarray(q)
    scale, x = _f32(scale), _f32(x)
    b = None if bias is None else _f32(bias)
    y = np.zeros(M * N, dtype=np.float32)
    if lib().orc_gemm_nt_q(_p(q), _p(scale), _p(x), _p(b), _p(y), M, N, K, group, bits):
        raise ValueError("bad shape")
    return y


def gemm_dx_q(q, scale, dy, M, N, K, group, bits):
    q = np.ascontiguousarray(q)
    scale, dy = _f32(scale), _f32(dy)
    dx = np.zeros(M * K, dtype=np.float32)
    if lib().orc_gemm_dx_q(_p(q), _p(scale), _p(dy), _p(dx), M, N, K, group, bits):
        raise ValueError("bad shape")
    return dx


# ---- DiT block pieces: kernels.metal:443-506, 807-993; DiT.swift:520-550 ----

def rmsnorm_fwd(x, weight, rows, cols, eps):
    x, weight = _f32(x), _f32(weight)
    y = np.zeros(rows * cols, dtype=np.float32)
    rstd = np.zeros(rows, dtype=np.float32)
    lib().orc_rmsnorm_fwd(_p(x), _p(y), _p(rstd), _p(weight), rows, cols, eps)
    return y, rstd


def rope_tables(maxT, dim, theta):
    c = np.zeros(maxT * dim, dtype=np.float32)
    s = np.zeros(maxT * dim, dtype=np.float32)
    lib().orc_rope_tables(maxT, dim, theta, _p(c), _p(s))
    return c, s


def rope_fwd(x, cosv, sinv, B, T, H, D):
    x, cosv, sinv = _f32(x), _f32(cosv), _f32(sinv)
    y = np.zeros_like(x)
    lib().orc_rope_fwd(_p(x), _p(y), _p(cosv), _p(sinv), B, T, H, D)
    return y


def repeat_heads(src, B, T, H, D):
    src = _f32(src)
    dst = np.zeros(B * T * H * D, dtype=np.float32)
    lib().orc_repeat_heads(_p(src), _p(dst), B, T, H, D)
    return dst


def attn_fwd(q, k, v, B, T, H, D, causal=0):
    q, k, v = _f32(q), _f32(k), _f32(v)
    scores = np.zeros(B * H * T * T, dtype=np.float32)
    probs = np.zeros_like(scores)
    av = np.zeros(B * T * H * D, dtype=np.float32)
    lib().orc_attn_fwd(_p(q), _p(k), _p(v), _p(scores), _p(probs), _p(av), B, T, H, D, causal)
    return scores, probs, av


def swiglu_fwd(gate, up):
    gate, up = _f32(gate), _f32(up)
    y = np.zeros_like(gate)
    lib().orc_swiglu_fwd(_p(gate), _p(up), _p(y), gate.size)
    return y


def mix(a, b, ca, cb):
    a, b = _f32(a), _f32(b)
    y = np.zeros_like(a)
    lib().orc_mix(_p(a), _p(b), _p(y), a.size, ca, cb)
    return y


@dataclass
class DiTCfg:
    """DiTConfig fields used by the loop body (src/DiT.swift:9-41)."""
    B: int = 8
    T: int = 64
    C: int = 192
    F: int = 768
    H: int = 4
    D: int = 48
    loops: int = 4
    group: int = 32
    bits: int = 8
    eps: float = 1e-6
    theta: float = 10000.0
    mix: float = 0.5


class _CCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("B", "T", "C", "F", "H", "D", "loops", "group", "bits")] + \
               [("eps", ctypes.c_float), ("theta", ctypes.c_float), ("mix", ctypes.c_float)]


DIT_LINEARS = ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")
DIT_NORMS = ("n1", "n1b", "n2", "n2b", "nf")


def dit_forward(cfg: DiTCfg, qw: dict, x0: np.ndarray) -> np.ndarray:
    """The looped block forward (src/DiT.swift:520-550) with quantized
    linears in the Metal kernel order. qw maps each of DIT_LINEARS to
    (codes, scales) and each of DIT_NORMS to its fp32 weight."""
    c = _CCfg(cfg.B, cfg.T, cfg.C, cfg.F, cfg.H, cfg.D, cfg.loops, cfg.group, cfg.bits,
              cfg.eps, cfg.theta, cfg.mix)
    nws = lib().orc_dit_workspace_floats(ctypes.byref(c))
    ws = np.zeros(nws, dtype=np.float32)
    x = np.array(x0, dtype=np.float32, copy=True).reshape(-1)
    args = []
    keep = []
    for name in DIT_LINEARS:
        q, s = qw[name]
        q = np.ascontiguousarray(q)
        s = _f32(s)
        keep += [q, s]
        args += [_p(q), _p(s)]
    for name in DIT_NORMS:
        w = _f32(qw[name])
        keep.append(w)
        args.append(_p(w))
    rc = lib().orc_dit_forward(ctypes.byref(c), *args, _p(x), _p(ws))
    if rc != 0:
        raise ValueError("bad DiT config")
    return x


# ---- training step: kernels.metal:285-295, 616-697, 749-802 -----------------

def adamw(w, g, m, v, lr, b1, b2, eps, wd, invBC1, invBC2):
    """adamw (kernels.metal:786-802). Returns the updated (w, m, v) copies."""
    w, m, v = (np.array(a, dtype=np.float32, copy=True).reshape(-1) for a in (w, m, v))
    g = _f32(g).reshape(-1)
    lib().orc_adamw(_p(w), _p(g), _p(m), _p(v), w.size, lr, b1, b2, eps, wd, invBC1, invBC2)
    return w, m, v


def adam_quantize(w, g, m, v, rows, cols, group, bits, lr, b1, b2, eps, wd, invBC1, invBC2, init=None):
    """adamw then cpuQuant of the updated master (GPT.swift:214-217, 441-447).
    Returns (w, m, v, codes, scales)."""
    w, m, v = adamw(w, g, m, v, lr, b1, b2, eps, wd, invBC1, invBC2)
    q, s = quant(w, rows, cols, group, bits, init=init)
    return w, m, v, q, s


def reduce_sumsq(x) -> float:
    """reduce_sumsq (kernels.metal:749-768) in its 256-lane order."""
    x = _f32(x).reshape(-1)
    return float(lib().orc_reduce_sumsq(_p(x), x.size))


def scale(x, s):
    x = np.array(x, dtype=np.float32, copy=True).reshape(-1)
    lib().orc_scale(_p(x), x.size, s)
    return x


def embed(tokens, wte, q, scale_, wpe, B, T, C, group, bits):
    """embed_f32 / embed_i8 / embed_i4 (kernels.metal:616-663)."""
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    wte = None if wte is None else _f32(wte)
    q = None if q is None else np.ascontiguousarray(q)
    scale_ = None if scale_ is None else _f32(scale_)
    wpe = _f32(wpe)
    y = np.zeros(B * T * C, dtype=np.float32)
    if lib().orc_embed(_p(tokens), _p(wte), _p(q), _p(scale_), _p(wpe), _p(y), B, T, C, group, bits):
        raise ValueError("bad embed shape")
    return y


def embed_bwd(tokens, dx, dwe, B, T, C, V):
    """embed_bwd (kernels.metal:665-682): returns dwe + per-token sums."""
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    dx = _f32(dx)
    out = np.array(dwe, dtype=np.float32, copy=True).reshape(-1)
    lib().orc_embed_bwd(_p(tokens), _p(dx), _p(out), B, T, C, V)
    return out


def pos_bwd(dx, B, T, C):
    dx = _f32(dx)
    out = np.zeros(T * C, dtype=np.float32)
    lib().orc_pos_bwd(_p(dx), _p(out), B, T, C)
    return out


def bias_grad(dy, M, N):
    dy = _f32(dy)
    out = np.zeros(N, dtype=np.float32)
    lib().orc_bias_grad(_p(dy), _p(out), M, N)
    return out


# ---- DiT block backward: kernels.metal:508-612, 827-868, 891-1010; DiT.swift:558-626

def rms_bwd(x, rstd, weight, dy, dweight, rows, cols):
    """rmsnorm_bwd_dx / rmsnorm_bwd_dw. Returns (dx, dweight + sum)."""
    x, rstd, weight, dy = _f32(x), _f32(rstd), _f32(weight), _f32(dy)
    dx = np.zeros(rows * cols, np.float32)
    dw = np.array(dweight, dtype=np.float32, copy=True).reshape(-1)
    lib().orc_rms_bwd(_p(x), _p(rstd), _p(weight), _p(dy), _p(dx), _p(dw), rows, cols)
    return dx, dw


def attn_bwd(q, k, v, probs, dout, B, T, H, D):
    """GPU.attnBwd (GPU.swift:312-322). Returns dq, dk, dv, dprobs, dscores."""
    q, k, v, probs, dout = (_f32(a) for a in (q, k, v, probs, dout))
    n, tt = B * T * H * D, B * H * T * T
    dq, dk, dv = (np.zeros(n, np.float32) for _ in range(3))
    dp, ds = np.zeros(tt, np.float32), np.zeros(tt, np.float32)
    lib().orc_attn_bwd(_p(q), _p(k), _p(v), _p(probs), _p(dout), _p(dq), _p(dk), _p(dv), _p(dp), _p(ds),
                       B, T, H, D)
    return dq, dk, dv, dp, ds


def rope_bwd(dy, cosv, sinv, B, T, H, D):
    dy, cosv, sinv = _f32(dy), _f32(cosv), _f32(sinv)
    dx = np.zeros_like(dy)
    lib().orc_rope_bwd(_p(dy), _p(dx), _p(cosv), _p(sinv), B, T, H, D)
    return dx


def swiglu_bwd(gate, up, dy):
    gate, up, dy = _f32(gate), _f32(up), _f32(dy)
    dg, du = np.zeros_like(gate), np.zeros_like(gate)
    lib().orc_swiglu_bwd(_p(gate), _p(up), _p(dy), _p(dg), _p(du), gate.size)
    return dg, du


def sum_heads(src, B, T, H, D):
    src = _f32(src)
    dst = np.zeros(B * T * D, np.float32)
    lib().orc_sum_heads(_p(src), _p(dst), B, T, H, D)
    return dst


def acc_scale(a, b, s):
    a = np.array(a, dtype=np.float32, copy=True).reshape(-1)
    lib().orc_acc_scale(_p(a), _p(_f32(b)), a.size, s)
    return a


def dit_train(cfg: DiTCfg, lin: dict, norms: dict, x0, gy):
    """One training step of the looped block (forward with saved activations,
    then DiT.swift:566-626). lin maps each of DIT_LINEARS to an fp32 weight
    (bits 32) or (codes, scales) (bits 8/4). Returns (xs[loops], dL/dxs[0],
    weight grads {name: [N*K]}, norm grads {name: [C]})."""
    c = _CCfg(cfg.B, cfg.T, cfg.C, cfg.F, cfg.H, cfg.D, cfg.loops, cfg.group, cfg.bits,
              cfg.eps, cfg.theta, cfg.mix)
    shapes = {"wq": (cfg.C, cfg.C), "wk": (cfg.D, cfg.C), "wv": (cfg.D, cfg.C), "wo": (cfg.C, cfg.C),
              "wgate": (cfg.F, cfg.C), "wup": (cfg.F, cfg.C), "wdown": (cfg.C, cfg.F)}
    keep = []
    W = (ctypes.c_void_p * 7)()
    Q = (ctypes.c_void_p * 7)()
    S = (ctypes.c_void_p * 7)()
    GW = (ctypes.c_void_p * 7)()
    gw = {}
    for i, name in enumerate(DIT_LINEARS):
        if cfg.bits == 32:
            w = _f32(lin[name]).reshape(-1)
            keep.append(w)
            W[i] = w.ctypes.data
        else:
            q, s = lin[name]
            q, s = np.ascontiguousarray(q), _f32(s)
            keep += [q, s]
            Q[i], S[i] = q.ctypes.data, s.ctypes.data
        gw[name] = np.zeros(shapes[name][0] * shapes[name][1], np.float32)
        GW[i] = gw[name].ctypes.data
    NR = (ctypes.c_void_p * 5)()
    GN = (ctypes.c_void_p * 5)()
    gn = {}
    for i, name in enumerate(DIT_NORMS):
        nw = _f32(norms[name])
        keep.append(nw)
        NR[i] = nw.ctypes.data
        gn[name] = np.zeros(cfg.C, np.float32)
        GN[i] = gn[name].ctypes.data
    x = np.array(x0, dtype=np.float32, copy=True).reshape(-1)
    g = np.array(gy, dtype=np.float32, copy=True).reshape(-1)
    ws = np.zeros(lib().orc_dit_train_floats(ctypes.byref(c)), np.float32)
    rc = lib().orc_dit_train(ctypes.byref(c), ctypes.cast(W, _P), ctypes.cast(Q, _P), ctypes.cast(S, _P),
                             ctypes.cast(NR, _P), _p(x), _p(g), ctypes.cast(GW, _P), ctypes.cast(GN, _P), _p(ws))
    if rc != 0:
        raise ValueError("bad DiT config")
    return x, g, gw, gn
