"""Python mirror of the reference's GPU class (src/GPU.swift:91-272) over the C ABI.

Same method names and argument meaning as the Swift wrappers (quantize,
gemmNT, gemmDX, gemmDW, gemmDWAcc, the DiT block's wrappers, the training
step's adam / reduceSumsq / scale / zero / embed / embedBwd / posBwd /
biasGrad, begin, end, lastKernel) plus the kernel-level entries (quant_i8 ...
gemm_dw_acc, adamw, embed_i4 ...) in the buffer slot order of
metal/kernels.metal. Buffers are device tensors (torch is used only to hold
device memory) or raw device addresses. A nonzero status raises DgmError,
where the reference calls fatalError / exit(1).
"""
from __future__ import annotations

import ctypes
from typing import Any, Optional

from .abi import (DGM_MATH_BF16, DGM_MATH_FP32, AdamP, BiasP, DgmError, DiTCfg,
                  DiTGrads, DiTWeights, EmbBwdP, EmbP, GemmP, PosP, QuantP, ReduceP, ScaleP,
                  UnaryP, load_library)


def _ptr(t: Any) -> Optional[int]:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if hasattr(t, "data_ptr"):
        if hasattr(t, "is_cuda") and not t.is_cuda:
            raise ValueError("buffers must live in device memory")
        return t.data_ptr()
    raise TypeError(f"cannot take a device address of {type(t).__name__}")


def Buf(count: int, device: str = "cuda"):
    """src/GPU.swift:31-55: zero-filled fp32 buffer of max(count, 1) floats."""
    import torch
    return torch.zeros(max(count, 1), dtype=torch.float32, device=device)


def RawBuf(nbytes: int, device: str = "cuda"):
    """src/GPU.swift:57-68: zero-filled byte buffer of max(bytes, 16)."""
    import torch
    return torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=device)


class GPU:
    """One context = one HIP stream, in-order dispatch (src/GPU.swift:91-198)."""

    def __init__(self, stream: Any = None, lib: Optional[ctypes.CDLL] = None):
        self.lib = lib or load_library()
        h = ctypes.c_void_p()
        rc = self.lib.dgm_gpu_create(ctypes.byref(h))
        if rc != 0:
            raise DgmError(rc, "dgm_gpu_create failed (no HIP device?)")
        self.h = h
        if stream is not None:
            self.set_stream(stream)

    # -- lifecycle -----------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "h", None):
            self.lib.dgm_gpu_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream: Any) -> None:
        """Accepts a torch.cuda.Stream, a raw hipStream_t address or None."""
        raw = getattr(stream, "cuda_stream", stream)
        self._check(self.lib.dgm_gpu_set_stream(self.h, raw))

    @property
    def stream(self) -> int:
        return self.lib.dgm_gpu_stream(self.h) or 0

    def set_math(self, mode: int) -> None:
        self._check(self.lib.dgm_set_math(self.h, mode))

    @property
    def math(self) -> int:
        return self.lib.dgm_get_math(self.h)

    @property
    def lastKernel(self) -> str:
        return self.lib.dgm_last_kernel(self.h).decode()

    @property
    def lastError(self) -> str:
        return self.lib.dgm_last_error(self.h).decode()

    def _check(self, rc: int) -> None:
        if rc != 0:
            raise DgmError(rc, self.lastError, self.lastKernel)

    # -- dispatch region (src/GPU.swift:158-180) ------------------------------
    def begin(self) -> None:
        self._check(self.lib.dgm_begin(self.h))

    def end(self) -> None:
        self._check(self.lib.dgm_end(self.h))

    # -- host call surface (src/GPU.swift:220-272) ----------------------------
    def quantize(self, w, q, scale, rows: int, cols: int, bits: int, qGroup: int) -> None:
        self._check(self.lib.dgm_quantize(self.h, _ptr(w), _ptr(q), _ptr(scale), rows, cols, bits, qGroup))

    def gemmNT(self, bits: int, w, q, scale, x, bias, y, M: int, N: int, K: int, qGroup: int) -> None:
        self._check(self.lib.dgm_gemmNT(self.h, bits, _ptr(w), _ptr(q), _ptr(scale), _ptr(x),
                                        _ptr(bias), _ptr(y), M, N, K, qGroup))

    def gemmNT_noalloc(self, bits: int, w, q, scale, x, bias, y, M: int, N: int, K: int, qGroup: int) -> None:
        """gemmNT with staging in the library's static device scratch (no
        allocation; DGM_ERR_UNSUPPORTED when the call needs more scratch)."""
        self._check(self.lib.dgm_gemmNT_noalloc(self.h, bits, _ptr(w), _ptr(q), _ptr(scale), _ptr(x),
                                                 _ptr(bias), _ptr(y), M, N, K, qGroup))

    def gemmNT_workspace_bound(self, M: int, N: int, K: int) -> int:
        """Bytes of workspace that cover any gemmNT call of this shape (no
        counterpart in the reference, whose buffers are all made at setup)."""
        return int(self.lib.dgm_gemmNT_workspace_bound(M, N, K))

    def reserve(self, nbytes: int) -> None:
        """Grow the context's workspace to at least nbytes now, so that later
        calls within it allocate nothing."""
        self._check(self.lib.dgm_gpu_reserve(self.h, nbytes))

    def workspaceBytes(self) -> int:
        return int(self.lib.dgm_gpu_workspace_bytes(self.h))

    def probeRead(self, src, nbytes: int, mode: int, workgroups: int, sink) -> None:
        """The bench's read-rate probe (no counterpart in the reference): mode 0
        16-byte register loads, mode 1 direct-to-LDS loads, `workgroups` 0 = one
        per CU; `sink` gets one u32 per workgroup."""
        self._check(self.lib.dgm_probe_read(self.h, _ptr(src), nbytes, mode, workgroups, _ptr(sink)))

    def probeGemvValu(self, q, scale, x, y, M: int, N: int, K: int, qGroup: int) -> None:
        """The bench's comparison GEMV (no counterpart in the reference): int4
        codes, fp32 VALU FMAs with a wave reduction, M = 1 or 16, no bias."""
        self._check(self.lib.dgm_probe_gemv_valu(self.h, _ptr(q), _ptr(scale), _ptr(x), _ptr(y), M, N, K, qGroup))

    def gemmDX(self, bits: int, w, q, scale, dy, dx, M: int, N: int, K: int, qGroup: int) -> None:
        self._check(self.lib.dgm_gemmDX(self.h, bits, _ptr(w), _ptr(q), _ptr(scale), _ptr(dy),
                                        _ptr(dx), M, N, K, qGroup))

    def gemmDW(self, dy, x, dw, M: int, N: int, K: int) -> None:
        self._check(self.lib.dgm_gemmDW(self.h, _ptr(dy), _ptr(x), _ptr(dw), M, N, K))

    def gemmDWAcc(self, dy, x, dw, M: int, N: int, K: int) -> None:
        self._check(self.lib.dgm_gemmDWAcc(self.h, _ptr(dy), _ptr(x), _ptr(dw), M, N, K))

    def gemmBwd(self, bits: int, w, q, scale, dy, x, dx, dw, M: int, N: int, K: int, qGroup: int,
                accumulate: bool = False) -> None:
        """gemmDW (or gemmDWAcc) then gemmDX on the same dY, in one launch
        where the shapes allow (bitwise the two calls)."""
        self._check(self.lib.dgm_gemmBwd(self.h, bits, _ptr(w), _ptr(q), _ptr(scale), _ptr(dy), _ptr(x), _ptr(dx),
                                         _ptr(dw), M, N, K, qGroup, 1 if accumulate else 0))

    # -- DiT block wrappers (src/GPU.swift:211-410) ---------------------------
    def rmsFwd(self, x, y, rstd, weight, rows: int, cols: int, eps: float) -> None:
        self._check(self.lib.dgm_rmsFwd(self.h, _ptr(x), _ptr(y), _ptr(rstd), _ptr(weight), rows, cols, eps))

    def ropeFwd(self, x, y, cos, sin, B: int, T: int, H: int, D: int) -> None:
        self._check(self.lib.dgm_ropeFwd(self.h, _ptr(x), _ptr(y), _ptr(cos), _ptr(sin), B, T, H, D))

    def repeatHeads(self, src, dst, B: int, T: int, H: int, D: int) -> None:
        self._check(self.lib.dgm_repeatHeads(self.h, _ptr(src), _ptr(dst), B, T, H, D))

    def attnFwd(self, q, k, v, scores, probs, av, B: int, T: int, H: int, D: int, causal: bool = True) -> None:
        """GPU.attnFwd; causal defaults to true as in src/GPU.swift:302-303."""
        self._check(self.lib.dgm_attnFwd(self.h, _ptr(q), _ptr(k), _ptr(v), _ptr(scores), _ptr(probs),
                                         _ptr(av), B, T, H, D, 1 if causal else 0))

    def swigluFwd(self, gate, up, y, n: int) -> None:
        self._check(self.lib.dgm_swigluFwd(self.h, _ptr(gate), _ptr(up), _ptr(y), n))

    def add(self, a, b, y, n: int) -> None:
        self._check(self.lib.dgm_add(self.h, _ptr(a), _ptr(b), _ptr(y), n))

    def mix(self, a, b, y, n: int, ca: float, cb: float) -> None:
        self._check(self.lib.dgm_mix(self.h, _ptr(a), _ptr(b), _ptr(y), n, ca, cb))

    def copy(self, x, y, n: int) -> None:
        self._check(self.lib.dgm_copy(self.h, _ptr(x), _ptr(y), n))

    def rmsBwd(self, x, rstd, weight, dy, dx, dweight, rows: int, cols: int, eps: float) -> None:
        self._check(self.lib.dgm_rmsBwd(self.h, _ptr(x), _ptr(rstd), _ptr(weight), _ptr(dy), _ptr(dx), _ptr(dweight),
                                        rows, cols, eps))

    def attnBwd(self, q, k, v, probs, dout, dq, dk, dv, dprobs, dscores, B: int, T: int, H: int, D: int) -> None:
        self._check(self.lib.dgm_attnBwd(self.h, _ptr(q), _ptr(k), _ptr(v), _ptr(probs), _ptr(dout), _ptr(dq),
                                         _ptr(dk), _ptr(dv), _ptr(dprobs), _ptr(dscores), B, T, H, D))

    def ropeBwd(self, dy, dx, cos, sin, B: int, T: int, H: int, D: int) -> None:
        self._check(self.lib.dgm_ropeBwd(self.h, _ptr(dy), _ptr(dx), _ptr(cos), _ptr(sin), B, T, H, D))

    def swigluBwd(self, gate, up, dy, dgate, dup, n: int) -> None:
        self._check(self.lib.dgm_swigluBwd(self.h, _ptr(gate), _ptr(up), _ptr(dy), _ptr(dgate), _ptr(dup), n))

    def sumHeads(self, src, dst, B: int, T: int, H: int, D: int) -> None:
        self._check(self.lib.dgm_sumHeads(self.h, _ptr(src), _ptr(dst), B, T, H, D))

    def acc(self, a, b, n: int) -> None:
        self._check(self.lib.dgm_acc(self.h, _ptr(a), _ptr(b), n))

    def accScale(self, a, b, n: int, by: float) -> None:
        self._check(self.lib.dgm_accScale(self.h, _ptr(a), _ptr(b), n, by))

    def dit_acts_floats(self, cfg: DiTCfg) -> int:
        return int(self.lib.dgm_dit_acts_floats(ctypes.byref(cfg)))

    def dit_backward_ws_floats(self, cfg: DiTCfg) -> int:
        return int(self.lib.dgm_dit_backward_ws_floats(ctypes.byref(cfg)))

    def dit_forward_train(self, cfg: DiTCfg, w: DiTWeights, cos, sin, x, acts, acts_floats: int) -> None:
        self._check(self.lib.dgm_dit_forward_train(self.h, ctypes.byref(cfg), ctypes.byref(w), _ptr(cos), _ptr(sin),
                                                   _ptr(x), _ptr(acts), acts_floats))

    def dit_backward(self, cfg: DiTCfg, w: DiTWeights, grads: DiTGrads, cos, sin, acts, acts_floats: int, gx, ws,
                     ws_floats: int) -> None:
        self._check(self.lib.dgm_dit_backward(self.h, ctypes.byref(cfg), ctypes.byref(w), ctypes.byref(grads),
                                              _ptr(cos), _ptr(sin), _ptr(acts), acts_floats, _ptr(gx), _ptr(ws),
                                              ws_floats))

    def dit_workspace_floats(self, cfg: DiTCfg) -> int:
        return int(self.lib.dgm_dit_workspace_floats(ctypes.byref(cfg)))

    def dit_forward(self, cfg: DiTCfg, w: DiTWeights, cos, sin, x, ws, ws_floats: int) -> None:
        self._check(self.lib.dgm_dit_forward(self.h, ctypes.byref(cfg), ctypes.byref(w), _ptr(cos), _ptr(sin),
                                             _ptr(x), _ptr(ws), ws_floats))

    # -- training step (src/GPU.swift:200-210, 274-277, 324-350, 420-429) -----
    def adam(self, w, g, m, v, n: int, lr: float, b1: float, b2: float, eps: float, wd: float,
             invBC1: float, invBC2: float) -> None:
        self._check(self.lib.dgm_adam(self.h, _ptr(w), _ptr(g), _ptr(m), _ptr(v), n, lr, b1, b2, eps, wd,
                                      invBC1, invBC2))

    def adamQuantize(self, w, g, m, v, q, scale, rows: int, cols: int, bits: int, qGroup: int, lr: float,
                     b1: float, b2: float, eps: float, wd: float, invBC1: float, invBC2: float) -> None:
        """adam followed by quantize of the same master, in one pass where the
        shape allows (dgm_adam_quantize); bit-identical to the two calls."""
        self._check(self.lib.dgm_adam_quantize(self.h, _ptr(w), _ptr(g), _ptr(m), _ptr(v), _ptr(q), _ptr(scale),
                                               rows, cols, bits, qGroup, lr, b1, b2, eps, wd, invBC1, invBC2))

    def reduceSumsq(self, x, into, n: int, slot: int) -> None:
        self._check(self.lib.dgm_reduceSumsq(self.h, _ptr(x), _ptr(into), n, slot))

    def zero(self, b, n: int) -> None:
        self._check(self.lib.dgm_zero(self.h, _ptr(b), n))

    def scale(self, b, n: int, by: float) -> None:
        self._check(self.lib.dgm_scale(self.h, _ptr(b), n, by))

    def embed(self, bits: int, tokens, wte, q, scale, wpe, y, B: int, T: int, C: int, qGroup: int) -> None:
        self._check(self.lib.dgm_embed(self.h, bits, _ptr(tokens), _ptr(wte), _ptr(q), _ptr(scale), _ptr(wpe),
                                       _ptr(y), B, T, C, qGroup))

    def embedBwd(self, tokens, dx, dwe, B: int, T: int, C: int, V: int) -> None:
        self._check(self.lib.dgm_embedBwd(self.h, _ptr(tokens), _ptr(dx), _ptr(dwe), B, T, C, V))

    def posBwd(self, dx, dwp, B: int, T: int, C: int) -> None:
        self._check(self.lib.dgm_posBwd(self.h, _ptr(dx), _ptr(dwp), B, T, C))

    def biasGrad(self, dy, db, M: int, N: int) -> None:
        self._check(self.lib.dgm_biasGrad(self.h, _ptr(dy), _ptr(db), M, N))

    # -- kernel-level entries (metal/kernels.metal slot order) ----------------
    def quant_i8(self, W, Q, scale, p: QuantP) -> None:
        self._check(self.lib.dgm_quant_i8(self.h, _ptr(W), _ptr(Q), _ptr(scale), ctypes.byref(p)))

    def quant_i4(self, W, Q, scale, p: QuantP) -> None:
        self._check(self.lib.dgm_quant_i4(self.h, _ptr(W), _ptr(Q), _ptr(scale), ctypes.byref(p)))

    def gemm_nt_f32(self, W, X, bias, Y, p: GemmP) -> None:
        self._check(self.lib.dgm_gemm_nt_f32(self.h, _ptr(W), _ptr(X), _ptr(bias), _ptr(Y), ctypes.byref(p)))

    def gemm_nt_i8(self, W, scale, X, bias, Y, p: GemmP) -> None:
        self._check(self.lib.dgm_gemm_nt_i8(self.h, _ptr(W), _ptr(scale), _ptr(X), _ptr(bias), _ptr(Y),
                                            ctypes.byref(p)))

    def gemm_nt_i4(self, W, scale, X, bias, Y, p: GemmP) -> None:
        self._check(self.lib.dgm_gemm_nt_i4(self.h, _ptr(W), _ptr(scale), _ptr(X), _ptr(bias), _ptr(Y),
                                            ctypes.byref(p)))

    def gemm_dx_f32(self, W, dY, dX, p: GemmP) -> None:
        self._check(self.lib.dgm_gemm_dx_f32(self.h, _ptr(W), _ptr(dY), _ptr(dX), ctypes.byref(p)))

    def gemm_dx_i8(self, W, scale, dY, dX, p: GemmP) -> None:
        self._check(self.lib.dgm_gemm_dx_i8(self.h, _ptr(W), _ptr(scale), _ptr(dY), _ptr(dX), ctypes.byref(p)))

    def gemm_dx_i4(self, W, scale, dY, dX, p: GemmP) -> None:
        self._check(self.lib.dgm_gemm_dx_i4(self.h, _ptr(W), _ptr(scale), _ptr(dY), _ptr(dX), ctypes.byref(p)))

    def gemm_dw(self, dY, X, dW, p: GemmP) -> None:
        self._check(self.lib.dgm_gemm_dw(self.h, _ptr(dY), _ptr(X), _ptr(dW), ctypes.byref(p)))

    def gemm_dw_acc(self, dY, X, dW, p: GemmP) -> None:
        self._check(self.lib.dgm_gemm_dw_acc(self.h, _ptr(dY), _ptr(X), _ptr(dW), ctypes.byref(p)))

    def adamw(self, w, g, m, v, p: AdamP) -> None:
        self._check(self.lib.dgm_adamw(self.h, _ptr(w), _ptr(g), _ptr(m), _ptr(v), ctypes.byref(p)))

    def reduce_sumsq(self, x, out, p: ReduceP) -> None:
        self._check(self.lib.dgm_reduce_sumsq(self.h, _ptr(x), _ptr(out), ctypes.byref(p)))

    def zero_f(self, x, p: UnaryP) -> None:
        self._check(self.lib.dgm_zero_f(self.h, _ptr(x), ctypes.byref(p)))

    def scale_f(self, x, p: ScaleP) -> None:
        self._check(self.lib.dgm_scale_f(self.h, _ptr(x), ctypes.byref(p)))

    def embed_f32(self, tokens, wte, wpe, y, p: EmbP) -> None:
        self._check(self.lib.dgm_embed_f32(self.h, _ptr(tokens), _ptr(wte), _ptr(wpe), _ptr(y), ctypes.byref(p)))

    def embed_i8(self, tokens, wte, scale, wpe, y, p: EmbP) -> None:
        self._check(self.lib.dgm_embed_i8(self.h, _ptr(tokens), _ptr(wte), _ptr(scale), _ptr(wpe), _ptr(y),
                                          ctypes.byref(p)))

    def embed_i4(self, tokens, wte, scale, wpe, y, p: EmbP) -> None:
        self._check(self.lib.dgm_embed_i4(self.h, _ptr(tokens), _ptr(wte), _ptr(scale), _ptr(wpe), _ptr(y),
                                          ctypes.byref(p)))

    def embed_bwd(self, tokens, dx, dwe, p: EmbBwdP) -> None:
        self._check(self.lib.dgm_embed_bwd(self.h, _ptr(tokens), _ptr(dx), _ptr(dwe), ctypes.byref(p)))

    def pos_bwd(self, dx, dwp, p: PosP) -> None:
        self._check(self.lib.dgm_pos_bwd(self.h, _ptr(dx), _ptr(dwp), ctypes.byref(p)))

    def bias_grad(self, dY, db, p: BiasP) -> None:
        self._check(self.lib.dgm_bias_grad(self.h, _ptr(dY), _ptr(db), ctypes.byref(p)))


__all__ = ["GPU", "Buf", "RawBuf", "DGM_MATH_FP32", "DGM_MATH_BF16"]
