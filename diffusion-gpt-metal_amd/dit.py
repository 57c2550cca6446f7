"""Host side of the looped DiT block forward (src/DiT.swift:505-550) over the C ABI.

DiTBlock holds the block's linears quantized once on the device
(GPU.quantize, src/GPU.swift:220-225), device copies of the RoPE tables
(ropeTables, src/Macro.swift:509-530, computed on the host as the reference
does) and the forward's workspace. forward() enqueues the whole loop body
(dgm_dit_forward) on the context's stream: nothing is allocated and nothing
waits on the host, so the call can be captured into a HIP graph.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict

import numpy as np

from .abi import DIT_LINEARS, DIT_NORMS, DgmError, DiTCfg, DiTGrads, DiTLinear, DiTWeights, load_library
from .gpu import GPU, _ptr


@dataclass
class DiTConfig:
    """The DiTConfig fields the block forward reads (src/DiT.swift:9-41).
    Defaults are the photos-dit block: 8 x 64 tokens, embd 192, 4 heads of 48
    with one KV head, SwiGLU 768, eps 1e-6, theta 1e4, mix 0.5, 4 loops."""
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
    theta: float = 1e4
    mix: float = 0.5

    def linear_shapes(self) -> Dict[str, tuple]:
        """[N, K] of each linear (src/DiT.swift:242-248); KV width = D."""
        C, F, KV = self.C, self.F, self.D
        return {"wq": (C, C), "wk": (KV, C), "wv": (KV, C), "wo": (C, C),
                "wgate": (F, C), "wup": (F, C), "wdown": (C, F)}

    def c_cfg(self) -> DiTCfg:
        return DiTCfg(self.B, self.T, self.C, self.F, self.H, self.D, self.loops, self.group, self.bits,
                      self.eps, self.mix, 0)


def rope_tables(maxT: int, dim: int, theta: float):
    """ropeTables (src/Macro.swift:509-530) on the host: (cos, sin), each a
    float32 array of maxT * dim."""
    lib = load_library()
    cos = np.zeros(max(maxT * dim, 1), dtype=np.float32)
    sin = np.zeros(max(maxT * dim, 1), dtype=np.float32)
    rc = lib.dgm_ropeTables(maxT, dim, theta, cos.ctypes.data, sin.ctypes.data)
    if rc != 0:
        raise DgmError(rc, f"ropeTables: bad sizes maxT={maxT} dim={dim}")
    return cos[: maxT * dim], sin[: maxT * dim]


class DiTBlock:
    """The shared block of a looped DiT with quantized linears.

    weights: fp32 device tensors keyed by DIT_LINEARS ([N, K] row-major) and
    DIT_NORMS ([C]). With bits 8 / 4 each linear is quantized once on the
    device; with bits 32 the fp32 weights are used as they are.
    """

    def __init__(self, gpu: GPU, cfg: DiTConfig, weights: Dict[str, object]):
        import torch
        self.gpu, self.cfg = gpu, cfg
        if cfg.bits not in (4, 8, 32):
            raise DgmError(5, f"unsupported bits {cfg.bits}")
        self.keep = []
        self.codes: Dict[str, object] = {}
        self.scales: Dict[str, object] = {}
        shapes = cfg.linear_shapes()
        for name in DIT_LINEARS:
            N, K = shapes[name]
            w = weights[name]
            if w.numel() != N * K or w.dtype != torch.float32 or not w.is_cuda:
                raise ValueError(f"{name}: expected {N}x{K} fp32 device tensor")
        # [wq; wk; wv] and [wgate; wup] are laid out back to back so that the
        # library runs each group as one GEMM (quantization is per row, so the
        # codes and scales of a row do not depend on its neighbours).
        groups = [("wq", "wk", "wv"), ("wo",), ("wgate", "wup"), ("wdown",)]
        lin = {}
        dev = weights["wq"].device
        gpu.begin()
        for grp in groups:
            rows = sum(shapes[n][0] for n in grp)
            K = shapes[grp[0]][1]
            if cfg.bits == 32:
                cat = torch.cat([weights[n].reshape(-1).contiguous() for n in grp])
                self.keep.append(cat)
                off = 0
                for n in grp:
                    lin[n] = DiTLinear(cat.data_ptr() + 4 * off, None, None)
                    off += shapes[n][0] * K
                continue
            per = (lambda r: r * K // 2) if cfg.bits == 4 else (lambda r: r * K)
            q = torch.zeros(max(per(rows), 16), dtype=torch.uint8, device=dev)
            s = torch.zeros(max(rows * (K // cfg.group), 1), dtype=torch.float32, device=dev)
            self.keep += [q, s]
            r0 = 0
            for n in grp:
                N = shapes[n][0]
                qv = q[per(r0): per(r0 + N)]
                sv = s[r0 * (K // cfg.group): (r0 + N) * (K // cfg.group)]
                gpu.quantize(weights[n].contiguous(), qv, sv, N, K, cfg.bits, cfg.group)
                self.codes[n], self.scales[n] = qv, sv
                lin[n] = DiTLinear(None, qv.data_ptr(), sv.data_ptr())
                r0 += N
        gpu.end()
        norms = {}
        for name in DIT_NORMS:
            w = weights[name].contiguous()
            if w.numel() != cfg.C or w.dtype != torch.float32 or not w.is_cuda:
                raise ValueError(f"{name}: expected {cfg.C} fp32 device tensor")
            self.keep.append(w)
            norms[name] = _ptr(w)
        self.c = cfg.c_cfg()
        self.w = DiTWeights(*[lin[n] for n in DIT_LINEARS], *[norms[n] for n in DIT_NORMS])
        cos, sin = rope_tables(cfg.T, cfg.D, cfg.theta)
        self.cos = torch.from_numpy(cos).to(dev)
        self.sin = torch.from_numpy(sin).to(dev)
        self.ws_floats = gpu.dit_workspace_floats(self.c)
        if self.ws_floats < 0:
            raise DgmError(1, "dit workspace size")
        self.ws = torch.zeros(self.ws_floats, dtype=torch.float32, device=dev)

    def forward(self, x) -> None:
        """xs[0] -> xs[loops] in place; x is a [B*T*C] fp32 device tensor.
        Must be called inside begin()/end() of the block's GPU."""
        cfg = self.cfg
        if x.numel() != cfg.B * cfg.T * cfg.C or not x.is_contiguous():
            raise ValueError("x must be a contiguous [B*T, C] tensor")
        self.gpu.dit_forward(self.c, self.w, self.cos, self.sin, x, self.ws, self.ws_floats)

    # -- training (src/DiT.swift:520-626) -------------------------------------
    def zero_grads(self) -> None:
        """Allocates (first call) or clears the fp32 parameter gradients."""
        import torch
        if not hasattr(self, "grads"):
            shapes = self.cfg.linear_shapes()
            dev = self.cos.device
            # One buffer, the linears in order: [wq; wk; wv] and [wgate; wup]
            # gradients sit back to back like their weights, so the backward
            # runs each group as one weight-gradient GEMM.
            sizes = [shapes[n][0] * shapes[n][1] for n in DIT_LINEARS]
            self._grad_buf = torch.zeros(sum(sizes), dtype=torch.float32, device=dev)
            self.grads = dict(zip(DIT_LINEARS, torch.split(self._grad_buf, sizes)))
            self.grads.update({n: torch.zeros(self.cfg.C, dtype=torch.float32, device=dev) for n in DIT_NORMS})
            self.c_grads = DiTGrads(*[self.grads[n].data_ptr() for n in DIT_LINEARS],
                                    *[self.grads[n].data_ptr() for n in DIT_NORMS])
            self.acts_floats = self.gpu.dit_acts_floats(self.c)
            self.bws_floats = self.gpu.dit_backward_ws_floats(self.c)
            self.acts = torch.zeros(max(self.acts_floats, 1), dtype=torch.float32, device=dev)
            self.bws = torch.zeros(max(self.bws_floats, 1), dtype=torch.float32, device=dev)
        else:
            self._grad_buf.zero_()
            for n in DIT_NORMS:
                self.grads[n].zero_()

    def forward_train(self, x) -> None:
        """xs[0] -> xs[loops] in place, keeping every loop's activations for
        backward(). Inside begin()/end(); call zero_grads() once first."""
        cfg = self.cfg
        if x.numel() != cfg.B * cfg.T * cfg.C or not x.is_contiguous():
            raise ValueError("x must be a contiguous [B*T, C] tensor")
        if not hasattr(self, "acts"):
            self.zero_grads()
        self.gpu.dit_forward_train(self.c, self.w, self.cos, self.sin, x, self.acts, self.acts_floats)

    def backward(self, gx) -> None:
        """gx: dL/dxs[loops] -> dL/dxs[0] in place; adds the parameter
        gradients into self.grads (fp32, keyed like the weights)."""
        self.gpu.dit_backward(self.c, self.w, self.c_grads, self.cos, self.sin, self.acts, self.acts_floats, gx,
                              self.bws, self.bws_floats)

    def workspace_view(self, name: str):
        """The last loop's intermediate `name` (scores, probs, ...) as a view of
        the workspace, in the order dgm_dit_forward lays them out."""
        sizes = _ws_sizes(self.cfg)
        off = 0
        for n, sz in sizes:
            if n == name:
                return self.ws[off:off + sz]
            off += (sz + 63) & ~63
        raise KeyError(name)


def _ws_sizes(cfg: DiTConfig):
    """The pieces of dgm_dit_forward's workspace, in order (each 256-byte aligned)."""
    M, C, F, KV = cfg.B * cfg.T, cfg.C, cfg.F, cfg.D
    att = cfg.B * cfg.H * cfg.T * cfg.T
    names = ["ln1", "qkv0", "qkv1", "scores", "probs", "av", "attn", "mid", "ln2", "gu", "sw", "mlp", "pre", "rstd"]
    sizes = [M * C, M * (C + 2 * KV), M * (C + 2 * KV), att, att, M * C, M * C, M * C, M * C, M * 2 * F, M * F,
             M * C, M * C, M]
    return list(zip(names, sizes))


__all__ = ["DiTConfig", "DiTBlock", "rope_tables", "DIT_LINEARS", "DIT_NORMS"]
