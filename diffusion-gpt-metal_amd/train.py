"""Host side of the optimizer half of a training step over the C ABI.

Param mirrors the reference's parameter record (src/GPT.swift:5-36): an fp32
master w with its gradient g and Adam moments m, v, and for quantized
parameters the int8 / int4 codes q and per-group scales the forward GEMMs
read. optimizer_step() is GPT.step's update (src/GPT.swift:193-218): the
squared-gradient sums for the global-norm clip, the clip scale, AdamW on
every master and the re-quantization of the quantized ones, the last two
fused into one pass per quantized parameter (GPU.adamQuantize), which leaves
every buffer bit-identical to the reference's adam-then-quantizeAll order.
"""
from __future__ import annotations

import math
from typing import Iterable, List, Optional

from .gpu import GPU, Buf, RawBuf


class Param:
    """src/GPT.swift:5-36. All buffers are zero-filled device tensors."""

    def __init__(self, name: str, rows: int, cols: int, quantized: bool, decay: bool, bits: int,
                 qGroup: int, device: str = "cuda"):
        self.name, self.rows, self.cols = name, rows, cols
        self.quantized, self.decay = quantized, decay
        self.bits, self.qGroup = bits, qGroup
        n = rows * cols
        self.w, self.g, self.m, self.v = (Buf(n, device) for _ in range(4))
        self.q = self.scale = None
        if quantized:
            self.scale = Buf(rows * (cols // qGroup), device)
            self.q = RawBuf(n // 2 if bits == 4 else n, device)

    @property
    def count(self) -> int:
        return self.rows * self.cols


def bias_corrections(b1: float, b2: float, step_index: int):
    """invBC1, invBC2 of src/GPT.swift:205-206 (Float arithmetic)."""
    import numpy as np
    f = np.float32
    inv1 = f(1) / (f(1) - f(b1) ** f(step_index))
    inv2 = f(1) / (f(1) - f(b2) ** f(step_index))
    return float(inv1), float(inv2)


def zero_grads(gpu: GPU, params: Iterable[Param]) -> None:
    """src/GPT.swift:437-439 (inside an open begin()/end() region)."""
    for p in params:
        gpu.zero(p.g, p.count)


def grad_norm(gpu: GPU, params: List[Param], sumsq=None) -> float:
    """src/GPT.swift:196-204: one reduceSumsq per parameter into its slot,
    then the host sums the slots in order and takes the square root."""
    import numpy as np
    if sumsq is None:
        sumsq = Buf(len(params))
    gpu.begin()
    for i, p in enumerate(params):
        gpu.reduceSumsq(p.g, sumsq, p.count, i)
    gpu.end()
    vals = sumsq[: len(params)].cpu().numpy().astype(np.float32)
    ss = np.float32(0)
    for x in vals:
        ss = np.float32(ss + x)
    return float(np.sqrt(ss))


def optimizer_step(gpu: GPU, params: List[Param], lr: float, wd: float, clip: float, step_index: int,
                   b1: float = 0.9, b2: float = 0.95, eps: float = 1e-8, sumsq=None,
                   fused: bool = True) -> float:
    """The update of GPT.step (src/GPT.swift:193-218) after the backward has
    filled every p.g. Returns the pre-clip gradient norm. With fused=False the
    reference's dispatch order is kept literally (adam for all, then quantize
    for all quantized parameters); the results are the same bits."""
    import numpy as np
    norm = grad_norm(gpu, params, sumsq)
    inv1, inv2 = bias_corrections(b1, b2, step_index)
    gpu.begin()
    if clip > 0 and norm > clip:
        s = float(np.float32(clip) / (np.float32(norm) + np.float32(1e-6)))
        for p in params:
            gpu.scale(p.g, p.count, s)
    for p in params:
        decay = wd if p.decay else 0.0
        if fused and p.quantized and p.bits != 32:
            gpu.adamQuantize(p.w, p.g, p.m, p.v, p.q, p.scale, p.rows, p.cols, p.bits, p.qGroup, lr, b1, b2,
                             eps, decay, inv1, inv2)
        else:
            gpu.adam(p.w, p.g, p.m, p.v, p.count, lr, b1, b2, eps, decay, inv1, inv2)
    if not fused:
        for p in params:
            if p.quantized and p.bits != 32:
                gpu.quantize(p.w, p.q, p.scale, p.rows, p.cols, p.bits, p.qGroup)
    gpu.end()
    return norm


__all__ = ["Param", "bias_corrections", "zero_grads", "grad_norm", "optimizer_step"]
