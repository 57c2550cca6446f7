"""The reference's checkpoint files on the host side, over the C ABI parsers.

TGMT (the quantized GPT, src/GPT.swift:265-324): header, the vocabulary's
bytes, then every parameter's fp32 master in GPT.init's creation order.
load_gpt() mirrors GPT.load: it reads the masters into device Param records
and re-quantizes the quantized ones (quantizeAll, src/GPT.swift:318-322).
TDIT (the DiT, src/DiT.swift:396-451): header, then the DiT's 17 parameters;
load_dit_block() builds a DiTBlock from the block's linears and norms,
quantized once with the requested bits and group.
save_tgmt() / save_tdit() write the same layouts (GPT.save, DiT.save).
"""
from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass
from typing import List, Optional

import numpy as np

from .abi import DgmError, ParamInfo, TditHeader, TgmtHeader, load_library

_TGMT_FIELDS = ("version", "bits", "vocab", "block", "layers", "heads", "embd", "qGroup")
_TDIT_FIELDS = ("side", "patch", "names", "loops", "heads", "kvHeads", "embd", "intermediate", "freqDim",
                "diffusionSteps")


@dataclass
class CkptParam:
    """One parameter of a checkpoint: the reference's name, shape and flags,
    and its fp32 master (a view of the file image)."""
    name: str
    rows: int
    cols: int
    quantized: bool
    decay: bool
    data: np.ndarray


def _read(path) -> bytes:
    with open(path, "rb") as f:
        return f.read()


def _params(lib, fn, hdr, n: int, image: bytes) -> List[CkptParam]:
    out = []
    for i in range(n):
        info = ParamInfo()
        rc = fn(ctypes.byref(hdr), i, ctypes.byref(info))
        if rc != 0:
            raise DgmError(rc, f"parameter {i} of the checkpoint")
        count = info.rows * info.cols
        data = np.frombuffer(image, dtype="<f4", count=count, offset=info.offset)
        out.append(CkptParam(info.name.decode(), info.rows, info.cols, bool(info.quantized), bool(info.decay), data))
    return out


def read_tgmt(path):
    """Returns (header dict, itos bytes, [CkptParam]). Raises DgmError for a
    file the reference would reject (magic, version, configuration, length)."""
    lib = load_library()
    image = _read(path)
    hdr = TgmtHeader()
    itos_off, nparams = ctypes.c_int64(), ctypes.c_int64()
    buf = ctypes.create_string_buffer(image, len(image))
    rc = lib.dgm_tgmt_parse(buf, len(image), ctypes.byref(hdr), ctypes.byref(itos_off), ctypes.byref(nparams))
    if rc != 0:
        raise DgmError(rc, f"{path}: not a valid TGMT checkpoint (magic, version, configuration or length)")
    h = {n: getattr(hdr, n) for n in _TGMT_FIELDS}
    itos = image[itos_off.value: itos_off.value + hdr.vocab]
    return h, itos, _params(lib, lib.dgm_tgmt_param, hdr, nparams.value, image)


def read_tdit(path):
    """Returns (header dict, [CkptParam]) for a TDIT file."""
    lib = load_library()
    image = _read(path)
    hdr = TditHeader()
    nparams = ctypes.c_int64()
    buf = ctypes.create_string_buffer(image, len(image))
    rc = lib.dgm_tdit_parse(buf, len(image), ctypes.byref(hdr), ctypes.byref(nparams))
    if rc != 0:
        raise DgmError(rc, f"{path}: not a valid TDIT checkpoint (magic, version, configuration or length)")
    h = {n: getattr(hdr, n) for n in ("version",) + _TDIT_FIELDS}
    h["lastAlpha"], h["valueMix"] = hdr.lastAlpha, hdr.valueMix
    return h, _params(lib, lib.dgm_tdit_param, hdr, nparams.value, image)


def save_tgmt(path, header: dict, itos: bytes, masters: List[np.ndarray]) -> None:
    """GPT.save (src/GPT.swift:265-281): masters in creation order."""
    with open(path, "wb") as f:
        f.write(b"TGMT")
        f.write(struct.pack("<8I", *[int(header.get(n, 1 if n == "version" else 0)) for n in _TGMT_FIELDS]))
        f.write(bytes(itos))
        for m in masters:
            f.write(np.ascontiguousarray(m, dtype="<f4").tobytes())


def save_tdit(path, header: dict, masters: List[np.ndarray], version: int = 2) -> None:
    """DiT.save (src/DiT.swift:396-411); version 1 omits lastAlpha."""
    with open(path, "wb") as f:
        f.write(b"TDIT")
        f.write(struct.pack("<I", version))
        f.write(struct.pack("<10I", *[int(header[n]) for n in _TDIT_FIELDS]))
        if version >= 2:
            f.write(struct.pack("<f", header.get("lastAlpha", 0.01)))
        f.write(struct.pack("<f", header["valueMix"]))
        for m in masters:
            f.write(np.ascontiguousarray(m, dtype="<f4").tobytes())


def load_gpt(path, gpu, device: str = "cuda"):
    """GPT.load (src/GPT.swift:283-324): (header, itos, [Param]) with every
    master on the device and the quantized parameters' codes and scales
    rebuilt by the GPU quantizer."""
    import torch
    from .train import Param
    h, itos, params = read_tgmt(path)
    out = []
    gpu.begin()
    for p in params:
        P = Param(p.name, p.rows, p.cols, p.quantized, p.decay, h["bits"], h["qGroup"], device)
        P.w.copy_(torch.from_numpy(p.data.copy()).to(device))
        if p.quantized and h["bits"] != 32:
            gpu.quantize(P.w, P.q, P.scale, P.rows, P.cols, h["bits"], h["qGroup"])
        out.append(P)
    gpu.end()
    return h, itos, out


def load_dit_block(path, gpu, bits: int = 8, group: int = 32, batch: int = 8, device: str = "cuda"):
    """The looped block of a TDIT checkpoint as a DiTBlock: its linears
    (wq ... wdown) quantized once with `bits` / `group` (or fp32 for bits 32)
    and its five RMSNorm weights. Returns (header, DiTConfig, DiTBlock)."""
    import torch
    from .dit import DiTBlock, DiTConfig
    h, params = read_tdit(path)
    grid = h["side"] // h["patch"]
    cfg = DiTConfig(B=batch, T=grid * grid, C=h["embd"], F=h["intermediate"], H=h["heads"],
                    D=h["embd"] // h["heads"], loops=h["loops"], group=group, bits=bits, mix=h["valueMix"])
    by_name = {p.name: p for p in params}
    weights = {n: torch.from_numpy(by_name[n].data.copy()).to(device)
               for n in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown", "n1", "n1b", "n2", "n2b", "nf")}
    return h, cfg, DiTBlock(gpu, cfg, weights)


__all__ = ["CkptParam", "read_tgmt", "read_tdit", "save_tgmt", "save_tdit", "load_gpt", "load_dit_block"]
