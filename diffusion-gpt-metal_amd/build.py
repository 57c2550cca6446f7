"""Builds libdgm_amd.so in-tree for gfx950 with hipcc.

Every .hip file under csrc/ is compiled to an object in _build/ and linked
into diffusion-gpt-metal_amd/libdgm_amd.so. Flags that matter for parity:
  -fhip-fp32-correctly-rounded-divide-sqrt  IEEE fp32 divide (the quantizer's
                                            w / s must round like the CPU's)
  -fno-gpu-flush-denormals-to-zero           keep fp32 denormals
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                            no packed fp32 VALU ops (their
                                            results are not trusted on these
                                            boxes); the host pass warns that it
                                            does not know the feature
No fast-math flag is used anywhere.

Usage: python diffusion-gpt-metal_amd/build.py [-j N]
"""
from __future__ import annotations

import argparse
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libdgm_amd.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libdgm_amd.so)")


# Sources whose kernels issue loads as inline asm and wait for them by hand
# (gemm_decode.hip, gemm_stream.hip, and the prefill producers of
# gemm_bf16.hip): a register spilled while such a load is in flight would be
# read before the load fills it, so these kernels must not use scratch. The
# build checks the compiler's resource-usage remarks.
NO_SCRATCH = {"gemm_decode.hip", "gemm_stream.hip", "gemm_bf16.hip", "gemm_slab.hip"}
REMARK = "-Rpass-analysis=kernel-resource-usage"


def _scratch_users(stderr: str) -> list:
    users, fn = [], None
    for line in stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            fn = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and fn and int(m.group(1)) > 0:
            users.append(f"{fn} ({m.group(1)} bytes/lane)")
    return users


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    check = os.path.basename(src) in NO_SCRATCH
    cmd = [hipcc(), *HIPCC_FLAGS, *([REMARK] if check else []), "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    lines = [l for l in proc.stderr.splitlines() if noise not in l]
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(lines))
    if check:
        bad = _scratch_users(proc.stderr)
        if bad:
            os.remove(obj)
            raise RuntimeError(f"{src}: kernels with hand-waited loads use scratch: {', '.join(bad)}")
        lines = [l for l in lines if REMARK not in l]
    err = "\n".join(lines)
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = jobs or min(8, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    print(build(ap.parse_args().j))
