"""Benchmark of the group-quantized linear path on one MI355X.

Headline ("c2"): one step = the int4 group-quant
linear forward plus its STE backward on the DiT down-projection shape,
X[512,768] ~ N(0,1), W[192,768] ~ N(0,0.02) int4 G=32, dY ~ N(0,1e-3):
    Y = X deq(W)^T   (gemm_nt_i4)
    dX = dY deq(W)   (gemm_dx_i4)
    dW = dY^T X      (gemm_dw)
Inputs are resident in HBM before timing; the weights are quantized once
before the timed region. value = algorithmic flop of the step / step time.

The same JSON line carries `roofline` (dominant kernel of the step, timed with
HIP events on the stream it runs on), `cpu_baseline` (the reference's scalar
CPU path restated in C, single thread, on a bounded sample), and `workloads`:
the other configs measured the same way (c1 int8 forward, c4 decode-shaped
int4 with weight copies rotated past the 256 MB Infinity Cache, c5 prefill,
quantization at the c4/c5 weight shape).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-extra] [--skip-cpu]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(REPO, "diffusion-gpt-metal_amd")

METRIC = "group-quant GEMM GB/s & TFLOP/s (% of MI355X roofline); DiT block fwd tokens/s"
PEAK = {"hbm_GBps": 8000.0, "fp32_TFLOPs": 157.3, "bf16_TFLOPs": 2500.0}


def load_package():
    if "dgm_amd" in sys.modules:
        return sys.modules["dgm_amd"]
    spec = importlib.util.spec_from_file_location(
        "dgm_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["dgm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Bench:
    def __init__(self, dgm, torch):
        self.dgm, self.torch = dgm, torch
        self.gpu = dgm.GPU()
        # Launch on torch's current stream so torch.cuda.Event brackets the
        # very stream the kernels run on.
        self.stream = torch.cuda.current_stream()
        self.gpu.set_stream(self.stream)
        self.gen = torch.Generator(device="cpu").manual_seed(1234)

    def randn(self, n: int, std: float):
        t = self.torch.randn(n, generator=self.gen, dtype=self.torch.float32) * std
        return t.to("cuda")

    def zeros(self, n: int, dtype=None):
        return self.torch.zeros(max(n, 1), dtype=dtype or self.torch.float32, device="cuda")

    def quantized(self, w, N: int, K: int, G: int, bits: int):
        t = self.torch
        q = self.zeros(N * K // (2 if bits == 4 else 1), t.uint8 if bits == 4 else t.int8)
        s = self.zeros(N * (K // G))
        self.gpu.begin()
        self.gpu.quantize(w, q, s, N, K, bits, G)
        self.gpu.end()
        return q, s

    def time_launches(self, fn, reps: int, warmup: int = 3) -> float:
        """Average ms per call of fn (which enqueues work) between HIP events
        recorded on the launch stream."""
        t = self.torch
        self.gpu.begin()
        for i in range(warmup):
            fn(i)
        self.gpu.end()
        e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        self.gpu.begin()
        e0.record(self.stream)
        for i in range(reps):
            fn(i)
        e1.record(self.stream)
        self.gpu.end()
        e1.synchronize()
        return e0.elapsed_time(e1) / reps


def roofline(achieved: float, peak: float, unit: str, bound: str, traffic=None) -> dict:
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 5), "traffic": traffic}


def load_traffic() -> dict:
    """Per-kernel HBM bytes per launch measured with rocprofv3 --pmc
    (FETCH_SIZE + WRITE_SIZE, scaled by a copy-kernel calibration) and
    committed under profiles/; absent entries report null."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f)
    return {}


# ---- headline: c2 step -------------------------------------------------------

C2 = dict(M=512, N=192, K=768, G=32, bits=4)


def c2_setup(b: Bench):
    M, N, K, G = C2["M"], C2["N"], C2["K"], C2["G"]
    x, w, dy = b.randn(M * K, 1.0), b.randn(N * K, 0.02), b.randn(M * N, 1e-3)
    q, s = b.quantized(w, N, K, G, 4)
    y, dx, dw = b.zeros(M * N), b.zeros(M * K), b.zeros(N * K)
    g = b.gpu
    kern = {
        "gemm_nt_i4": lambda i: g.gemmNT(4, None, q, s, x, None, y, M, N, K, G),
        "gemm_dx_i4": lambda i: g.gemmDX(4, None, q, s, dy, dx, M, N, K, G),
        "gemm_dw": lambda i: g.gemmDW(dy, x, dw, M, N, K),
    }
    return kern


def c2_flops() -> int:
    return 3 * 2 * C2["M"] * C2["N"] * C2["K"]


def c2_bytes() -> dict:
    M, N, K, G = C2["M"], C2["N"], C2["K"], C2["G"]
    q, s = N * K // 2, N * (K // G) * 4
    return {"gemm_nt_i4": q + s + 4 * (M * K + M * N), "gemm_dx_i4": q + s + 4 * (M * N + M * K),
            "gemm_dw": 4 * (M * K + M * N + N * K)}


def cpu_baseline_c2(budget_s: float = 12.0) -> dict:
    """The reference's scalar CPU path (Check.swift:399-494 restated in C,
    kernel orders of metal/kernels.metal:180-283), single thread, timed on
    whole c2 steps until ~budget_s of CPU work."""
    import numpy as np
    if REPO not in sys.path:
        sys.path.insert(0, REPO)
    from oracle import oracle as orc
    M, N, K, G = C2["M"], C2["N"], C2["K"], C2["G"]
    rng = np.random.default_rng(0)
    x = rng.standard_normal(M * K, dtype=np.float32)
    w = (rng.standard_normal(N * K, dtype=np.float32) * np.float32(0.02))
    dy = (rng.standard_normal(M * N, dtype=np.float32) * np.float32(1e-3))
    q, s = orc.quant(w, N, K, G, 4)
    steps, t0 = 0, time.perf_counter()
    while True:
        orc.gemm_nt_q(q, s, x, None, M, N, K, G, 4)
        orc.gemm_dx_q(q, s, dy, M, N, K, G, 4)
        orc.gemm_dw(dy, x, M, N, K)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= 50:
            break
    per_step = el / steps
    return {"value": round(c2_flops() / per_step / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"{steps} full c2 steps (gemm_nt_i4 kernel order + gemm_dx_i4 + gemm_dw), "
                      f"{per_step * 1e3:.1f} ms/step, oracle/oracle.c -O2 -ffp-contract=off, 1 thread",
            "host_cpu": _cpu_model(), "host_nproc": os.cpu_count()}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---- other configs -------------------------------------------------------------


def bench_c1(b: Bench, reps: int) -> dict:
    M, N, K, G = 512, 768, 192, 32
    x, w = b.randn(M * K, 1.0), b.randn(N * K, 0.02)
    q, s = b.quantized(w, N, K, G, 8)
    y = b.zeros(M * N)
    ms = b.time_launches(lambda i: b.gpu.gemmNT(8, None, q, s, x, None, y, M, N, K, G), reps)
    flops = 2 * M * N * K
    nbytes = N * K + N * (K // G) * 4 + 4 * (M * K + M * N)
    return {"kernel": "gemm_nt_i8", "shape": "M=512 K=192 N=768 int8 G=32", "us": round(ms * 1e3, 3),
            "TFLOPs": round(flops / ms / 1e9, 3), "GBps": round(nbytes / ms / 1e6, 2),
            "roofline": roofline(flops / ms / 1e9, PEAK["fp32_TFLOPs"], "TFLOP/s", "mfma"),
            "note": "latency-bound; fp32 MFMA is the nearer roof"}


def bench_quant(b: Bench, reps: int, bits: int) -> dict:
    N, K, G = 14336, 4096, 128
    w = b.randn(N * K, 0.02)
    q = b.zeros(N * K // (2 if bits == 4 else 1), b.torch.uint8)
    s = b.zeros(N * (K // G))
    ms = b.time_launches(lambda i: b.gpu.quantize(w, q, s, N, K, bits, G), reps)
    nbytes = 4 * N * K + (N * K // (2 if bits == 4 else 1)) + 4 * N * (K // G)
    return {"kernel": f"quant_i{bits}", "shape": "W[14336,4096] G=128", "us": round(ms * 1e3, 3),
            "GBps": round(nbytes / ms / 1e6, 2),
            "roofline": roofline(nbytes / ms / 1e6, PEAK["hbm_GBps"], "GB/s", "hbm")}


def bench_c4(b: Bench, reps: int, M: int, math_mode: int) -> dict:
    """Decode-shaped int4: K=4096, N=14336, G=128. Weight copies are rotated so
    that successive launches never find W in the 256 MB Infinity Cache."""
    N, K, G = 14336, 4096, 128
    wq_bytes = N * K // 2 + N * (K // G) * 4
    copies = max(2, -(-512 * 2 ** 20 // wq_bytes))
    w = b.randn(N * K, 0.02)
    qs = [b.quantized(w, N, K, G, 4) for _ in range(1)]
    q0, s0 = qs[0]
    Q = [q0] + [q0.clone() for _ in range(copies - 1)]
    S = [s0] + [s0.clone() for _ in range(copies - 1)]
    x = b.randn(M * K, 1.0)
    y = b.zeros(M * N)
    b.gpu.set_math(math_mode)
    try:
        ms = b.time_launches(lambda i: b.gpu.gemmNT(4, None, Q[i % copies], S[i % copies], x, None, y,
                                                    M, N, K, G), reps)
    finally:
        b.gpu.set_math(b.dgm.DGM_MATH_FP32)
    flops = 2 * M * N * K
    nbytes = wq_bytes + 4 * (M * K + M * N)
    mode = "fp32" if math_mode == b.dgm.DGM_MATH_FP32 else "bf16"
    del Q, S
    return {"kernel": "gemm_nt_i4", "math": mode, "shape": f"M={M} K=4096 N=14336 int4 G=128",
            "us": round(ms * 1e3, 3), "GBps": round(nbytes / ms / 1e6, 2),
            "TFLOPs": round(flops / ms / 1e9, 3), "weight_copies_rotated": copies,
            "roofline": roofline(nbytes / ms / 1e6, PEAK["hbm_GBps"], "GB/s", "hbm")}


def bench_c5(b: Bench, reps: int, bits: int, math_mode: int) -> dict:
    M, N, K, G = 8192, 14336, 4096, 128
    w = b.randn(N * K, 0.02)
    q, s = b.quantized(w, N, K, G, bits)
    del w
    x = b.randn(M * K, 1.0)
    y = b.zeros(M * N)
    b.gpu.set_math(math_mode)
    try:
        ms = b.time_launches(lambda i: b.gpu.gemmNT(bits, None, q, s, x, None, y, M, N, K, G), reps, warmup=1)
    finally:
        b.gpu.set_math(b.dgm.DGM_MATH_FP32)
    flops = 2 * M * N * K
    mode = "fp32" if math_mode == b.dgm.DGM_MATH_FP32 else "bf16"
    peak = PEAK["fp32_TFLOPs"] if mode == "fp32" else PEAK["bf16_TFLOPs"]
    return {"kernel": f"gemm_nt_i{bits}", "math": mode, "shape": f"M=8192 K=4096 N=14336 int{bits} G=128",
            "us": round(ms * 1e3, 3), "TFLOPs": round(flops / ms / 1e9, 3),
            "roofline": roofline(flops / ms / 1e9, peak, "TFLOP/s", "mfma")}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--reps", type=int, default=100, help="launches per per-kernel timing")
    ap.add_argument("--skip-extra", action="store_true", help="headline only")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list of extra workloads to run")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the reference is single-device); run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    dgm = load_package()
    b = Bench(dgm, torch)

    # -- headline step --------------------------------------------------------
    log("[bench] c2 step setup")
    kern = c2_setup(b)
    order = ["gemm_nt_i4", "gemm_dx_i4", "gemm_dw"]

    def step(i):
        for k in order:
            kern[k](i)

    b.gpu.begin()
    for i in range(args.warmup):
        step(i)
    b.gpu.end()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    b.gpu.begin()
    for i in range(args.steps):
        step(i)
    b.gpu.end()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    log(f"[bench] c2 step {ms_step * 1e3:.2f} us")

    per_kernel = {k: b.time_launches(kern[k], args.reps) for k in order}
    dom = max(per_kernel, key=per_kernel.get)
    flops_k = 2 * C2["M"] * C2["N"] * C2["K"]
    traffic = load_traffic().get(f"c2:{dom}")
    roof = roofline(flops_k / per_kernel[dom] / 1e9, PEAK["fp32_TFLOPs"], "TFLOP/s", "mfma", traffic)
    roof["kernel"] = dom
    roof["avg_launch_us"] = round(per_kernel[dom] * 1e3, 3)
    roof["algorithmic_bytes"] = c2_bytes()[dom]
    roof["algorithmic_flop"] = flops_k
    roof["note"] = ("latency-bound shape; fp32 MFMA (157.3 TFLOP/s) is the nearer roof than HBM "
                    f"({c2_bytes()[dom] / 8e12 * 1e6:.2f} us at 8 TB/s)")

    out = {
        "metric": METRIC,
        "value": round(c2_flops() / (ms_step * 1e-3) / 1e12, 4),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (torch CPU generator, seed 1234: X~N(0,1), W~N(0,0.02), dY~N(0,1e-3))",
        "config": {"workload": "c2: int4 group-quant linear fwd + STE bwd (gemm_nt_i4, gemm_dx_i4, gemm_dw)",
                   "M": C2["M"], "K": C2["K"], "N": C2["N"], "group": C2["G"], "bits": 4,
                   "parallelism": "single GPU"},
        "GBps": round(sum(c2_bytes().values()) / (ms_step * 1e-3) / 1e9, 2),
        "per_kernel_us": {k: round(v * 1e3, 3) for k, v in per_kernel.items()},
        "roofline": roof,
    }

    if not args.skip_extra:
        only = set(filter(None, args.only.split(",")))
        W = {}
        jobs = [
            ("c1_int8_fwd", lambda: bench_c1(b, args.reps)),
            ("quant_i4_14336x4096", lambda: bench_quant(b, 20, 4)),
            ("quant_i8_14336x4096", lambda: bench_quant(b, 20, 8)),
            ("c4_int4_m1_fp32", lambda: bench_c4(b, 50, 1, dgm.DGM_MATH_FP32)),
            ("c4_int4_m16_fp32", lambda: bench_c4(b, 50, 16, dgm.DGM_MATH_FP32)),
            ("c4_int4_m16_bf16", lambda: bench_c4(b, 50, 16, dgm.DGM_MATH_BF16)),
            ("c4_int4_m64_bf16", lambda: bench_c4(b, 50, 64, dgm.DGM_MATH_BF16)),
            ("c5_int4_bf16", lambda: bench_c5(b, 5, 4, dgm.DGM_MATH_BF16)),
            ("c5_int8_bf16", lambda: bench_c5(b, 5, 8, dgm.DGM_MATH_BF16)),
        ]
        for name, fn in jobs:
            if only and name not in only:
                continue
            log(f"[bench] {name}")
            try:
                W[name] = fn()
            except Exception as e:   # report, keep the headline line intact
                W[name] = {"error": str(e)}
            torch.cuda.empty_cache()
        out["workloads"] = W

    if not args.skip_cpu:
        log("[bench] cpu baseline (oracle, 1 thread)")
        out["cpu_baseline"] = cpu_baseline_c2()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
