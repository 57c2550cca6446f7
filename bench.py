"""Benchmark of the group-quantized linear path on one MI355X.

Headline: BASELINE.json's largest configuration, c5 — the prefill-shaped int4
group-quant GEMM forward, M=8192, K=4096, N=14336, G=128, on bf16 MFMA with
the weights dequantized to bf16 in LDS and fp32 accumulation:
    X[8192,4096] ~ N(0,1) fp32,  W[14336,4096] ~ N(0,0.02) -> int4 codes + fp32
    scales (quantized once, before the timed region),  Y = X deq(W)^T fp32.
One step = one gemmNT call (the reference's GPU.gemmNT, src/GPU.swift:227-243)
with inputs resident in HBM. value = 2*M*N*K / (wall time of the K timed
steps / K), in TFLOP/s.

The same JSON line carries:
  * `roofline`: the dominant kernel (the only kernel of the headline call),
    algorithmic flop per launch / its average launch duration from HIP events
    recorded on the launch stream around every timed step, against the dense
    bf16 MFMA peak; `traffic` = HBM bytes per launch from rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE runs (profiles/traffic.json), each scaled by the
    counter's reading for a plain copy of known size;
  * `cpu_baseline`: the reference's scalar CPU path (src/Check.swift:433-494:
    dequant, then cpuGemmNT), restated in C (oracle/oracle.c, -O2
    -ffp-contract=off), one thread pinned to one core, on a contiguous slice
    of N (cost is linear in N; the rate is extrapolated and the slice named);
  * `hbm_ceiling`: a measured stream copy (512 MiB each way) on this GPU;
  * `workloads`: every other configuration (c1, c2 step, c3 forward and
    training step, c4 M = 1/16/64 in both math modes, c5 int8, quantization,
    AdamW + re-quantization, embed_bwd), each with its own roofline, traffic
    and one-core CPU baseline.

GPU timings of the short workloads replay a captured HIP graph of many
launches (through torch.cuda.CUDAGraph) so host overhead never leaks into
kernel times; HIP events on the launch stream bracket the replay.

Usage:
  python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-extra] [--skip-cpu]
                  [--only name,name] [--calib-copy]
  python bench.py --list                              workload names
  python bench.py --summarize DIR [--title TEXT]      rocprofv3 csv -> markdown
  python bench.py --traffic NAME FETCH_DIR WRITE_DIR  PMC runs -> profiles/traffic.json
"""
from __future__ import annotations

import argparse
import contextlib
import csv
import importlib.util
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(REPO, "diffusion-gpt-metal_amd")
TRAFFIC_JSON = os.path.join(REPO, "profiles", "traffic.json")

METRIC = "group-quant GEMM GB/s & TFLOP/s (% of MI355X roofline); DiT block fwd tokens/s"
# MI355X published peaks (dense).
PEAK = {"hbm_GBps": 8000.0, "fp32_TFLOPs": 157.3, "bf16_TFLOPs": 2500.0, "int8_TOPs": 5000.0}
CALIB_BYTES = 256 * 2 ** 20   # plain copy kernel used to scale FETCH_SIZE / WRITE_SIZE
CEIL_BYTES = 512 * 2 ** 20    # stream-copy ceiling leg

C5 = dict(M=8192, N=14336, K=4096, G=128)
C4 = dict(N=14336, K=4096, G=128)
C2 = dict(M=512, N=192, K=768, G=32)
C1 = dict(M=512, N=768, K=192, G=32)


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
        # A dedicated stream: graph capture needs a non-default stream, and the
        # library launches on it, so events recorded on it bracket the kernels.
        self.stream = torch.cuda.Stream()
        self.gpu = dgm.GPU(stream=self.stream)
        self.gen = torch.Generator(device="cpu").manual_seed(1234)
        self.read_ceiling_c4 = None   # GB/s, set by hbm_read_ceiling

    def randn(self, n: int, std: float):
        t = self.torch.randn(n, generator=self.gen, dtype=self.torch.float32) * std
        return t.to("cuda")

    def zeros(self, n: int, dtype=None):
        return self.torch.zeros(max(n, 1), dtype=dtype or self.torch.float32, device="cuda")

    def sync(self):
        self.torch.cuda.synchronize()

    def quantized(self, w, N: int, K: int, G: int, bits: int):
        t = self.torch
        q = self.zeros(N * K // (2 if bits == 4 else 1), t.uint8 if bits == 4 else t.int8)
        s = self.zeros(N * (K // G))
        self.sync()
        self.gpu.begin()
        self.gpu.quantize(w, q, s, N, K, bits, G)
        self.gpu.end()
        return q, s

    @contextlib.contextmanager
    def math(self, mode: int):
        self.gpu.set_math(mode)
        try:
            yield
        finally:
            self.gpu.set_math(self.dgm.DGM_MATH_FP32)

    def capture(self, fn, calls: int):
        """A CUDA graph of `calls` invocations fn(0..calls-1). fn runs eagerly
        first, so workspaces exist before capture (no allocation in a graph)."""
        t = self.torch
        self.sync()
        with t.cuda.stream(self.stream):
            self.gpu.begin()
            for i in range(min(calls, 3)):
                fn(i)
            self.gpu.end()
        g = t.cuda.CUDAGraph()
        with t.cuda.graph(g, stream=self.stream):
            self.gpu.begin()
            for i in range(calls):
                fn(i)
        # dgm end() synchronizes, which a capture forbids; status is checked
        # at launch and by the synchronizing replay below.
        self.gpu.begin()
        return g

    def graph_ms(self, g, replays: int = 1) -> float:
        t = self.torch
        with t.cuda.stream(self.stream):
            g.replay()
        self.stream.synchronize()
        e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        e0.record(self.stream)
        with t.cuda.stream(self.stream):
            for _ in range(replays):
                g.replay()
        e1.record(self.stream)
        e1.synchronize()
        return e0.elapsed_time(e1)

    def time_launches(self, fn, reps: int) -> float:
        """Average ms per call of fn, from a graph replay of reps calls."""
        g = self.capture(fn, reps)
        ms = self.graph_ms(g) / reps
        del g
        return ms

    def time_steps(self, fn, steps: int, warmup: int) -> dict:
        """Eager calls: `warmup` untimed, then exactly `steps` timed between two
        device synchronizations, with a HIP event on the launch stream before
        and after every step. Returns the wall time per step and the event
        duration of every step."""
        t = self.torch
        self.sync()
        self.gpu.begin()
        for i in range(warmup):
            fn(i)
        self.gpu.end()
        ev = [t.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        self.sync()
        t0 = time.perf_counter()
        self.gpu.begin()
        ev[0].record(self.stream)
        for i in range(steps):
            fn(i)
            ev[i + 1].record(self.stream)
        self.gpu.end()
        self.sync()
        wall = time.perf_counter() - t0
        per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
        return {"wall_ms_per_step": wall * 1e3 / steps, "event_ms": per}


def roofline(achieved: float, peak: float, unit: str, bound: str, traffic=None) -> dict:
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 5), "traffic": traffic}


def load_traffic() -> dict:
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE runs, scaled by a copy-kernel calibration (bench.py --traffic);
    absent entries report null."""
    if os.path.exists(TRAFFIC_JSON):
        with open(TRAFFIC_JSON) as f:
            return json.load(f)
    return {}


def traffic_for(workload: str, kernel_keys, per_call: str = "") -> object:
    """Counted HBM bytes per call: the sum over the call's kernels (names
    matched by substring), or None when the workload was not profiled. With
    per_call naming a kernel that runs exactly once per call, each kernel's
    bytes per launch are weighted by its launches per call (its dispatches
    over that kernel's); without it every matched kernel counts once."""
    ent = load_traffic().get(workload, {})
    kern = {n: r for n, r in ent.items() if n != "_calibration" and any(key in n for key in kernel_keys)}
    if not kern:
        return None
    calls = None
    if per_call:
        once = [r for n, r in kern.items() if per_call in n]
        if len(once) != 1 or not once[0].get("dispatches"):
            return None
        calls = once[0]["dispatches"]
    total = 0.0
    for rec in kern.values():
        weight = rec.get("dispatches", 0) / calls if calls else 1.0
        total += rec.get("total_bytes", 0) * weight
    return round(total)


# ---- the reference's scalar CPU path, one core ---------------------------------


def _oracle():
    if REPO not in sys.path:
        sys.path.insert(0, REPO)
    from oracle import oracle as orc
    return orc


@contextlib.contextmanager
def one_core():
    """Pins the calling thread to one core (the first this process may use)
    for the CPU leg, and restores the previous affinity afterwards. The GPU
    runtime's own threads are not affected."""
    prev = os.sched_getaffinity(0)
    core = min(prev)
    os.sched_setaffinity(0, {core})
    try:
        yield core
    finally:
        os.sched_setaffinity(0, prev)


def cpu_time(fn, budget_s: float, max_calls: int = 1000) -> tuple:
    """Calls fn until budget_s of CPU time has passed (at least once); returns
    (seconds per call, calls)."""
    calls, t0 = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        el = time.perf_counter() - t0
        if el >= budget_s or calls >= max_calls:
            return el / calls, calls


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_record(value: float, unit: str, core: int, sample: str) -> dict:
    return {"value": round(value, 6), "unit": unit, "cores": 1, "kind": "port", "sample": sample,
            "pinned_core": core, "host_cpu": _cpu_model(), "host_nproc": os.cpu_count()}


def cpu_gemm_slice(M: int, N: int, K: int, G: int, bits: int, n_slice: int, budget_s: float) -> dict:
    """dequant + cpuGemmNT (src/Check.swift:433-494) of the first n_slice output
    columns of an [M,K] x [N,K]^T forward; the cost is linear in N, so the
    rate of the slice is the rate of the whole."""
    import numpy as np
    orc = _oracle()
    rng = np.random.default_rng(0)
    n = min(n_slice, N)
    x = rng.standard_normal(M * K, dtype=np.float32)
    w = rng.standard_normal(n * K, dtype=np.float32) * np.float32(0.02)
    q, s = orc.quant(w, n, K, G, bits)

    def run():
        wd = orc.dequant(q, s, n, K, G, bits)
        orc.gemm_nt(x, wd, None, M, n, K)

    with one_core() as core:
        per, calls = cpu_time(run, budget_s, 50)
    flops = 2.0 * M * n * K
    what = "all of N" if n == N else f"N-slice {n} of {N} (cost linear in N; rate extrapolated)"
    return cpu_record(flops / per / 1e12, "TFLOP/s", core,
                      f"M={M} K={K} int{bits} G={G}, {what}: {calls} call(s) of dequant + cpuGemmNT, "
                      f"{per:.3f} s/call, oracle/oracle.c -O2 -ffp-contract=off, 1 thread")


# ---- workloads -------------------------------------------------------------------


def bench_c5(b: Bench, bits: int, steps: int, warmup: int, cpu: bool) -> dict:
    """c5: prefill-shaped int4/int8 forward on bf16 MFMA (DGM_MATH_BF16)."""
    M, N, K, G = C5["M"], C5["N"], C5["K"], C5["G"]
    w = b.randn(N * K, 0.02)
    q, s = b.quantized(w, N, K, G, bits)
    del w
    x = b.randn(M * K, 1.0)
    y = b.zeros(M * N)
    with b.math(b.dgm.DGM_MATH_BF16):
        r = b.time_steps(lambda i: b.gpu.gemmNT(bits, None, q, s, x, None, y, M, N, K, G), steps, warmup)
    flops = 2 * M * N * K
    ev = r["event_ms"]
    med, mean = statistics.median(ev), sum(ev) / len(ev)
    nbytes = N * K // (2 if bits == 4 else 1) + N * (K // G) * 4 + 4 * (M * K + M * N)
    kernels = [f"gemm_bf16_kernel<{bits}>", "x_to_bf16_kernel"]   # the call's two launches
    roof = roofline(flops / mean / 1e9, PEAK["bf16_TFLOPs"], "TFLOP/s", "mfma",
                    traffic_for(f"c5_int{bits}", kernels))
    roof.update({"kernel": f"gemm_nt_i{bits}", "device_kernels": kernels, "avg_launch_us": round(mean * 1e3, 3),
                 "algorithmic_flop": flops, "algorithmic_bytes": nbytes})
    out = {"kernel": f"gemm_nt_i{bits}", "math": "bf16", "shape": f"M=8192 K=4096 N=14336 int{bits} G=128",
           "steps": steps, "us_wall_per_step": round(r["wall_ms_per_step"] * 1e3, 3),
           "us_median": round(med * 1e3, 3), "us_mean": round(mean * 1e3, 3),
           "us_min": round(min(ev) * 1e3, 3), "us_max": round(max(ev) * 1e3, 3),
           "TFLOPs": round(flops / r["wall_ms_per_step"] / 1e9, 3),
           "TFLOPs_median": round(flops / med / 1e9, 3), "roofline": roof}
    if cpu:
        log(f"[bench] c5 int{bits}: cpu baseline")
        out["cpu_baseline"] = cpu_gemm_slice(M, N, K, G, bits, 256, 8.0)
    return out


def bench_c4(b: Bench, reps: int, M: int, math_mode: int, cpu: bool, valu: bool = False) -> dict:
    """Decode-shaped int4: K=4096, N=14336, G=128. Weight copies are rotated so
    that successive launches never find W in the 256 MB Infinity Cache. With
    valu, the same call on the wave-reduction VALU GEMV probe
    (dgm_probe_gemv_valu, no bias), the design the MFMA kernels are measured
    against."""
    N, K, G = C4["N"], C4["K"], C4["G"]
    wq_bytes = N * K // 2 + N * (K // G) * 4
    copies = max(2, -(-512 * 2 ** 20 // wq_bytes))
    w = b.randn(N * K, 0.02)
    q0, s0 = b.quantized(w, N, K, G, 4)
    del w
    Q = [q0] + [q0.clone() for _ in range(copies - 1)]
    S = [s0] + [s0.clone() for _ in range(copies - 1)]
    x = b.randn(M * K, 1.0)
    y = b.zeros(M * N)
    if valu:
        call = lambda i: b.gpu.probeGemvValu(Q[i % copies], S[i % copies], x, y, M, N, K, G)
    else:
        call = lambda i: b.gpu.gemmNT(4, None, Q[i % copies], S[i % copies], x, None, y, M, N, K, G)
    with b.math(math_mode):
        ms = b.time_launches(call, reps)
    flops = 2 * M * N * K
    nbytes = wq_bytes + 4 * (M * K + M * N)
    mode = "fp32" if math_mode == b.dgm.DGM_MATH_FP32 else "bf16"
    del Q, S
    name = f"c4_valu_gemv_m{M}" if valu else f"c4_int4_m{M}_{mode}"
    keys = ["gemv_valu"] if valu else ["skinny", "tiled", "decode", "stream", "slab"]
    out = {"kernel": "probe_gemv_valu" if valu else "gemm_nt_i4", "math": mode,
           "shape": f"M={M} K=4096 N=14336 int4 G=128",
           "us": round(ms * 1e3, 3), "GBps": round(nbytes / ms / 1e6, 2),
           "TFLOPs": round(flops / ms / 1e9, 3), "weight_copies_rotated": copies,
           "algorithmic_bytes": nbytes,
           "roofline": roofline(nbytes / ms / 1e6, PEAK["hbm_GBps"], "GB/s", "hbm",
                                traffic_for(name, keys))}
    if b.read_ceiling_c4:
        out["frac_of_read_ceiling"] = round(nbytes / ms / 1e6 / b.read_ceiling_c4, 4)
    if cpu:
        # The reference's CPU path does the same work at any M per output
        # column; time a slice of N sized to about a second.
        out["cpu_baseline"] = cpu_gemm_slice(M, N, K, G, 4, N if M == 1 else max(256, 16384 // M), 1.5)
        out["cpu_baseline"]["unit"] = "TFLOP/s"
    return out


def c2_parts(b: Bench):
    M, N, K, G = C2["M"], C2["N"], C2["K"], C2["G"]
    x, w, dy = b.randn(M * K, 1.0), b.randn(N * K, 0.02), b.randn(M * N, 1e-3)
    q, s = b.quantized(w, N, K, G, 4)
    y, dx, dw = b.zeros(M * N), b.zeros(M * K), b.zeros(N * K)
    g = b.gpu
    return {
        "gemm_nt_i4": lambda i: g.gemmNT(4, None, q, s, x, None, y, M, N, K, G),
        "gemm_bwd_i4": lambda i: g.gemmBwd(4, None, q, s, dy, x, dx, dw, M, N, K, G),
        "gemm_dx_i4": lambda i: g.gemmDX(4, None, q, s, dy, dx, M, N, K, G),
        "gemm_dw": lambda i: g.gemmDW(dy, x, dw, M, N, K),
    }


def bench_c2(b: Bench, reps: int, cpu: bool) -> dict:
    """c2: one int4 linear forward plus its STE backward, M=512, K=768, N=192,
    G=32: gemmNT, then gemmBwd (the reference's gemmDW + gemmDX pair in one
    launch, bitwise the two calls). The separate dX and dW launches are timed
    beside it."""
    M, N, K, G = C2["M"], C2["N"], C2["K"], C2["G"]
    kern = c2_parts(b)
    step = lambda i: (kern["gemm_nt_i4"](i), kern["gemm_bwd_i4"](i))
    ms_step = b.time_launches(step, reps)
    per = {k: b.time_launches(f, reps) for k, f in kern.items()}
    gemm = 2 * M * N * K
    q, s = N * K // 2, N * (K // G) * 4
    nbytes = {"gemm_nt_i4": q + s + 4 * (M * K + M * N), "gemm_bwd_i4": q + s + 4 * (M * N + 2 * M * K + N * K)}
    out = {"kernel": "gemmNT + gemmBwd", "shape": "M=512 K=768 N=192 int4 G=32",
           "us_per_step": round(ms_step * 1e3, 3), "TFLOPs": round(3 * gemm / ms_step / 1e9, 3),
           "per_kernel_us": {k: round(v * 1e3, 3) for k, v in per.items()},
           "roofline": roofline(2 * gemm / per["gemm_bwd_i4"] / 1e9, PEAK["fp32_TFLOPs"], "TFLOP/s", "mfma",
                                traffic_for("c2", ["gemm_bwd_pair_kernel<4, 2>"])),
           "roofline_kernel": "gemm_bwd_i4 (gemm_bwd_pair_kernel<4, 2>)",
           "algorithmic_bytes": nbytes,
           "note": "latency-bound shape; fp32 MFMA (157.3 TFLOP/s) is the nearer roof"}
    if cpu:
        import numpy as np
        orc = _oracle()
        rng = np.random.default_rng(0)
        x = rng.standard_normal(M * K, dtype=np.float32)
        w = rng.standard_normal(N * K, dtype=np.float32) * np.float32(0.02)
        dy = rng.standard_normal(M * N, dtype=np.float32) * np.float32(1e-3)
        qh, sh = orc.quant(w, N, K, G, 4)

        def run():
            wd = orc.dequant(qh, sh, N, K, G, 4)
            orc.gemm_nt(x, wd, None, M, N, K)
            orc.gemm_dx(dy, wd, M, N, K)
            orc.gemm_dw(dy, x, M, N, K)

        with one_core() as core:
            per_s, calls = cpu_time(run, 3.0, 50)
        out["cpu_baseline"] = cpu_record(3 * gemm / per_s / 1e12, "TFLOP/s", core,
                                         f"{calls} whole c2 steps (dequant, cpuGemmNT, cpuGemmDX, cpuGemmDW), "
                                         f"{per_s * 1e3:.1f} ms/step, 1 thread")
    return out


def bench_c1(b: Bench, reps: int, cpu: bool) -> dict:
    M, N, K, G = C1["M"], C1["N"], C1["K"], C1["G"]
    x, w = b.randn(M * K, 1.0), b.randn(N * K, 0.02)
    q, s = b.quantized(w, N, K, G, 8)
    y = b.zeros(M * N)
    ms = b.time_launches(lambda i: b.gpu.gemmNT(8, None, q, s, x, None, y, M, N, K, G), reps)
    flops = 2 * M * N * K
    nbytes = N * K + N * (K // G) * 4 + 4 * (M * K + M * N)
    out = {"kernel": "gemm_nt_i8", "shape": "M=512 K=192 N=768 int8 G=32", "us": round(ms * 1e3, 3),
           "TFLOPs": round(flops / ms / 1e9, 3), "GBps": round(nbytes / ms / 1e6, 2),
           "roofline": roofline(flops / ms / 1e9, PEAK["fp32_TFLOPs"], "TFLOP/s", "mfma",
                                traffic_for("c1", ["gemm_fwd"])),
           "note": "latency-bound; fp32 MFMA is the nearer roof"}
    if cpu:
        out["cpu_baseline"] = cpu_gemm_slice(M, N, K, G, 8, N, 1.5)
    return out


# Kernels of one c3 forward (dit_loop.hip) and of the block backward.
C3_FWD_KERNELS = ["loop_row_kernel", "loop_attn_kernel", "loop_mlp_kernel", "loop_tail_kernel"]
C3_BWD_KERNELS = ["rms_bwd", "gemm_bwd", "loop_attn_bwd_kernel", "wt_prep_kernel", "acc_kernel"]


def c3_flops(cfg) -> int:
    """Linear + attention flop of the looped block forward (src/DiT.swift:520-550)."""
    M, C, F, KV, T, H, D = cfg.B * cfg.T, cfg.C, cfg.F, cfg.D, cfg.T, cfg.H, cfg.D
    lin = 2 * M * C * (C + 2 * KV + C + 2 * F) + 2 * M * F * C
    att = 2 * 2 * cfg.B * H * T * T * D
    return cfg.loops * (lin + att)


def _dit_block(b: Bench):
    dgm = b.dgm
    cfg = dgm.DiTConfig()
    w = {n: b.randn(N * K, 0.02) for n, (N, K) in cfg.linear_shapes().items()}
    for n in dgm.DIT_NORMS:
        w[n] = b.torch.ones(cfg.C, dtype=b.torch.float32, device="cuda")
    b.sync()
    with b.torch.cuda.stream(b.stream):
        blk = dgm.DiTBlock(b.gpu, cfg, w)
    return cfg, w, blk


def _cpu_dit(cfg, train: bool, budget_s: float) -> dict:
    import numpy as np
    orc = _oracle()
    dgm = load_package()
    rng = np.random.default_rng(0)
    ocfg = orc.DiTCfg(B=cfg.B, T=cfg.T, C=cfg.C, F=cfg.F, H=cfg.H, D=cfg.D, loops=cfg.loops, group=cfg.group,
                      bits=cfg.bits, eps=cfg.eps, theta=cfg.theta, mix=cfg.mix)
    shapes = cfg.linear_shapes()
    wts = {n: (rng.standard_normal(N * K, dtype=np.float32) * np.float32(0.02)) for n, (N, K) in shapes.items()}
    qw = {n: orc.quant(wts[n], shapes[n][0], shapes[n][1], cfg.group, cfg.bits) for n in dgm.DIT_LINEARS}
    norms = {n: np.ones(cfg.C, np.float32) for n in dgm.DIT_NORMS}
    x0 = rng.standard_normal(cfg.B * cfg.T * cfg.C, dtype=np.float32)
    if train:
        gy = rng.standard_normal(cfg.B * cfg.T * cfg.C, dtype=np.float32) * np.float32(1e-2)
        run = lambda: orc.dit_train(ocfg, qw, norms, x0, gy)
    else:
        qw.update(norms)
        run = lambda: orc.dit_forward(ocfg, qw, x0)
    with one_core() as core:
        per, calls = cpu_time(run, budget_s, 20)
    tokens = cfg.B * cfg.T
    what = "forward with saved activations + block backward" if train else "forward"
    return cpu_record(tokens / per, "tokens/s", core,
                      f"{calls} whole c3 {what} call(s) (4 loops, int8 G=32, quantized linears in the Metal "
                      f"kernel order), {per * 1e3:.1f} ms/call, 1 thread")


def bench_c3(b: Bench, reps: int, cpu: bool) -> dict:
    """c3: the photos-dit looped block forward, 8x64 tokens, 4 loops, int8 G=32
    linears; weights ~N(0,0.02), norms 1, xs[0] ~N(0,1), all resident. The
    timed call is the whole 4-loop forward (dgm_dit_forward), in place on x."""
    cfg, _, blk = _dit_block(b)
    x = b.randn(cfg.B * cfg.T * cfg.C, 1.0)
    ms = b.time_launches(lambda i: blk.forward(x), reps)
    tokens = cfg.B * cfg.T
    flops = c3_flops(cfg)
    out = {"kernel": "dit_forward (4 loops)", "shape": "B=8 T=64 C=192 F=768 H=4 D=48 int8 G=32",
           "us": round(ms * 1e3, 3), "tokens_per_s": round(tokens / (ms * 1e-3), 1),
           "TFLOPs": round(flops / ms / 1e9, 3), "flop": flops,
           "roofline": roofline(flops / ms / 1e9, PEAK["fp32_TFLOPs"], "TFLOP/s", "mfma",
                                traffic_for("c3", C3_FWD_KERNELS, "loop_tail_kernel")),
           "note": "launch/latency-bound: ~2.3 GFLOP and ~0.6 MB of weights per forward; traffic = the "
                   "forward's 13 launches (three per loop and the tail), each at its counted bytes"}
    if cpu:
        out["cpu_baseline"] = _cpu_dit(cfg, False, 3.0)
    return out


def bench_c3_train(b: Bench, reps: int, cpu: bool) -> dict:
    """One training step of the c3 block (weights as in bench_c3): the forward
    that saves every loop's activations, then the block backward (int8 STE:
    dX through the codes, dW into fp32 gradients) from dL/dxs[4] ~N(0,1e-2).
    Flop: the forward's, plus dX and dW of every linear and the four
    attention backward products (3x the forward)."""
    cfg, _, blk = _dit_block(b)
    with b.torch.cuda.stream(b.stream):
        blk.zero_grads()
    x0 = b.randn(cfg.B * cfg.T * cfg.C, 1.0)
    g0 = b.randn(cfg.B * cfg.T * cfg.C, 1e-2)
    x, g = x0.clone(), g0.clone()

    def step(i):
        blk.forward_train(x)
        blk.backward(g)

    ms = b.time_launches(step, reps)
    flops = 3 * c3_flops(cfg)
    tokens = cfg.B * cfg.T
    out = {"kernel": "dit_forward_train + dit_backward (4 loops)",
           "shape": "B=8 T=64 C=192 F=768 H=4 D=48 int8 G=32",
           "us": round(ms * 1e3, 3), "tokens_per_s": round(tokens / (ms * 1e-3), 1),
           "TFLOPs": round(flops / ms / 1e9, 3), "flop": flops,
           "roofline": roofline(flops / ms / 1e9, PEAK["fp32_TFLOPs"], "TFLOP/s", "mfma",
                                traffic_for("c3_train", C3_FWD_KERNELS + C3_BWD_KERNELS, "wt_prep_kernel")),
           "note": "launch/latency-bound; x and dL/dx are reused in place across the timed steps; traffic = "
                   "every launch of one step at its counted bytes"}
    if cpu:
        out["cpu_baseline"] = _cpu_dit(cfg, True, 4.0)
    return out


def bench_quant(b: Bench, reps: int, bits: int, cpu: bool) -> dict:
    """quantize of the c4/c5 weight, W[14336,4096] G=128. Successive launches
    rotate over distinct (W, codes, scales) sets totalling at least 768 MiB,
    so that no launch finds its operands in the 256 MB Infinity Cache."""
    N, K, G = C4["N"], C4["K"], C4["G"]
    nbytes = 4 * N * K + (N * K // (2 if bits == 4 else 1)) + 4 * N * (K // G)
    sets = max(2, -(-768 * 2 ** 20 // nbytes))
    w0 = b.randn(N * K, 0.02)
    W = [w0] + [w0.clone() for _ in range(sets - 1)]
    Q = [b.zeros(N * K // (2 if bits == 4 else 1), b.torch.uint8) for _ in range(sets)]
    S = [b.zeros(N * (K // G)) for _ in range(sets)]
    ms = b.time_launches(lambda i: b.gpu.quantize(W[i % sets], Q[i % sets], S[i % sets], N, K, bits, G), reps)
    del W, Q, S
    out = {"kernel": f"quant_i{bits}", "shape": "W[14336,4096] G=128", "us": round(ms * 1e3, 3),
           "GBps": round(nbytes / ms / 1e6, 2), "operand_sets_rotated": sets,
           "roofline": roofline(nbytes / ms / 1e6, PEAK["hbm_GBps"], "GB/s", "hbm",
                                traffic_for(f"quant_i{bits}", ["quant_vec_kernel"]))}
    if cpu:
        import numpy as np
        orc = _oracle()
        rows = 1024
        wh = np.random.default_rng(0).standard_normal(rows * K, dtype=np.float32) * np.float32(0.02)
        with one_core() as core:
            per, calls = cpu_time(lambda: orc.quant(wh, rows, K, G, bits), 1.0, 200)
        out["cpu_baseline"] = cpu_record(rows * K * (4 + (0.5 if bits == 4 else 1)) / per / 1e9, "GB/s", core,
                                         f"cpuQuant of a {rows}x{K} slice, {calls} calls, {per * 1e3:.1f} ms "
                                         f"each, 1 thread")
    return out


def bench_adam_quant(b: Bench, reps: int, bits: int, cpu: bool) -> dict:
    """AdamW + re-quantization of the c4/c5 weight (W[14336,4096], G=128): the
    fused pass against adam followed by quantize. Algorithmic bytes per
    element: w, g, m, v read (16) + w, m, v written (12) + codes (0.5 or 1),
    plus the scales."""
    N, K, G = C4["N"], C4["K"], C4["G"]
    n = N * K
    w, g = b.randn(n, 0.02), b.randn(n, 1.0)
    m, v = b.zeros(n), b.zeros(n)
    q = b.zeros(n // (2 if bits == 4 else 1), b.torch.uint8)
    s = b.zeros(N * (K // G))
    hp = (1e-4, 0.9, 0.95, 1e-8, 0.1, 10.0, 20.0)
    fused = b.time_launches(lambda i: b.gpu.adamQuantize(w, g, m, v, q, s, N, K, bits, G, *hp), reps)

    def pair(i):
        b.gpu.adam(w, g, m, v, n, *hp)
        b.gpu.quantize(w, q, s, N, K, bits, G)

    unfused = b.time_launches(pair, reps)
    code_b = n // (2 if bits == 4 else 1)
    nbytes = 28 * n + code_b + 4 * N * (K // G)
    out = {"kernel": "adam_quantize", "shape": f"W[14336,4096] int{bits} G=128", "us": round(fused * 1e3, 3),
           "GBps": round(nbytes / fused / 1e6, 2), "unfused_us": round(unfused * 1e3, 3),
           "roofline": roofline(nbytes / fused / 1e6, PEAK["hbm_GBps"], "GB/s", "hbm",
                                traffic_for(f"adam_quant_i{bits}", ["adam_quant_kernel"]))}
    if cpu:
        import numpy as np
        orc = _oracle()
        rows = 512
        rng = np.random.default_rng(0)
        wh = rng.standard_normal(rows * K, dtype=np.float32) * np.float32(0.02)
        gh = rng.standard_normal(rows * K, dtype=np.float32)
        z = np.zeros(rows * K, np.float32)
        with one_core() as core:
            per, calls = cpu_time(lambda: orc.adam_quantize(wh, gh, z, z, rows, K, G, bits, *hp), 1.0, 200)
        out["cpu_baseline"] = cpu_record(rows * K * (28 + (0.5 if bits == 4 else 1)) / per / 1e9, "GB/s", core,
                                         f"adamw then cpuQuant of a {rows}x{K} slice, {calls} calls, "
                                         f"{per * 1e3:.1f} ms each, 1 thread")
    return out


def bench_embed_bwd(b: Bench, reps: int, cpu: bool) -> dict:
    """embed_bwd at the quantized GPT's default shape (src/GPT.swift:374-376;
    16 x 64 tokens, C 128, a 65-symbol vocabulary) with Zipf-like token counts."""
    t = b.torch
    B, T, C, V = 16, 64, 128, 65
    ranks = t.arange(1, V + 1, dtype=t.float64)
    probs = (1.0 / ranks) / (1.0 / ranks).sum()
    toks = t.multinomial(probs, B * T, replacement=True, generator=b.gen).to(t.int32)
    dx, dwe = b.randn(B * T * C, 1.0), b.zeros(V * C)
    toks_d = toks.to("cuda")
    ms = b.time_launches(lambda i: b.gpu.embedBwd(toks_d, dx, dwe, B, T, C, V), reps)
    nbytes = 4 * (B * T * C + 2 * V * C + B * T)
    out = {"kernel": "embed_bwd", "shape": "B=16 T=64 C=128 V=65", "us": round(ms * 1e3, 3),
           "GBps": round(nbytes / ms / 1e6, 2), "note": "latency-bound: 1 MB of traffic",
           "roofline": roofline(nbytes / ms / 1e6, PEAK["hbm_GBps"], "GB/s", "hbm",
                                traffic_for("embed_bwd", ["embed_bwd_kernel"]))}
    if cpu:
        import numpy as np
        orc = _oracle()
        th = toks.numpy().astype(np.uint32)
        dxh = np.random.default_rng(0).standard_normal(B * T * C, dtype=np.float32)
        z = np.zeros(V * C, np.float32)
        with one_core() as core:
            per, calls = cpu_time(lambda: orc.embed_bwd(th, dxh, z, B, T, C, V), 1.0, 200)
        out["cpu_baseline"] = cpu_record(nbytes / per / 1e9, "GB/s", core,
                                         f"embed_bwd (V*B*T*C scan of the reference kernel), {calls} calls, "
                                         f"{per * 1e3:.2f} ms each, 1 thread")
    return out


def hbm_ceiling(b: Bench) -> dict:
    """The box's measured stream ceiling: a device copy of CEIL_BYTES (read
    CEIL_BYTES + write CEIL_BYTES, 2x the 256 MB Infinity Cache each way),
    20 copies bracketed by HIP events."""
    t = b.torch
    n = CEIL_BYTES // 4
    src = t.ones(n, device="cuda")
    dst = t.zeros(n, device="cuda")
    b.sync()
    with t.cuda.stream(b.stream):
        for _ in range(3):
            dst.copy_(src)
        e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        e0.record(b.stream)
        for _ in range(20):
            dst.copy_(src)
        e1.record(b.stream)
    e1.synchronize()
    ms = e0.elapsed_time(e1) / 20
    gbps = 2 * CEIL_BYTES / ms / 1e6
    del src, dst
    return {"kernel": "torch device copy", "bytes_each_way": CEIL_BYTES, "us": round(ms * 1e3, 3),
            "GBps": round(gbps, 1), "frac_of_8TBps": round(gbps / PEAK["hbm_GBps"], 4)}


def hbm_read_ceiling(b: Bench) -> dict:
    """The box's measured read ceiling for one launch: this library's read-only
    probe (dgm_probe_read) over (i) one c4 weight copy (codes + scales,
    31,195,136 bytes), rotated over as many copies as bench_c4 uses so that no
    launch finds it in the 256 MB Infinity Cache, and (ii) 512 MiB (two
    buffers, alternated); 16-byte register loads and direct-to-LDS loads, one
    workgroup per CU and more. Graph replays, as for the c4 lines, so the
    per-launch cost is included the same way."""
    t = b.torch
    N, K, G = C4["N"], C4["K"], C4["G"]
    wq = N * K // 2 + N * (K // G) * 4
    copies = max(2, -(-512 * 2 ** 20 // wq))
    sink = b.zeros(1 << 16, t.int32)
    out = {}
    big = 512 * 2 ** 20
    for name, nbytes, nbuf, reps in (("c4_weight_copy", wq, copies, 72), ("512MiB", big, 2, 10)):
        buf = t.ones(nbytes * nbuf, dtype=t.uint8, device="cuda")
        rows = []
        for mode in (0, 1):
            for wgs in (256, 512, 1024):
                ms = b.time_launches(
                    lambda i: b.gpu.probeRead(buf[(i % nbuf) * nbytes:], nbytes, mode, wgs, sink), reps)
                rows.append({"mode": ("registers", "direct-to-LDS")[mode], "workgroups": wgs,
                             "us": round(ms * 1e3, 3), "GBps": round(nbytes / ms / 1e6, 1)})
        best = max(rows, key=lambda r: r["GBps"])
        out[name] = {"bytes": nbytes, "buffers_rotated": nbuf, "launches_per_graph": reps, "results": rows,
                     "best_GBps": best["GBps"], "best": f"{best['mode']}, {best['workgroups']} workgroups",
                     "frac_of_8TBps": round(best["GBps"] / PEAK["hbm_GBps"], 4)}
        del buf
        t.cuda.empty_cache()
    b.read_ceiling_c4 = out["c4_weight_copy"]["best_GBps"]
    return out


def calib_copy(b: Bench) -> dict:
    """A plain device copy of CALIB_BYTES, for scaling the --pmc traffic
    counters (its algorithmic traffic is CALIB_BYTES read + CALIB_BYTES written)."""
    t = b.torch
    n = CALIB_BYTES // 4
    src = t.ones(n, device="cuda")
    dst = t.zeros(n, device="cuda")
    b.sync()
    for _ in range(10):
        dst.copy_(src)
    b.sync()
    return {"bytes": CALIB_BYTES}


def workload_table(b, args, cpu: bool):
    F, H = 0, 1   # DGM_MATH_FP32, DGM_MATH_BF16 (include/dgm_quant.h)
    return [
        ("c5_int8", lambda: bench_c5(b, 8, max(args.steps, 20), max(args.warmup, 3), cpu)),
        ("c4_int4_m1_fp32", lambda: bench_c4(b, 72, 1, F, cpu)),
        ("c4_int4_m1_bf16", lambda: bench_c4(b, 72, 1, H, cpu)),
        ("c4_int4_m16_fp32", lambda: bench_c4(b, 72, 16, F, cpu)),
        ("c4_int4_m16_bf16", lambda: bench_c4(b, 72, 16, H, cpu)),
        ("c4_int4_m64_fp32", lambda: bench_c4(b, 72, 64, F, cpu)),
        ("c4_int4_m64_bf16", lambda: bench_c4(b, 72, 64, H, cpu)),
        ("c4_valu_gemv_m1", lambda: bench_c4(b, 72, 1, F, False, valu=True)),
        ("c4_valu_gemv_m16", lambda: bench_c4(b, 72, 16, F, False, valu=True)),
        ("c1", lambda: bench_c1(b, args.reps, cpu)),
        ("c2", lambda: bench_c2(b, args.reps, cpu)),
        ("c3", lambda: bench_c3(b, 50, cpu)),
        ("c3_train", lambda: bench_c3_train(b, 10, cpu)),
        ("quant_i4", lambda: bench_quant(b, 20, 4, cpu)),
        ("quant_i8", lambda: bench_quant(b, 20, 8, cpu)),
        ("adam_quant_i4", lambda: bench_adam_quant(b, 10, 4, cpu)),
        ("adam_quant_i8", lambda: bench_adam_quant(b, 10, 8, cpu)),
        ("embed_bwd", lambda: bench_embed_bwd(b, 50, cpu)),
    ]


# ---- rocprofv3 output helpers (run on the CPU) ---------------------------------


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "")
    return name.split("(")[0] if "(" in name else name


def _find(d: str, suffix: str):
    for root, _, files in os.walk(d):
        for f in files:
            if f.endswith(suffix):
                return os.path.join(root, f)
    return None


def summarize(d: str, title: str) -> str:
    out = [f"# {title}", ""]
    ks = _find(d, "kernel_stats.csv")
    if ks:
        rows = list(csv.DictReader(open(ks)))
        out += ["| kernel | calls | avg us | min us | max us | total % |", "|---|---|---|---|---|---|"]
        for r in rows:
            out.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.3f} | "
                       f"{float(r['MinNs']) / 1e3:.3f} | {float(r['MaxNs']) / 1e3:.3f} | "
                       f"{float(r['Percentage']):.2f} |")
        out.append("")
    cc = _find(d, "counter_collection.csv")
    if cc:
        agg: dict = {}
        for r in csv.DictReader(open(cc)):
            k = _short(r["Kernel_Name"])
            agg.setdefault(k, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
        names = sorted({c for v in agg.values() for c in v})
        out += ["| kernel | dispatches | " + " | ".join(names) + " |", "|---" * (len(names) + 2) + "|"]
        for k, v in agg.items():
            n = max(len(x) for x in v.values())
            out.append(f"| `{k}` | {n} | " + " | ".join(
                f"{sum(v[c]) / len(v[c]):.1f}" if c in v else "" for c in names) + " |")
        out.append("")
    return "\n".join(out)


def _counter_values(d: str, counter: str) -> dict:
    cc = _find(d, "counter_collection.csv")
    if not cc:
        raise FileNotFoundError(f"no counter_collection.csv under {d}")
    agg: dict = {}
    for r in csv.DictReader(open(cc)):
        if r["Counter_Name"] == counter:
            agg.setdefault(_short(r["Kernel_Name"]), []).append(float(r["Counter_Value"]))
    return agg


def traffic(name: str, fetch_dir: str, write_dir: str) -> dict:
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) -> bytes per launch, scaled so
    that the calibration copy reads and writes exactly CALIB_BYTES. The
    calibration copy is the largest single dispatch of the copy kernel (the
    workloads' own buffer copies use the same kernel); every other kernel is
    averaged over its dispatches."""
    fv = _counter_values(fetch_dir, "FETCH_SIZE")
    wv = _counter_values(write_dir, "WRITE_SIZE")
    fetch = {k: sum(v) / len(v) for k, v in fv.items()}
    write = {k: sum(v) / len(v) for k, v in wv.items()}
    copy = [k for k in fetch if "copy" in k.lower() or "elementwise" in k.lower()]
    if not copy:
        raise RuntimeError("calibration copy kernel not found (run the PMC passes with --calib-copy)")
    ck = max(copy, key=lambda k: max(fv[k]))
    f_scale = CALIB_BYTES / (max(fv[ck]) * 1024.0)
    w_scale = CALIB_BYTES / (max(wv[ck]) * 1024.0) if wv.get(ck) else 1.0
    rec = {"_calibration": {"kernel": ck, "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4)}}
    for k in fetch:
        if k == ck or "copy" in k.lower() or "elementwise" in k.lower() or "fill" in k.lower():
            continue
        fb = fetch[k] * 1024.0 * f_scale
        wb = write.get(k, 0.0) * 1024.0 * w_scale
        rec[k] = {"fetch_bytes": round(fb), "write_bytes": round(wb), "total_bytes": round(fb + wb),
                  "dispatches": len(fv[k])}
    allt = load_traffic()
    allt[name] = rec
    os.makedirs(os.path.dirname(TRAFFIC_JSON), exist_ok=True)
    with open(TRAFFIC_JSON, "w") as f:
        json.dump(allt, f, indent=1, sort_keys=True)
    return rec


# ---- main -------------------------------------------------------------------------


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--reps", type=int, default=100, help="launches per graph-timed workload")
    ap.add_argument("--skip-extra", action="store_true", help="headline only")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list of workloads (c5_int4 = the headline)")
    ap.add_argument("--list", action="store_true")
    ap.add_argument("--calib-copy", action="store_true", help="run the traffic calibration copy at the end")
    ap.add_argument("--summarize", metavar="DIR")
    ap.add_argument("--title", default="rocprofv3 summary")
    ap.add_argument("--traffic", nargs=3, metavar=("NAME", "FETCH_DIR", "WRITE_DIR"))
    args = ap.parse_args()

    if args.summarize:
        print(summarize(args.summarize, args.title))
        return 0
    if args.traffic:
        print(json.dumps(traffic(*args.traffic), indent=1))
        return 0

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the reference is single-device); run with --gpus 1.", file=sys.stderr)
        return 2

    if args.list:
        print("\n".join(["c5_int4 (headline)", "hbm_ceiling", "hbm_read_ceiling"] +
                        [n for n, _ in workload_table(None, args, False)]))
        return 0
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    dgm = load_package()
    b = Bench(dgm, torch)
    cpu = not args.skip_cpu
    only = set(filter(None, args.only.split(",")))
    want = lambda name: not only or name in only

    out: dict = {}
    if want("c5_int4"):
        log(f"[bench] headline c5 int4: {args.warmup} warmup + {args.steps} timed steps")
        head = bench_c5(b, 4, args.steps, args.warmup, cpu)
        torch.cuda.empty_cache()
        M, N, K = C5["M"], C5["N"], C5["K"]
        out = {
            "metric": METRIC,
            "value": head["TFLOPs"],
            "unit": "TFLOP/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(head["us_wall_per_step"] / 1e3, 6),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16",
            "data": "synthetic (torch CPU generator, seed 1234: X~N(0,1), W~N(0,0.02) quantized int4 G=128 once "
                    "before timing)",
            "config": {"workload": "c5: prefill-shaped int4 group-quant GEMM forward (gemmNT), W dequantized to "
                                   "bf16 in LDS, bf16 MFMA, fp32 accumulate",
                       "M": M, "K": K, "N": N, "group": C5["G"], "bits": 4, "math": "DGM_MATH_BF16",
                       "parallelism": "single GPU", "timing": "eager calls, wall clock over the timed steps"},
            "us_median": head["us_median"],
            "TFLOPs_median": head["TFLOPs_median"],
            "frac_of_bf16_peak": round(head["TFLOPs"] / PEAK["bf16_TFLOPs"], 4),
            "roofline": head["roofline"],
        }
        if "cpu_baseline" in head:
            out["cpu_baseline"] = head["cpu_baseline"]
        log(f"[bench] c5 int4 {head['us_wall_per_step']:.1f} us/step = {head['TFLOPs']:.1f} TFLOP/s")

    if want("hbm_ceiling") or not only:
        log("[bench] hbm ceiling (stream copy)")
        out["hbm_ceiling"] = hbm_ceiling(b)
        torch.cuda.empty_cache()
    if want("hbm_read_ceiling") or not only or any(n.startswith("c4_") for n in only):
        log("[bench] hbm read ceiling (read-only probe)")
        out["hbm_read_ceiling"] = hbm_read_ceiling(b)
        torch.cuda.empty_cache()

    if not args.skip_extra:
        W = {}
        for name, fn in workload_table(b, args, cpu):
            if not want(name):
                continue
            log(f"[bench] {name}")
            try:
                W[name] = fn()
            except Exception as e:   # report, keep the headline line intact
                W[name] = {"error": f"{type(e).__name__}: {e}"}
            torch.cuda.empty_cache()
        out["workloads"] = W

    if args.calib_copy:
        log("[bench] calibration copy")
        out["calibration_copy"] = calib_copy(b)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
