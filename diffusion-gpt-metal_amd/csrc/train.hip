// The training step around the quantized linears: AdamW on the fp32 masters
// and their re-quantization, the gradient-norm clip, and the quantized token
// embedding (forward and backward) that shares the codes.
//
// Semantics follow the Metal kernels element for element (each fp32 operation
// rounded on its own, fp contraction off):
//   adamw          metal/kernels.metal:786-802
//   reduce_sumsq   metal/kernels.metal:749-768 (own summation order, below)
//   zero_f/scale_f metal/kernels.metal:770-784
//   embed_*        metal/kernels.metal:616-663
//   embed_bwd      metal/kernels.metal:665-682
//   pos_bwd        metal/kernels.metal:684-697
//   bias_grad      metal/kernels.metal:285-295
// and the host wrappers src/GPU.swift:200-210, 274-277, 324-350, 420-429.
//
// Design. Everything here is HBM-bound streaming or a gather, so the kernels
// are built for full-line vector traffic, not for MFMA:
// * adamw: each lane owns 8 consecutive elements (two 16-byte loads per
//   stream): 16 B read + 12 B written per element.
// * adam_quantize: the same lanes then reduce each group's maxAbs with xor
//   shuffles (G/8 lanes per group, as the quantizer does) and write codes and
//   scales, so the re-quantization reads no byte a second time: the pair
//   adamw + quant_i4 moves 32.5 B per element, the fused pass 28.5 B.
// * embed_bwd: the reference gives each (v, c) a thread that scans all B*T
//   tokens (V*B*T*C loads). Here one wave owns one vocabulary row and a strip
//   of columns: it ballots 64 tokens at a time (1024 loaded at once) into an
//   ordered LDS list of the matching positions, then adds those dx rows into
//   per-lane sums, 16 or 32 rows per batch with all loads issued first. dx is
//   read once in total and each sum keeps the reference's order, so results
//   are bitwise the reference's.
#include "common.hpp"
#include "quant_math.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 256;

struct AdamArgs {
    float lr, b1, b2, eps, wd, invBC1, invBC2;
};

// One element of adamw (metal/kernels.metal:795-801), literally.
__device__ __forceinline__ void adam_elem(float& w, float g, float& m, float& v, const AdamArgs& a) {
    const float mi = a.b1 * m + (1.0f - a.b1) * g;
    const float vi = a.b2 * v + (1.0f - a.b2) * g * g;
    m = mi;
    v = vi;
    const float upd = (mi * a.invBC1) / (sqrtf(vi * a.invBC2) + a.eps);
    w -= a.lr * (upd + a.wd * w);
}

// 8 elements per lane; n8 = n / 8 lanes do vector work, the tail (n % 8) is
// done element-wise by the first lanes of the last block.
__global__ __launch_bounds__(kThreads) void adamw_vec_kernel(float* __restrict__ W,
                                                             const float* __restrict__ G,
                                                             float* __restrict__ Mo,
                                                             float* __restrict__ Vo, int64_t n,
                                                             AdamArgs a) {
    const int64_t t = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t n8 = n / 8;
    if (t < n8) {
        float4* w4 = reinterpret_cast<float4*>(W) + 2 * t;
        float4* m4 = reinterpret_cast<float4*>(Mo) + 2 * t;
        float4* v4 = reinterpret_cast<float4*>(Vo) + 2 * t;
        const float4* g4 = reinterpret_cast<const float4*>(G) + 2 * t;
        float4 w0 = w4[0], w1 = w4[1], g0 = g4[0], g1 = g4[1];
        float4 m0 = m4[0], m1 = m4[1], v0 = v4[0], v1 = v4[1];
        adam_elem(w0.x, g0.x, m0.x, v0.x, a);
        adam_elem(w0.y, g0.y, m0.y, v0.y, a);
        adam_elem(w0.z, g0.z, m0.z, v0.z, a);
        adam_elem(w0.w, g0.w, m0.w, v0.w, a);
        adam_elem(w1.x, g1.x, m1.x, v1.x, a);
        adam_elem(w1.y, g1.y, m1.y, v1.y, a);
        adam_elem(w1.z, g1.z, m1.z, v1.z, a);
        adam_elem(w1.w, g1.w, m1.w, v1.w, a);
        w4[0] = w0; w4[1] = w1; m4[0] = m0; m4[1] = m1; v4[0] = v0; v4[1] = v1;
    }
    const int64_t tail = n - 8 * n8;
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x < tail) {
        const int64_t i = 8 * n8 + threadIdx.x;
        float w = W[i], m = Mo[i], v = Vo[i];
        adam_elem(w, G[i], m, v, a);
        W[i] = w; Mo[i] = m; Vo[i] = v;
    }
}

__global__ __launch_bounds__(kThreads) void adamw_scalar_kernel(float* __restrict__ W,
                                                                const float* __restrict__ G,
                                                                float* __restrict__ Mo,
                                                                float* __restrict__ Vo, int64_t n,
                                                                AdamArgs a) {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    float w = W[i], m = Mo[i], v = Vo[i];
    adam_elem(w, G[i], m, v, a);
    W[i] = w; Mo[i] = m; Vo[i] = v;
}

// AdamW + re-quantization, flat over the [rows, cols] master with
// cols % G == 0: L = G / 8 lanes per group, each lane 8 consecutive weights.
template <int BITS, int L>
__global__ __launch_bounds__(kThreads) void adam_quant_kernel(
    float* __restrict__ W, const float* __restrict__ G, float* __restrict__ Mo,
    float* __restrict__ Vo, void* __restrict__ Q, float* __restrict__ S, int64_t nthreads,
    AdamArgs a, float qmax, int lim) {
    const int64_t t = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    const bool valid = t < nthreads;
    // The valid count is a multiple of L and groups are L-aligned, so either
    // all lanes of a group are valid or none is; invalid lanes compute nothing
    // that is stored and take no part in a valid group's reduction.
    float w[8];
    if (valid) {
        float4* w4 = reinterpret_cast<float4*>(W) + 2 * t;
        float4* m4 = reinterpret_cast<float4*>(Mo) + 2 * t;
        float4* v4 = reinterpret_cast<float4*>(Vo) + 2 * t;
        const float4* g4 = reinterpret_cast<const float4*>(G) + 2 * t;
        float4 w0 = w4[0], w1 = w4[1], g0 = g4[0], g1 = g4[1];
        float4 m0 = m4[0], m1 = m4[1], v0 = v4[0], v1 = v4[1];
        adam_elem(w0.x, g0.x, m0.x, v0.x, a);
        adam_elem(w0.y, g0.y, m0.y, v0.y, a);
        adam_elem(w0.z, g0.z, m0.z, v0.z, a);
        adam_elem(w0.w, g0.w, m0.w, v0.w, a);
        adam_elem(w1.x, g1.x, m1.x, v1.x, a);
        adam_elem(w1.y, g1.y, m1.y, v1.y, a);
        adam_elem(w1.z, g1.z, m1.z, v1.z, a);
        adam_elem(w1.w, g1.w, m1.w, v1.w, a);
        w4[0] = w0; w4[1] = w1; m4[0] = m0; m4[1] = m1; v4[0] = v0; v4[1] = v1;
        w[0] = w0.x; w[1] = w0.y; w[2] = w0.z; w[3] = w0.w;
        w[4] = w1.x; w[5] = w1.y; w[6] = w1.z; w[7] = w1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = 0.0f;
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float x = fabsf(w[i]);
        mx = x >= mx ? x : mx;
    }
#pragma unroll
    for (int off = L / 2; off >= 1; off >>= 1) {
        const float o = __shfl_xor(mx, off, 64);
        mx = o >= mx ? o : mx;
    }
    const float s = dgm::group_scale(mx, qmax);
    if (!valid) return;
    if ((t % L) == 0) S[t / L] = s;
    if constexpr (BITS == 8) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) lo |= (uint32_t(dgm::quant_code(w[i], s, lim)) & 0xFFu) << (8 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i) hi |= (uint32_t(dgm::quant_code(w[4 + i], s, lim)) & 0xFFu) << (8 * i);
        reinterpret_cast<uint2*>(Q)[t] = make_uint2(lo, hi);
    } else {
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) packed |= (uint32_t(dgm::quant_code(w[i], s, lim)) & 0xFu) << (4 * i);
        reinterpret_cast<uint32_t*>(Q)[t] = packed;
    }
}

// ---- sum of squares ------------------------------------------------------
// Order (fixed for a given n): NB = ceil(n / kSumChunk) blocks, block b sums
// the contiguous range [b*kSumChunk, (b+1)*kSumChunk): lane l accumulates
// elements l, l+256, ... of the range with fmaf, then the block reduces its
// 256 lane sums with the halving tree 128, ..., 1. A second one-block pass
// sums the NB block sums the same way (lane l: partials l, l+256, ...). With
// NB == 1 the first pass writes out[slot] directly.
constexpr int64_t kSumChunk = 16384;

__device__ __forceinline__ float block_tree(float v, float* sh) {
    sh[threadIdx.x] = v;
    __syncthreads();
#pragma unroll
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (int(threadIdx.x) < s) sh[threadIdx.x] += sh[threadIdx.x + s];
        __syncthreads();
    }
    return sh[0];
}

__global__ __launch_bounds__(kThreads) void sumsq_partial_kernel(const float* __restrict__ X,
                                                                 int64_t n,
                                                                 float* __restrict__ out) {
    __shared__ float sh[kThreads];
    const int64_t base = int64_t(blockIdx.x) * kSumChunk;
    const int64_t end = base + kSumChunk < n ? base + kSumChunk : n;
    float v = 0.0f;
    for (int64_t i = base + threadIdx.x; i < end; i += kThreads) {
        const float a = X[i];
        v = fmaf(a, a, v);
    }
    const float total = block_tree(v, sh);
    if (threadIdx.x == 0) out[blockIdx.x] = total;
}

__global__ __launch_bounds__(kThreads) void sum_final_kernel(const float* __restrict__ part,
                                                             int64_t nb, float* __restrict__ out) {
    __shared__ float sh[kThreads];
    float v = 0.0f;
    for (int64_t i = threadIdx.x; i < nb; i += kThreads) v += part[i];
    const float total = block_tree(v, sh);
    if (threadIdx.x == 0) out[0] = total;
}

// ---- zero / scale ----------------------------------------------------------
__global__ __launch_bounds__(kThreads) void fill_scale_kernel(float* __restrict__ X, int64_t n,
                                                              float s, int zero) {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    X[i] = zero ? 0.0f : X[i] * s;
}

// ---- embedding forward -----------------------------------------------------
// One lane per output element; consecutive lanes take consecutive columns of
// one token row, so the table row, wpe row and y row are read and written as
// whole lines.
template <int BITS>
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint32_t* __restrict__ tokens,
                                                         const float* __restrict__ wte,
                                                         const void* __restrict__ q,
                                                         const float* __restrict__ scale,
                                                         const float* __restrict__ wpe,
                                                         float* __restrict__ y, int64_t BT, int T,
                                                         int C, int G) {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= BT * C) return;
    const int64_t bt = i / C;
    const int c = int(i - bt * C);
    const int t = int(bt % T);
    const int64_t tok = tokens[bt];
    float e;
    if constexpr (BITS == 32) {
        e = wte[tok * C + c];
    } else {
        const float s = scale[tok * (C / G) + c / G];
        int code;
        if constexpr (BITS == 8) {
            code = static_cast<const int8_t*>(q)[tok * C + c];
        } else {
            const uint8_t b = static_cast<const uint8_t*>(q)[(tok * C + c) >> 1];
            const int nib = (c & 1) ? (b >> 4) : (b & 0xF);   // metal/kernels.metal:69-75
            code = nib >= 8 ? nib - 16 : nib;
        }
        e = float(code) * s;
    }
    y[i] = e + wpe[int64_t(t) * C + c];
}

// ---- embedding backward ------------------------------------------------------
// One wave per vocabulary row v and strip of 64*COLS columns. Per round the
// wave loads 16 tokens per lane (1024 positions) and, 64 at a time, ballots
// them and writes the matching positions, in increasing order, into its own
// LDS list (each matching lane at its rank among the matches below it). It
// then walks the list BATCH positions at a time: lane b holds position b of
// the batch, every row's address comes from readlane, all BATCH x COLS loads
// are issued, and the rows are added into the lane sums in list order. Rows
// past the end of the list are loaded from a valid position and added as
// +0.0f, which leaves a sum unchanged (a sum starts at +0.0f and so is never
// -0.0f).
constexpr int kEbTok = 16;                 // tokens per lane per round
constexpr int kEbList = 64 * kEbTok;       // list entries per wave

template <int COLS, int BATCH>
__global__ __launch_bounds__(kThreads) void embed_bwd_kernel(const uint32_t* __restrict__ tokens,
                                                             const float* __restrict__ dx,
                                                             float* __restrict__ dwe, int BT,
                                                             int C, int V) {
    static_assert(BATCH <= 64, "one list position per lane");
    __shared__ int list[kThreads / 64][kEbList];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int v = blockIdx.x * (kThreads / 64) + wave;
    if (v >= V) return;   // whole wave; no workgroup barrier below
    int* L = list[wave];
    const int c0 = blockIdx.y * (64 * COLS) + lane;
    float sum[COLS];
#pragma unroll
    for (int j = 0; j < COLS; ++j) sum[j] = 0.0f;
    for (int base = 0; base < BT; base += kEbList) {
        uint32_t tok[kEbTok];
#pragma unroll
        for (int u = 0; u < kEbTok; ++u) {
            const int bt = base + 64 * u + lane;
            tok[u] = bt < BT ? tokens[bt] : 0xFFFFFFFFu;
        }
        int np = 0;
#pragma unroll
        for (int u = 0; u < kEbTok; ++u) {
            const bool hit = tok[u] == uint32_t(v);
            const uint64_t mask = __ballot(hit);
            const int rank = __builtin_amdgcn_mbcnt_hi(uint32_t(mask >> 32),
                                                       __builtin_amdgcn_mbcnt_lo(uint32_t(mask), 0));
            if (hit) L[np + rank] = base + 64 * u + lane;
            np += __popcll(mask);
        }
        // The list was written by other lanes of this wave; LDS accesses of one
        // wave complete in issue order, the fence keeps the compiler's order.
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        for (int i = 0; i < np; i += BATCH) {
            const int cnt = np - i < BATCH ? np - i : BATCH;
            const int mine = L[i + (lane < cnt ? lane : 0)];
            float r[BATCH][COLS];
#pragma unroll
            for (int b = 0; b < BATCH; ++b) {
                const int64_t row = __builtin_amdgcn_readlane(mine, b);
#pragma unroll
                for (int j = 0; j < COLS; ++j) {
                    const int c = c0 + 64 * j;
                    r[b][j] = c < C ? dx[row * C + c] : 0.0f;
                }
            }
#pragma unroll
            for (int b = 0; b < BATCH; ++b)
#pragma unroll
                for (int j = 0; j < COLS; ++j) sum[j] += b < cnt ? r[b][j] : 0.0f;
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int j = 0; j < COLS; ++j) {
        const int c = c0 + 64 * j;
        if (c < C) {
            float* dst = dwe + int64_t(v) * C + c;
            *dst = *dst + sum[j];
        }
    }
}

// ---- column sums over rows: pos_bwd and bias_grad ------------------------------
// out[r, c] = sum over s < S (increasing) of in[(s*R + r) * C + c]; one lane per
// (r, c), 16 loads issued before their adds.
__global__ __launch_bounds__(kThreads) void strided_sum_kernel(const float* __restrict__ in,
                                                               float* __restrict__ out, int64_t S,
                                                               int64_t R, int64_t C) {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= R * C) return;
    const int64_t stride = R * C;
    const float* p = in + i;
    float acc = 0.0f;
    int64_t s = 0;
    for (; s + 16 <= S; s += 16) {
        float r[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) r[u] = p[(s + u) * stride];
#pragma unroll
        for (int u = 0; u < 16; ++u) acc += r[u];
    }
    for (; s < S; ++s) acc += p[s * stride];
    out[i] = acc;
}

bool size_ok(int64_t n) { return n >= 0 && n <= dgm::kMaxIndex; }

int launch_adamw(dgm_gpu* g, float* w, const float* grad, float* m, float* v, int64_t n,
                 const AdamArgs& a) {
    if (n == 0) return DGM_OK;
    if (!w || !grad || !m || !v) return dgm::fail(g, DGM_ERR_ARG, "adamw: null buffer");
    const bool vec = dgm::aligned(w, 16) && dgm::aligned(grad, 16) && dgm::aligned(m, 16) &&
                     dgm::aligned(v, 16);
    if (vec) {
        const int64_t lanes = n / 8 > 0 ? n / 8 : 1;
        hipLaunchKernelGGL(adamw_vec_kernel, dim3(dgm::ceil_div(lanes, kThreads)), dim3(kThreads), 0,
                           g->stream, w, grad, m, v, n, a);
    } else {
        hipLaunchKernelGGL(adamw_scalar_kernel, dim3(dgm::ceil_div(n, kThreads)), dim3(kThreads), 0,
                           g->stream, w, grad, m, v, n, a);
    }
    DGM_LAUNCH_CHECK(g, "adamw");
    return DGM_OK;
}

int launch_sumsq(dgm_gpu* g, const float* x, float* out, int64_t n) {
    if (!x || !out) return dgm::fail(g, DGM_ERR_ARG, "reduce_sumsq: null buffer");
    const int64_t nb = n > 0 ? (n + kSumChunk - 1) / kSumChunk : 1;
    if (nb == 1) {
        hipLaunchKernelGGL(sumsq_partial_kernel, dim3(1), dim3(kThreads), 0, g->stream, x, n, out);
    } else {
        float* part = static_cast<float*>(dgm::workspace(g, size_t(nb) * sizeof(float)));
        if (!part) return dgm::ws_error(g);
        hipLaunchKernelGGL(sumsq_partial_kernel, dim3(unsigned(nb)), dim3(kThreads), 0, g->stream, x,
                           n, part);
        hipLaunchKernelGGL(sum_final_kernel, dim3(1), dim3(kThreads), 0, g->stream, part, nb, out);
    }
    DGM_LAUNCH_CHECK(g, "reduce_sumsq");
    return DGM_OK;
}

int launch_fill(dgm_gpu* g, const char* name, float* x, int64_t n, float s, int zero) {
    if (n == 0) return DGM_OK;
    if (!x) return dgm::fail(g, DGM_ERR_ARG, "%s: null buffer", name);
    hipLaunchKernelGGL(fill_scale_kernel, dim3(dgm::ceil_div(n, kThreads)), dim3(kThreads), 0,
                       g->stream, x, n, s, zero);
    DGM_LAUNCH_CHECK(g, name);
    return DGM_OK;
}

template <int BITS>
int launch_embed(dgm_gpu* g, const char* name, const uint32_t* tokens, const float* wte,
                 const void* q, const float* scale, const float* wpe, float* y,
                 const dgm_EmbP* p) {
    int rc = dgm::enter(g, name);
    if (rc) return rc;
    if (!p) return dgm::fail(g, DGM_ERR_ARG, "%s: null EmbP", name);
    const int64_t B = p->B, T = p->T, C = p->C, G = p->qGroup;
    const int64_t BT = B * T;
    if (BT * C == 0) return DGM_OK;
    if (BT * C > dgm::kMaxIndex) return dgm::fail(g, DGM_ERR_UNSUPPORTED, "%s: B*T*C beyond 2^31", name);
    if (BITS != 32) {
        if (G <= 0 || C % G != 0)
            return dgm::fail(g, DGM_ERR_SHAPE, "%s: C %% qGroup != 0", name);
        if (BITS == 4 && G % 2 != 0)
            return dgm::fail(g, DGM_ERR_SHAPE, "%s: quant group must be even for int4", name);
        if (!q || !scale) return dgm::fail(g, DGM_ERR_ARG, "%s: null codes or scales", name);
    } else if (!wte) {
        return dgm::fail(g, DGM_ERR_ARG, "%s: null table", name);
    }
    if (!tokens || !wpe || !y) return dgm::fail(g, DGM_ERR_ARG, "%s: null buffer", name);
    hipLaunchKernelGGL((embed_kernel<BITS>), dim3(dgm::ceil_div(BT * C, kThreads)), dim3(kThreads), 0,
                       g->stream, tokens, wte, q, scale, wpe, y, BT, int(T), int(C),
                       int(BITS == 32 ? 1 : G));
    DGM_LAUNCH_CHECK(g, name);
    return DGM_OK;
}

}  // namespace

extern "C" {

int dgm_adamw(dgm_gpu* g, float* w, const float* grad, float* m, float* v, const dgm_AdamP* p) {
    int rc = dgm::enter(g, "adamw");
    if (rc) return rc;
    if (!p) return dgm::fail(g, DGM_ERR_ARG, "adamw: null AdamP");
    const AdamArgs a{p->lr, p->b1, p->b2, p->eps, p->wd, p->invBC1, p->invBC2};
    return launch_adamw(g, w, grad, m, v, p->n, a);
}

int dgm_adam(dgm_gpu* g, float* w, const float* grad, float* m, float* v, int64_t n, float lr,
             float b1, float b2, float eps, float wd, float invBC1, float invBC2) {
    if (!g) return DGM_ERR_ARG;
    if (!size_ok(n)) return dgm::fail(g, DGM_ERR_ARG, "adam: bad count %lld", (long long)n);
    dgm_AdamP p{uint32_t(n), lr, b1, b2, eps, wd, invBC1, invBC2};
    return dgm_adamw(g, w, grad, m, v, &p);
}

int dgm_adam_quantize(dgm_gpu* g, float* w, const float* grad, float* m, float* v, void* q,
                      float* scale, int64_t rows, int64_t cols, int64_t bits, int64_t qGroup,
                      float lr, float b1, float b2, float eps, float wd, float invBC1,
                      float invBC2) {
    if (!g) return DGM_ERR_ARG;
    if (bits != 4 && bits != 8)
        return dgm::fail(g, DGM_ERR_BITS, "adam_quantize: unsupported bits %lld", (long long)bits);
    if (rows < 0 || cols < 0 || qGroup <= 0 || !size_ok(rows * cols) || qGroup > dgm::kMaxIndex)
        return dgm::fail(g, DGM_ERR_ARG, "adam_quantize: bad sizes rows=%lld cols=%lld group=%lld",
                         (long long)rows, (long long)cols, (long long)qGroup);
    const int64_t G = qGroup;
    const bool pow2 = (G & (G - 1)) == 0;
    const bool fused = cols % G == 0 && G >= 8 && G <= 512 && pow2 && rows * cols > 0 &&
                       dgm::aligned(w, 16) && dgm::aligned(grad, 16) && dgm::aligned(m, 16) &&
                       dgm::aligned(v, 16) && dgm::aligned(q, bits == 8 ? 8 : 4) && q && scale;
    if (!fused) {
        // Same results through the two reference dispatches.
        int rc = dgm_adam(g, w, grad, m, v, rows * cols, lr, b1, b2, eps, wd, invBC1, invBC2);
        if (rc) return rc;
        return dgm_quantize(g, w, q, scale, rows, cols, bits, qGroup);
    }
    int rc = dgm::enter(g, "adam_quantize");
    if (rc) return rc;
    const AdamArgs a{lr, b1, b2, eps, wd, invBC1, invBC2};
    const float qmax = bits == 4 ? 7.0f : 127.0f;
    const int lim = bits == 4 ? 7 : 127;
    const int64_t nthreads = rows * cols / 8;
    const unsigned blocks = dgm::ceil_div(nthreads, kThreads);
    switch ((bits == 4 ? 100 : 0) + int(G / 8)) {
#define DGM_AQ_CASE(BB, LL)                                                                      \
    case (BB == 4 ? 100 : 0) + LL:                                                               \
        hipLaunchKernelGGL((adam_quant_kernel<BB, LL>), dim3(blocks), dim3(kThreads), 0, g->stream, \
                           w, grad, m, v, q, scale, nthreads, a, qmax, lim);                     \
        break;
        DGM_AQ_CASE(8, 1) DGM_AQ_CASE(8, 2) DGM_AQ_CASE(8, 4) DGM_AQ_CASE(8, 8)
        DGM_AQ_CASE(8, 16) DGM_AQ_CASE(8, 32) DGM_AQ_CASE(8, 64)
        DGM_AQ_CASE(4, 1) DGM_AQ_CASE(4, 2) DGM_AQ_CASE(4, 4) DGM_AQ_CASE(4, 8)
        DGM_AQ_CASE(4, 16) DGM_AQ_CASE(4, 32) DGM_AQ_CASE(4, 64)
#undef DGM_AQ_CASE
        default: return dgm::fail(g, DGM_ERR_ARG, "adam_quantize: group %lld", (long long)G);
    }
    DGM_LAUNCH_CHECK(g, "adam_quantize");
    return DGM_OK;
}

int dgm_reduce_sumsq(dgm_gpu* g, const float* x, float* out, const dgm_ReduceP* p) {
    int rc = dgm::enter(g, "reduce_sumsq");
    if (rc) return rc;
    if (!p) return dgm::fail(g, DGM_ERR_ARG, "reduce_sumsq: null ReduceP");
    return launch_sumsq(g, x, out ? out + p->slot : nullptr, p->n);
}

int dgm_reduceSumsq(dgm_gpu* g, const float* x, float* into, int64_t n, int64_t slot) {
    if (!g) return DGM_ERR_ARG;
    if (!size_ok(n) || slot < 0 || slot > dgm::kMaxIndex)
        return dgm::fail(g, DGM_ERR_ARG, "reduceSumsq: bad n=%lld slot=%lld", (long long)n,
                         (long long)slot);
    dgm_ReduceP p{uint32_t(n), uint32_t(slot), 0, 0};
    return dgm_reduce_sumsq(g, x, into, &p);
}

int dgm_zero_f(dgm_gpu* g, float* x, const dgm_UnaryP* p) {
    int rc = dgm::enter(g, "zero_f");
    if (rc) return rc;
    if (!p) return dgm::fail(g, DGM_ERR_ARG, "zero_f: null UnaryP");
    return launch_fill(g, "zero_f", x, p->n, 0.0f, 1);
}

int dgm_scale_f(dgm_gpu* g, float* x, const dgm_ScaleP* p) {
    int rc = dgm::enter(g, "scale_f");
    if (rc) return rc;
    if (!p) return dgm::fail(g, DGM_ERR_ARG, "scale_f: null ScaleP");
    return launch_fill(g, "scale_f", x, p->n, p->s, 0);
}

int dgm_zero(dgm_gpu* g, float* x, int64_t n) {
    // src/GPU.swift:200-204: nothing is dispatched for n <= 0.
    if (!g) return DGM_ERR_ARG;
    if (n <= 0) return n < 0 ? dgm::fail(g, DGM_ERR_ARG, "zero: negative count") : DGM_OK;
    if (!size_ok(n)) return dgm::fail(g, DGM_ERR_ARG, "zero: count beyond 2^31");
    dgm_UnaryP p{uint32_t(n), 0, 0, 0};
    return dgm_zero_f(g, x, &p);
}

int dgm_scale(dgm_gpu* g, float* x, int64_t n, float s) {
    // src/GPU.swift:206-210.
    if (!g) return DGM_ERR_ARG;
    if (n <= 0) return n < 0 ? dgm::fail(g, DGM_ERR_ARG, "scale: negative count") : DGM_OK;
    if (!size_ok(n)) return dgm::fail(g, DGM_ERR_ARG, "scale: count beyond 2^31");
    dgm_ScaleP p{uint32_t(n), s, 0, 0};
    return dgm_scale_f(g, x, &p);
}

int dgm_embed_f32(dgm_gpu* g, const uint32_t* tokens, const float* wte, const float* wpe, float* y,
                  const dgm_EmbP* p) {
    return launch_embed<32>(g, "embed_f32", tokens, wte, nullptr, nullptr, wpe, y, p);
}

int dgm_embed_i8(dgm_gpu* g, const uint32_t* tokens, const int8_t* wte, const float* scale,
                 const float* wpe, float* y, const dgm_EmbP* p) {
    return launch_embed<8>(g, "embed_i8", tokens, nullptr, wte, scale, wpe, y, p);
}

int dgm_embed_i4(dgm_gpu* g, const uint32_t* tokens, const uint8_t* wte, const float* scale,
                 const float* wpe, float* y, const dgm_EmbP* p) {
    return launch_embed<4>(g, "embed_i4", tokens, nullptr, wte, scale, wpe, y, p);
}

int dgm_embed(dgm_gpu* g, int64_t bits, const uint32_t* tokens, const float* wte, const void* q,
              const float* scale, const float* wpe, float* y, int64_t B, int64_t T, int64_t C,
              int64_t qGroup) {
    if (!g) return DGM_ERR_ARG;
    if (B < 0 || T < 0 || C < 0 || !size_ok(B) || !size_ok(T) || !size_ok(C) || qGroup < 0 ||
        qGroup > dgm::kMaxIndex)
        return dgm::fail(g, DGM_ERR_ARG, "embed: bad sizes");
    dgm_EmbP p{uint32_t(B), uint32_t(T), uint32_t(C), uint32_t(qGroup)};
    switch (bits) {
        case 32: return dgm_embed_f32(g, tokens, wte, wpe, y, &p);
        case 8: return dgm_embed_i8(g, tokens, static_cast<const int8_t*>(q), scale, wpe, y, &p);
        case 4: return dgm_embed_i4(g, tokens, static_cast<const uint8_t*>(q), scale, wpe, y, &p);
        default: return dgm::fail(g, DGM_ERR_BITS, "embed: unsupported bits %lld", (long long)bits);
    }
}

int dgm_embed_bwd(dgm_gpu* g, const uint32_t* tokens, const float* dx, float* dwe,
                  const dgm_EmbBwdP* p) {
    int rc = dgm::enter(g, "embed_bwd");
    if (rc) return rc;
    if (!p) return dgm::fail(g, DGM_ERR_ARG, "embed_bwd: null EmbBwdP");
    const int64_t BT = int64_t(p->B) * p->T, C = p->C, V = p->V;
    if (C == 0 || V == 0) return DGM_OK;
    if (BT * C > dgm::kMaxIndex || V * C > dgm::kMaxIndex)
        return dgm::fail(g, DGM_ERR_UNSUPPORTED, "embed_bwd: sizes beyond 2^31");
    if (!dwe || (BT > 0 && (!tokens || !dx))) return dgm::fail(g, DGM_ERR_ARG, "embed_bwd: null buffer");
    if (C <= 128) {
        const dim3 grid(dgm::ceil_div(V, kThreads / 64), 1);
        hipLaunchKernelGGL((embed_bwd_kernel<2, 32>), grid, dim3(kThreads), 0, g->stream, tokens, dx, dwe,
                           int(BT), int(C), int(V));
    } else {
        const dim3 grid(dgm::ceil_div(V, kThreads / 64), dgm::ceil_div(C, 256));
        hipLaunchKernelGGL((embed_bwd_kernel<4, 16>), grid, dim3(kThreads), 0, g->stream, tokens, dx, dwe,
                           int(BT), int(C), int(V));
    }
    DGM_LAUNCH_CHECK(g, "embed_bwd");
    return DGM_OK;
}

int dgm_embedBwd(dgm_gpu* g, const uint32_t* tokens, const float* dx, float* dwe, int64_t B,
                 int64_t T, int64_t C, int64_t V) {
    if (!g) return DGM_ERR_ARG;
    if (!size_ok(B) || !size_ok(T) || !size_ok(C) || !size_ok(V))
        return dgm::fail(g, DGM_ERR_ARG, "embedBwd: bad sizes");
    dgm_EmbBwdP p{uint32_t(B), uint32_t(T), uint32_t(C), uint32_t(V)};
    return dgm_embed_bwd(g, tokens, dx, dwe, &p);
}

int dgm_pos_bwd(dgm_gpu* g, const float* dx, float* dwp, const dgm_PosP* p) {
    int rc = dgm::enter(g, "pos_bwd");
    if (rc) return rc;
    if (!p) return dgm::fail(g, DGM_ERR_ARG, "pos_bwd: null PosP");
    const int64_t B = p->B, T = p->T, C = p->C;
    if (T * C == 0) return DGM_OK;
    if (B * T * C > dgm::kMaxIndex) return dgm::fail(g, DGM_ERR_UNSUPPORTED, "pos_bwd: B*T*C beyond 2^31");
    if (!dwp || (B > 0 && !dx)) return dgm::fail(g, DGM_ERR_ARG, "pos_bwd: null buffer");
    hipLaunchKernelGGL(strided_sum_kernel, dim3(dgm::ceil_div(T * C, kThreads)), dim3(kThreads), 0,
                       g->stream, dx, dwp, B, T, C);
    DGM_LAUNCH_CHECK(g, "pos_bwd");
    return DGM_OK;
}

int dgm_posBwd(dgm_gpu* g, const float* dx, float* dwp, int64_t B, int64_t T, int64_t C) {
    if (!g) return DGM_ERR_ARG;
    if (!size_ok(B) || !size_ok(T) || !size_ok(C)) return dgm::fail(g, DGM_ERR_ARG, "posBwd: bad sizes");
    dgm_PosP p{uint32_t(B), uint32_t(T), uint32_t(C), 0};
    return dgm_pos_bwd(g, dx, dwp, &p);
}

int dgm_bias_grad(dgm_gpu* g, const float* dY, float* db, const dgm_BiasP* p) {
    int rc = dgm::enter(g, "bias_grad");
    if (rc) return rc;
    if (!p) return dgm::fail(g, DGM_ERR_ARG, "bias_grad: null BiasP");
    const int64_t M = p->M, N = p->N;
    if (N == 0) return DGM_OK;
    if (M * N > dgm::kMaxIndex) return dgm::fail(g, DGM_ERR_UNSUPPORTED, "bias_grad: M*N beyond 2^31");
    if (!db || (M > 0 && !dY)) return dgm::fail(g, DGM_ERR_ARG, "bias_grad: null buffer");
    hipLaunchKernelGGL(strided_sum_kernel, dim3(dgm::ceil_div(N, kThreads)), dim3(kThreads), 0,
                       g->stream, dY, db, M, int64_t(1), N);
    DGM_LAUNCH_CHECK(g, "bias_grad");
    return DGM_OK;
}

int dgm_biasGrad(dgm_gpu* g, const float* dy, float* db, int64_t M, int64_t N) {
    if (!g) return DGM_ERR_ARG;
    if (!size_ok(M) || !size_ok(N)) return dgm::fail(g, DGM_ERR_ARG, "biasGrad: bad sizes");
    dgm_BiasP p{uint32_t(M), uint32_t(N), 0, 0};
    return dgm_bias_grad(g, dy, db, &p);
}

}  // extern "C"
