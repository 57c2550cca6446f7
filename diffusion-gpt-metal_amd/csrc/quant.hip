// Per-group absmax quantization and int4 nibble packing for gfx950.
//
// Semantics (bit-exact with metal/kernels.metal:62-124 and the CPU reference
// src/Check.swift:399-431): for each row and each group of G consecutive
// columns, maxAbs = max |w|, s = max(maxAbs / qmax, 1e-8f) with a correctly
// rounded fp32 divide, code = clamp(rint(w / s), -lim, lim) with ties to even.
// int4 packs the even column in the low nibble.
//
// Design: the reference runs one thread per row and walks the groups
// serially. Here the matrix is viewed flat (cols % G == 0, so groups never
// straddle rows): each lane owns 8 consecutive weights (two 128-bit loads),
// the G/8 lanes of a group reduce maxAbs with cross-lane xor shuffles, and
// each lane writes its 8 codes with one 64-bit (int8) or 32-bit (int4) store.
// Groups that are not a power of two multiple of 8 (or G > 512), and rows
// that are not a whole number of groups, take a one-thread-per-group kernel
// with the same arithmetic.
#include "common.hpp"
#include "quant_math.hpp"

namespace {

constexpr int kThreads = 256;

using dgm::group_scale;
using dgm::quant_code;

// L = G / 8 lanes per group, L in {1, 2, 4, ..., 64}.
template <int BITS, int L>
__global__ __launch_bounds__(kThreads) void quant_vec_kernel(
    const float* __restrict__ W, void* __restrict__ Q, float* __restrict__ S,
    int64_t nthreads, float qmax, int lim) {
    const int64_t t = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    const bool valid = t < nthreads;
    const int64_t tt = valid ? t : 0;   // out-of-range lanes read element 0 (in bounds)
    const float4* src = reinterpret_cast<const float4*>(W) + 2 * tt;
    const float4 a = src[0];
    const float4 b = src[1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float x = fabsf(v[i]);
        m = x >= m ? x : m;
    }
    // A group's L lanes are consecutive and L-aligned within the wave, so the
    // xor butterfly never leaves the group. Either all of a group's lanes are
    // valid or none is (the valid count is a multiple of L).
#pragma unroll
    for (int off = L / 2; off >= 1; off >>= 1) {
        float o = __shfl_xor(m, off, 64);
        m = o >= m ? o : m;
    }
    const float s = group_scale(m, qmax);
    if (!valid) return;
    if ((t % L) == 0) S[t / L] = s;
    if constexpr (BITS == 8) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) lo |= (uint32_t(quant_code(v[i], s, lim)) & 0xFFu) << (8 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i) hi |= (uint32_t(quant_code(v[4 + i], s, lim)) & 0xFFu) << (8 * i);
        reinterpret_cast<uint2*>(Q)[t] = make_uint2(lo, hi);
    } else {
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) packed |= (uint32_t(quant_code(v[i], s, lim)) & 0xFu) << (4 * i);
        reinterpret_cast<uint32_t*>(Q)[t] = packed;
    }
}

// One thread per (row, group) for any even G (int4) or any G (int8). Rows
// need not hold a whole number of groups: like the reference, only
// floor(cols/G) groups per row are quantized, the tail columns' codes are
// left untouched and scales are strided by floor(cols/G).
template <int BITS>
__global__ __launch_bounds__(kThreads) void quant_generic_kernel(
    const float* __restrict__ W, void* __restrict__ Q, float* __restrict__ S,
    int64_t ngroups, int64_t cols, int64_t gpr, int G, float qmax, int lim) {
    const int64_t gi = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (gi >= ngroups) return;
    const int64_t row = gi / gpr;
    const int64_t base = row * cols + (gi - row * gpr) * G;
    float m = 0.0f;
    for (int i = 0; i < G; ++i) {
        float x = fabsf(W[base + i]);
        m = x >= m ? x : m;
    }
    const float s = group_scale(m, qmax);
    S[gi] = s;
    if constexpr (BITS == 8) {
        int8_t* q = static_cast<int8_t*>(Q);
        for (int i = 0; i < G; ++i) q[base + i] = static_cast<int8_t>(quant_code(W[base + i], s, lim));
    } else {
        uint8_t* q = static_cast<uint8_t*>(Q);
        for (int i = 0; i < G; i += 2) {
            int c0 = quant_code(W[base + i], s, lim);
            int c1 = quant_code(W[base + i + 1], s, lim);
            q[(base + i) >> 1] = static_cast<uint8_t>((c0 & 0xF) | ((c1 & 0xF) << 4));
        }
    }
}

template <int BITS>
int launch_quant(dgm_gpu* g, const char* name, const float* W, void* Q, float* S,
                 const dgm_QuantP* p) {
    int rc = dgm::enter(g, name);
    if (rc) return rc;
    if (!p) return dgm::fail(g, DGM_ERR_ARG, "%s: null QuantP", name);
    const int64_t rows = p->rows, cols = p->cols, G = p->qGroup;
    if (G <= 0) return dgm::fail(g, DGM_ERR_SHAPE, "%s: qGroup must be positive", name);
    // An odd int4 group would pack across groups (the reference rejects it in
    // GPTConfig.validate, src/Params.swift:171).
    if (BITS == 4 && (G % 2) != 0)
        return dgm::fail(g, DGM_ERR_SHAPE, "%s: quant group must be even for int4 packing", name);
    const int64_t total = rows * cols;
    const int64_t gpr = cols / G;   // groups per row (quant_i8: p.cols / G)
    if (total == 0 || gpr == 0) return DGM_OK;
    if (!W || !Q || !S) return dgm::fail(g, DGM_ERR_ARG, "%s: null buffer", name);
    if (!(p->qmax >= 1.0f) || p->qmax > 127.0f)
        return dgm::fail(g, DGM_ERR_ARG, "%s: qmax %g outside [1, 127]", name, double(p->qmax));
    const float qmax = p->qmax;
    const int lim = static_cast<int>(qmax);
    const int64_t ngroups = rows * gpr;

    const bool pow2 = (G & (G - 1)) == 0;
    const bool vec_ok = cols % G == 0 && G >= 8 && G <= 512 && pow2 && dgm::aligned(W, 16) &&
                        dgm::aligned(Q, BITS == 8 ? 8 : 4);
    hipStream_t st = g->stream;
    if (vec_ok) {
        const int64_t nthreads = total / 8;
        const unsigned blocks = dgm::ceil_div(nthreads, kThreads);
        switch (G / 8) {
#define DGM_Q_CASE(LL)                                                                      \
    case LL:                                                                                \
        hipLaunchKernelGGL((quant_vec_kernel<BITS, LL>), dim3(blocks), dim3(kThreads), 0, st, \
                           W, Q, S, nthreads, qmax, lim);                                   \
        break;
            DGM_Q_CASE(1) DGM_Q_CASE(2) DGM_Q_CASE(4) DGM_Q_CASE(8)
            DGM_Q_CASE(16) DGM_Q_CASE(32) DGM_Q_CASE(64)
#undef DGM_Q_CASE
            default: break;
        }
    } else {
        const unsigned blocks = dgm::ceil_div(ngroups, kThreads);
        hipLaunchKernelGGL((quant_generic_kernel<BITS>), dim3(blocks), dim3(kThreads), 0, st, W, Q,
                           S, ngroups, cols, gpr, static_cast<int>(G), qmax, lim);
    }
    DGM_LAUNCH_CHECK(g, name);
    return DGM_OK;
}

}  // namespace

extern "C" {

int dgm_quant_i8(dgm_gpu* g, const float* W, int8_t* Q, float* scale, const dgm_QuantP* p) {
    return launch_quant<8>(g, "quant_i8", W, Q, scale, p);
}

int dgm_quant_i4(dgm_gpu* g, const float* W, uint8_t* Q, float* scale, const dgm_QuantP* p) {
    return launch_quant<4>(g, "quant_i4", W, Q, scale, p);
}

int dgm_quantize(dgm_gpu* g, const float* w, void* q, float* scale, int64_t rows, int64_t cols,
                 int64_t bits, int64_t qGroup) {
    // src/GPU.swift:220-225: qmax 7 for bits 4, otherwise 127 (and the int8
    // kernel); here any bits other than 4 or 8 is rejected.
    if (!g) return DGM_ERR_ARG;
    if (bits != 4 && bits != 8) return dgm::fail(g, DGM_ERR_BITS, "quantize: unsupported bits %lld", (long long)bits);
    if (rows < 0 || cols < 0 || qGroup <= 0 || rows > dgm::kMaxIndex || cols > dgm::kMaxIndex ||
        qGroup > dgm::kMaxIndex)
        return dgm::fail(g, DGM_ERR_ARG, "quantize: bad sizes rows=%lld cols=%lld group=%lld",
                         (long long)rows, (long long)cols, (long long)qGroup);
    dgm_QuantP p;
    p.rows = uint32_t(rows);
    p.cols = uint32_t(cols);
    p.qmax = bits == 4 ? 7.0f : 127.0f;
    p.qGroup = uint32_t(qGroup);
    if (bits == 4) return dgm_quant_i4(g, w, static_cast<uint8_t*>(q), scale, &p);
    return dgm_quant_i8(g, w, static_cast<int8_t*>(q), scale, &p);
}

}  // extern "C"
