// Looped DiT block forward (src/DiT.swift:520-550) on gfx950: the block's
// non-GEMM kernels, their GPU.swift-style C entry points, and the block
// orchestrator that runs the loops with every linear on the quantized GEMMs.
//
// Kernels (semantics of metal/kernels.metal, cited per kernel):
//  * rmsnorm_fwd: one wave per row, wave-reduced sum of squares.
//  * rope_fwd, repeat_heads, add_f, mix_f, copy_f, swiglu_fwd: elementwise,
//    with fp contraction off so each product and sum rounds as in the
//    reference's separate operations.
//  * attn_fwd: scores, row softmax and P.V fused in one kernel. A workgroup
//    owns (batch, head, 16 query rows); the head's K and V rows (of the one
//    KV head when the caller repeats it, or of any head) stay in LDS, scores
//    and probabilities of the 16 rows in LDS too. It also writes the scores
//    and probabilities the reference's API returns.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "dit_rows.hpp"

namespace dgm {
int gemm_check_sizes(dgm_gpu* g, const char* name, const dgm_GemmP* p, int bits);
int gemm_f32_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X,
                 const float* bias, float* Y, const dgm_GemmP* p);
}  // namespace dgm

namespace {

constexpr int kThreads = 256;
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---- rmsnorm_fwd (metal/kernels.metal:807-825) --------------------------------
// y = x * rsqrt(mean(x^2) + eps) * w; rstd = rsqrt(mean(x^2) + eps).
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                           float* __restrict__ rstd, const float* __restrict__ w,
                                                           int rows, int cols, float eps) {
#pragma clang fp contract(off)
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + size_t(row) * cols;
    float ss = 0.0f;
    for (int c = lane; c < cols; c += 64) ss += xr[c] * xr[c];
    ss = wave_sum(ss);
    const float mean = ss / float(cols);
    const float rs = 1.0f / sqrtf(mean + eps);   // correctly rounded divide and sqrt
    if (lane == 0 && rstd) rstd[row] = rs;
    float* yr = y + size_t(row) * cols;
    for (int c = lane; c < cols; c += 64) yr[c] = (xr[c] * rs) * w[c];
}

// ---- rope_fwd (metal/kernels.metal:871-889): rotate-half, tables [T, D] ----------
__global__ __launch_bounds__(kThreads) void rope_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                        const float* __restrict__ cosv,
                                                        const float* __restrict__ sinv, int B, int T, int H,
                                                        int D) {
#pragma clang fp contract(off)
    const int64_t total = int64_t(B) * T * H * D;
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= total) return;
    const int d = int(i % D);
    const int mid = D >> 1;
    const int t = int((i / (int64_t(H) * D)) % T);
    const float rot = d < mid ? -x[i + mid] : x[i - mid];
    const float a = x[i] * cosv[t * D + d];
    const float b = rot * sinv[t * D + d];
    y[i] = a + b;
}

// ---- repeat_heads (metal/kernels.metal:980-993): [B,T,D] -> [B,T,H,D] ----------
__global__ __launch_bounds__(kThreads) void repeat_heads_kernel(const float* __restrict__ src,
                                                                float* __restrict__ dst, int B, int T, int H,
                                                                int D) {
    const int64_t total = int64_t(B) * T * H * D;
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= total) return;
    const int d = int(i % D);
    const int64_t bt = i / (int64_t(H) * D);   // b * T + t
    dst[i] = src[bt * D + d];
}

// ---- swiglu_fwd (metal/kernels.metal:911-930) ----------------------------------
using dgm_rows::silu_sigmoid;

__global__ __launch_bounds__(kThreads) void swiglu_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                          float* __restrict__ y, int64_t n) {
#pragma clang fp contract(off)
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    const float z = gate[i];
    const float a = z * silu_sigmoid(z);
    y[i] = a * up[i];
}

// ---- add_f / mix_f / copy_f (metal/kernels.metal:419-427, 951-968) --------------
__global__ __launch_bounds__(kThreads) void add_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                       float* __restrict__ y, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) y[i] = a[i] + b[i];
}

__global__ __launch_bounds__(kThreads) void mix_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                       float* __restrict__ y, int64_t n, float ca, float cb) {
#pragma clang fp contract(off)
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    const float p = ca * a[i];
    const float r = cb * b[i];
    y[i] = p + r;
}

__global__ __launch_bounds__(kThreads) void copy_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) y[i] = x[i];
}

// ---- attention (metal/kernels.metal:443-506), fused ------------------------------
// q, k, v, av: [B, T, H, D]; scores, probs: [B, H, T, T]. scale = 1/sqrt(D).
// Workgroup = (b, h, 16 query rows). K/V rows of head h in LDS.
constexpr int kQRows = 16;

__global__ __launch_bounds__(kThreads) void attn_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                        const float* __restrict__ v, float* __restrict__ scores,
                                                        float* __restrict__ probs, float* __restrict__ av, int B,
                                                        int T, int H, int D, float scale, int causal) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) float sm[];
    float* ks = sm;                    // [T][D]
    float* vs = ks + T * D;            // [T][D]
    float* qs = vs + T * D;            // [16][D]
    float* ps = qs + kQRows * D;       // [16][T]
    const int tblocks = (T + kQRows - 1) / kQRows;
    const int tb = blockIdx.x % tblocks;
    const int h = (blockIdx.x / tblocks) % H;
    const int b = blockIdx.x / (tblocks * H);
    const int t0 = tb * kQRows;
    const int nq = min(kQRows, T - t0);
    const int64_t rowstride = int64_t(H) * D;
    const float* qb = q + (int64_t(b) * T) * rowstride + int64_t(h) * D;
    const float* kb = k + (int64_t(b) * T) * rowstride + int64_t(h) * D;
    const float* vb = v + (int64_t(b) * T) * rowstride + int64_t(h) * D;
    for (int e = threadIdx.x; e < T * D; e += kThreads) {
        const int s = e / D, d = e - s * D;
        ks[e] = kb[int64_t(s) * rowstride + d];
        vs[e] = vb[int64_t(s) * rowstride + d];
    }
    for (int e = threadIdx.x; e < nq * D; e += kThreads) {
        const int t = e / D, d = e - t * D;
        qs[e] = qb[int64_t(t0 + t) * rowstride + d];
    }
    __syncthreads();
    // scores: sequential d, then * scale (attn_scores order).
    for (int e = threadIdx.x; e < nq * T; e += kThreads) {
        const int t = e / T, s = e - t * T;
        float acc = 0.0f;
        for (int d = 0; d < D; ++d) acc += qs[t * D + d] * ks[s * D + d];
        acc *= scale;
        if (causal && s > t0 + t) acc = -1.0e30f;
        ps[e] = acc;
        scores[((int64_t(b) * H + h) * T + t0 + t) * T + s] = acc;
    }
    __syncthreads();
    // softmax: one wave per row (attn_softmax's max / sum / normalize).
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int t = wave; t < nq; t += kThreads / 64) {
        float* row = ps + t * T;
        float mx = -INFINITY;
        for (int s = lane; s < T; s += 64) mx = fmaxf(mx, row[s]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        float sum = 0.0f;
        for (int s = lane; s < T; s += 64) sum += expf(row[s] - mx);
        sum = wave_sum(sum);
        const float inv = 1.0f / sum;
        for (int s = lane; s < T; s += 64) {
            const float pv = expf(row[s] - mx) * inv;
            row[s] = pv;
            probs[((int64_t(b) * H + h) * T + t0 + t) * T + s] = pv;
        }
    }
    __syncthreads();
    // av = probs . v, sequential s (attn_av order).
    for (int e = threadIdx.x; e < nq * D; e += kThreads) {
        const int t = e / D, d = e - t * D;
        float acc = 0.0f;
        for (int s = 0; s < T; ++s) acc += ps[t * T + s] * vs[s * D + d];
        av[(int64_t(b) * T + t0 + t) * rowstride + int64_t(h) * D + d] = acc;
    }
}

// ---- attention on fp32 MFMA (T % 16 == 0, D % 16 == 0) ----------------------------
// Same three stages as attn_scores / attn_softmax / attn_av
// (metal/kernels.metal:443-506), fused: a workgroup owns (b, h, 16 query
// rows). Products run on v_mfma_f32_16x16x4_f32 (fp32 operands, fp32
// accumulation); each lane reads 4 consecutive contraction indices with one
// 16-byte LDS load and the 4 MFMA steps consume them, the same permutation for
// both operands. Rows in LDS are padded to D+4 / T+4 floats so the 16 rows of an
// operand fetch hit distinct banks. Optional prologue work of the DiT loop
// body, applied while staging (each element computed exactly as the
// standalone kernels compute it):
//  * rope: rotate-half RoPE of q and k (rope_fwd, metal/kernels.metal:871-889);
//  * kv_heads == 1: the single KV head is read for every query head
//    (repeat_heads, metal/kernels.metal:980-993);
//  * vmix: v = ca * v + cb * vfirst (mix_f, metal/kernels.metal:951-959).
struct AttnArgs {
    const float *q, *k, *v, *vfirst, *cosv, *sinv;
    float *scores, *probs, *av;
    int B, T, H, D;
    int q_ld, kv_ld, vf_ld, av_ld;   // floats between consecutive token rows
    int kv_heads;                    // 1 (shared head) or H
    float scale, ca, cb;
    int causal, rope, vmix;
    // Optional saves for the training forward ([B*T, o_ld] rows, head h at
    // column h*D): q after RoPE, and k after RoPE and v after the value mix,
    // each repeated to every query head. Null = not stored.
    float *qo, *ko, *vo;
    int o_ld;
};

__global__ __launch_bounds__(kThreads) void attn_mfma_kernel(AttnArgs a) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) float sm[];
    const int T = a.T, D = a.D, H = a.H;
    const int qs_ld = D + 4, vt_ld = T + 4;
    float* qs = sm;                      // [16][D+4]
    float* ks = qs + 16 * qs_ld;         // [T][D+4]
    float* vt = ks + T * qs_ld;          // [D][T+4]  (V transposed)
    float* ps = vt + D * vt_ld;          // [16][T+4]
    const int tiles = T >> 4;
    const int tb = blockIdx.x % tiles;
    const int h = (blockIdx.x / tiles) % H;
    const int b = blockIdx.x / (tiles * H);
    const int t0 = tb * 16;
    const int hk = a.kv_heads == 1 ? 0 : h;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;

    // -- stage q (16 rows), k and v (T rows) of this (b, h) in one pass of
    // 16-byte loads, all issued before any is used (D % 16 == 0, rows 16-byte
    // aligned). q and k are handled as chunk pairs (d .. d+3, d+D/2 .. d+D/2+3)
    // so RoPE is applied in registers: each element from the unrotated pair
    // and the table entries at its own index, as rope_fwd computes it.
    const int cpr = D >> 2;                        // float4 chunks per row
    const int hc = cpr >> 1, half = D >> 1;        // chunk pairs per row
    const int np = (16 + T) * hc;                  // pairs: 16 q rows first, then T k rows
    const int nv = T * cpr;                        // v chunks
    constexpr int PB = 2, VB = 3;                  // pairs / v chunks per thread per batch
    for (int bp = 0, bv = 0; bp < np || bv < nv; bp += PB * kThreads, bv += VB * kThreads) {
        float4 x1[PB], x2[PB], c1[PB], c2[PB], s1[PB], s2[PB], vv[VB], fv[VB];
#pragma unroll
        for (int u = 0; u < PB; ++u) {
            const int e = min(bp + u * kThreads + int(threadIdx.x), np - 1);
            const int row = e / hc, c = e - row * hc;
            const int t = row < 16 ? t0 + row : row - 16;
            const float* src = row < 16 ? a.q + size_t(b * T + t) * a.q_ld + h * D
                                        : a.k + size_t(b * T + t) * a.kv_ld + hk * D;
            x1[u] = *reinterpret_cast<const float4*>(src + 4 * c);
            x2[u] = *reinterpret_cast<const float4*>(src + 4 * c + half);
            if (a.rope) {
                c1[u] = *reinterpret_cast<const float4*>(a.cosv + t * D + 4 * c);
                c2[u] = *reinterpret_cast<const float4*>(a.cosv + t * D + 4 * c + half);
                s1[u] = *reinterpret_cast<const float4*>(a.sinv + t * D + 4 * c);
                s2[u] = *reinterpret_cast<const float4*>(a.sinv + t * D + 4 * c + half);
            }
        }
#pragma unroll
        for (int u = 0; u < VB; ++u) {
            const int e = min(bv + u * kThreads + int(threadIdx.x), nv - 1);
            const int t = e / cpr, c = e - t * cpr;
            const size_t r = size_t(b * T + t);
            vv[u] = *reinterpret_cast<const float4*>(a.v + r * a.kv_ld + hk * D + 4 * c);
            if (a.vmix) fv[u] = *reinterpret_cast<const float4*>(a.vfirst + r * a.vf_ld + 4 * c);
        }
#pragma unroll
        for (int u = 0; u < PB; ++u) {
            const int e = bp + u * kThreads + int(threadIdx.x);
            if (e >= np) break;
            const int row = e / hc, c = e - row * hc;
            float* dst = row < 16 ? qs + row * qs_ld : ks + (row - 16) * qs_ld;
            float4 y1 = x1[u], y2 = x2[u];
            if (a.rope) {
                const float xa[4] = {x1[u].x, x1[u].y, x1[u].z, x1[u].w};
                const float xb[4] = {x2[u].x, x2[u].y, x2[u].z, x2[u].w};
                const float ca4[4] = {c1[u].x, c1[u].y, c1[u].z, c1[u].w};
                const float cb4[4] = {c2[u].x, c2[u].y, c2[u].z, c2[u].w};
                const float sa4[4] = {s1[u].x, s1[u].y, s1[u].z, s1[u].w};
                const float sb4[4] = {s2[u].x, s2[u].y, s2[u].z, s2[u].w};
                float ya[4], yb[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p1 = xa[i] * ca4[i], r1 = -xb[i] * sa4[i];   // d < D/2: rot = -x[d + D/2]
                    const float p2 = xb[i] * cb4[i], r2 = xa[i] * sb4[i];    // d >= D/2: rot = x[d - D/2]
                    ya[i] = p1 + r1;
                    yb[i] = p2 + r2;
                }
                y1 = make_float4(ya[0], ya[1], ya[2], ya[3]);
                y2 = make_float4(yb[0], yb[1], yb[2], yb[3]);
            }
            *reinterpret_cast<float4*>(dst + 4 * c) = y1;
            *reinterpret_cast<float4*>(dst + 4 * c + half) = y2;
        }
#pragma unroll
        for (int u = 0; u < VB; ++u) {
            const int e = bv + u * kThreads + int(threadIdx.x);
            if (e >= nv) break;
            const int t = e / cpr, c = e - t * cpr;
            float v4[4] = {vv[u].x, vv[u].y, vv[u].z, vv[u].w};
            if (a.vmix) {
                const float f4[4] = {fv[u].x, fv[u].y, fv[u].z, fv[u].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = a.ca * v4[i];
                    const float r = a.cb * f4[i];
                    v4[i] = p + r;
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) vt[(4 * c + i) * vt_ld + t] = v4[i];
        }
    }
    __syncthreads();

    // -- training saves: this workgroup's 16 query rows of q, and the same 16
    // token rows of k and v for head h (all workgroups of (b, h) cover T).
    if (a.qo) {
        for (int e = threadIdx.x; e < 16 * D; e += kThreads) {
            const int r = e / D, d = e - r * D;
            const size_t o = size_t(b * T + t0 + r) * a.o_ld + h * D + d;
            a.qo[o] = qs[r * qs_ld + d];
            a.ko[o] = ks[(t0 + r) * qs_ld + d];
            a.vo[o] = vt[d * vt_ld + t0 + r];
        }
    }

    // -- scores: wave w takes key tiles w, w+4, ...
    const size_t srow0 = (size_t(b) * H + h) * T + t0;   // row index into [B,H,T,T]
    for (int kt = wave; kt < tiles; kt += 4) {
        f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const float* qa = qs + r16 * qs_ld + 4 * q4;
        const float* kb = ks + (kt * 16 + r16) * qs_ld + 4 * q4;
        for (int d0 = 0; d0 < D; d0 += 16) {
            const float4 x = *reinterpret_cast<const float4*>(qa + d0);
            const float4 y = *reinterpret_cast<const float4*>(kb + d0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, y.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, y.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, y.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, y.w, acc, 0, 0, 0);
        }
        // acc[r]: query row 4*q4 + r, key kt*16 + r16.
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 4 * q4 + r, s2 = kt * 16 + r16;
            float v = acc[r] * a.scale;
            if (a.causal && s2 > t0 + t) v = -1.0e30f;
            ps[t * vt_ld + s2] = v;
        }
    }
    __syncthreads();

    // -- row softmax (max, sum of exp, normalize as attn_softmax does): wave w
    // takes rows 4w .. 4w+3 at once, 16 lanes per row, each lane T/16 keys.
    {
        const int t = 4 * wave + q4;
        float* row = ps + t * vt_ld;
        float* so = a.scores + (srow0 + t) * T;
        float* po = a.probs + (srow0 + t) * T;
        float mx = -INFINITY;
        for (int s2 = r16; s2 < T; s2 += 16) {
            const float v = row[s2];
            so[s2] = v;
            mx = fmaxf(mx, v);
        }
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 16));
        float sum = 0.0f;
        for (int s2 = r16; s2 < T; s2 += 16) sum += expf(row[s2] - mx);
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 16);
        const float inv = 1.0f / sum;
        for (int s2 = r16; s2 < T; s2 += 16) {
            const float pv = expf(row[s2] - mx) * inv;
            row[s2] = pv;
            po[s2] = pv;
        }
    }
    __syncthreads();

    // -- av = probs . v: wave w takes d tiles w, w+4, ...
    for (int dt = wave; dt < (D >> 4); dt += 4) {
        f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const float* pa = ps + r16 * vt_ld + 4 * q4;
        const float* vb = vt + (dt * 16 + r16) * vt_ld + 4 * q4;
        for (int s0 = 0; s0 < T; s0 += 16) {
            const float4 x = *reinterpret_cast<const float4*>(pa + s0);
            const float4 y = *reinterpret_cast<const float4*>(vb + s0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, y.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, y.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, y.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, y.w, acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + 4 * q4 + r;
            a.av[size_t(b * T + t) * a.av_ld + h * D + dt * 16 + r16] = acc[r];
        }
    }
}

size_t attn_mfma_lds_bytes(int T, int D) {
    return sizeof(float) * (size_t(16 + T) * (D + 4) + size_t(D + 16) * (T + 4));
}

bool attn_mfma_ok(int T, int D) {
    return T > 0 && D > 0 && T % 16 == 0 && D % 16 == 0 && attn_mfma_lds_bytes(T, D) <= 160 * 1024;
}

int launch_attn_mfma(dgm_gpu* g, const AttnArgs& a) {
    const size_t lds = attn_mfma_lds_bytes(a.T, a.D);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_mfma_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess)
            return dgm::fail(g, DGM_ERR_HIP, "attn_fwd: cannot reserve %zu bytes of LDS: %s", lds,
                             hipGetErrorString(e));
    }
    hipLaunchKernelGGL(attn_mfma_kernel, dim3(unsigned(a.B * a.H * (a.T / 16))), dim3(kThreads), lds, g->stream, a);
    return dgm::check_launch(g, "attn_fwd");
}

inline unsigned blocks_for(int64_t n) { return unsigned((n + kThreads - 1) / kThreads); }

size_t attn_lds_bytes(int T, int D) {
    return sizeof(float) * (size_t(2) * T * D + size_t(kQRows) * D + size_t(kQRows) * T);
}

// Launchers shared by the C entry points and the block orchestrator. They
// validate only what the kernels index; the entry points add the reference's
// argument checks.
int launch_rms(dgm_gpu* g, const float* x, float* y, float* rstd, const float* w, int64_t rows, int64_t cols,
               float eps) {
    if (rows == 0 || cols == 0) return DGM_OK;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(unsigned((rows + 3) / 4)), dim3(kThreads), 0, g->stream, x, y, rstd,
                       w, int(rows), int(cols), eps);
    return dgm::check_launch(g, "rmsnorm_fwd");
}

int launch_rope(dgm_gpu* g, const float* x, float* y, const float* c, const float* s, int B, int T, int H, int D) {
    const int64_t n = int64_t(B) * T * H * D;
    if (n == 0) return DGM_OK;
    hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, x, y, c, s, B, T, H, D);
    return dgm::check_launch(g, "rope_fwd");
}

int launch_repeat(dgm_gpu* g, const float* src, float* dst, int B, int T, int H, int D) {
    const int64_t n = int64_t(B) * T * H * D;
    if (n == 0) return DGM_OK;
    hipLaunchKernelGGL(repeat_heads_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, src, dst, B, T, H,
                       D);
    return dgm::check_launch(g, "repeat_heads");
}

int launch_attn(dgm_gpu* g, const float* q, const float* k, const float* v, float* scores, float* probs,
                float* av, int B, int T, int H, int D, int causal) {
    if (int64_t(B) * T * H * D == 0) return DGM_OK;
    if (attn_mfma_ok(T, D)) {
        AttnArgs a{};
        a.q = q; a.k = k; a.v = v; a.scores = scores; a.probs = probs; a.av = av;
        a.B = B; a.T = T; a.H = H; a.D = D;
        a.q_ld = a.kv_ld = a.av_ld = H * D;
        a.kv_heads = H;
        a.scale = 1.0f / sqrtf(float(D));
        a.causal = causal;
        return launch_attn_mfma(g, a);
    }
    const size_t lds = attn_lds_bytes(T, D);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess)
            return dgm::fail(g, DGM_ERR_HIP, "attn_fwd: cannot reserve %zu bytes of LDS: %s", lds,
                             hipGetErrorString(e));
    }
    const int tblocks = (T + kQRows - 1) / kQRows;
    const float scale = 1.0f / sqrtf(float(D));
    hipLaunchKernelGGL(attn_kernel, dim3(unsigned(B * H * tblocks)), dim3(kThreads), lds, g->stream, q, k, v,
                       scores, probs, av, B, T, H, D, scale, causal);
    return dgm::check_launch(g, "attn_fwd");
}

int launch_swiglu(dgm_gpu* g, const float* gate, const float* up, float* y, int64_t n) {
    if (n == 0) return DGM_OK;
    hipLaunchKernelGGL(swiglu_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, gate, up, y, n);
    return dgm::check_launch(g, "swiglu_fwd");
}

int launch_add(dgm_gpu* g, const float* a, const float* b, float* y, int64_t n) {
    if (n == 0) return DGM_OK;
    hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, a, b, y, n);
    return dgm::check_launch(g, "add_f");
}

int launch_mix(dgm_gpu* g, const float* a, const float* b, float* y, int64_t n, float ca, float cb) {
    if (n == 0) return DGM_OK;
    hipLaunchKernelGGL(mix_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, a, b, y, n, ca, cb);
    return dgm::check_launch(g, "mix_f");
}

int launch_copy(dgm_gpu* g, const float* x, float* y, int64_t n) {
    if (n == 0) return DGM_OK;
    hipLaunchKernelGGL(copy_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, x, y, n);
    return dgm::check_launch(g, "copy_f");
}

bool bad_count(int64_t n) { return n < 0 || n > (int64_t(1) << 40); }

int check_bthd(dgm_gpu* g, const char* name, int64_t B, int64_t T, int64_t H, int64_t D) {
    if (B < 0 || T < 0 || H < 0 || D < 0 || B > dgm::kMaxIndex || T > dgm::kMaxIndex || H > dgm::kMaxIndex ||
        D > dgm::kMaxIndex || B * T * H * D > (int64_t(1) << 40))
        return dgm::fail(g, DGM_ERR_ARG, "%s: bad sizes B=%lld T=%lld H=%lld D=%lld", name, (long long)B,
                         (long long)T, (long long)H, (long long)D);
    return DGM_OK;
}

// ---- fused row kernels of the loop body ----------------------------------------------
// One wave per row; every RMSNorm reduces its sum of squares in exactly the
// lane order rmsnorm_kernel uses, and every add/product rounds as the
// standalone kernels do, so the fused results equal running rmsFwd, add,
// rmsFwd (, rmsFwd) in sequence, bit for bit.
//   mid  = res + rms(a) * w1          (rmsnorm_fwd + add_f)
//   out2 = rms(mid) * w2              (rmsnorm_fwd)
//   out3 = rms(out2) * w3             (rmsnorm_fwd; when w3 != nullptr)
constexpr int kRowMax = 16;   // columns per lane: cols <= 1024

__device__ __forceinline__ float row_rstd(const float (&v)[kRowMax], int lane, int cols, float eps) {
#pragma clang fp contract(off)
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kRowMax; ++u)
        if (lane + 64 * u < cols) ss += v[u] * v[u];
    ss = wave_sum(ss);
    const float mean = ss / float(cols);
    return 1.0f / sqrtf(mean + eps);
}

__global__ __launch_bounds__(kThreads) void row_fuse_kernel(const float* __restrict__ a, const float* __restrict__ res,
                                                            float* __restrict__ mid, float* __restrict__ out2,
                                                            float* __restrict__ out3, const float* __restrict__ w1,
                                                            const float* __restrict__ w2, const float* __restrict__ w3,
                                                            float* __restrict__ rstd, float* __restrict__ rstd1,
                                                            int rows, int cols, float eps) {
#pragma clang fp contract(off)
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const size_t base = size_t(row) * cols;
    float v[kRowMax];
#pragma unroll
    for (int u = 0; u < kRowMax; ++u) v[u] = lane + 64 * u < cols ? a[base + lane + 64 * u] : 0.0f;
    float rs = row_rstd(v, lane, cols, eps);
    if (lane == 0 && rstd1) rstd1[row] = rs;
#pragma unroll
    for (int u = 0; u < kRowMax; ++u) {
        const int c = lane + 64 * u;
        if (c < cols) {
            const float t1 = (v[u] * rs) * w1[c];
            v[u] = res[base + c] + t1;
            if (mid) mid[base + c] = v[u];
        }
    }
    rs = row_rstd(v, lane, cols, eps);
#pragma unroll
    for (int u = 0; u < kRowMax; ++u) {
        const int c = lane + 64 * u;
        if (c < cols) {
            v[u] = (v[u] * rs) * w2[c];
            out2[base + c] = v[u];
        }
    }
    if (w3) {
        rs = row_rstd(v, lane, cols, eps);
#pragma unroll
        for (int u = 0; u < kRowMax; ++u) {
            const int c = lane + 64 * u;
            if (c < cols) out3[base + c] = (v[u] * rs) * w3[c];
        }
    }
    if (lane == 0 && rstd) rstd[row] = rs;
}

// swiglu_fwd over row-strided gate / up (the halves of a fused [gate; up]
// projection, or two separate buffers): y[m, j] = gate * sigmoid(gate) * up.
__global__ __launch_bounds__(kThreads) void swiglu_rows_kernel(const float* __restrict__ gate,
                                                               const float* __restrict__ up, float* __restrict__ y,
                                                               int rows, int F, int ldg, int ldu) {
#pragma clang fp contract(off)
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= int64_t(rows) * F) return;
    const int m = int(i / F), j = int(i - int64_t(m) * F);
    const float z = gate[size_t(m) * ldg + j];
    const float act = z * silu_sigmoid(z);
    y[i] = act * up[size_t(m) * ldu + j];
}

// ---- projection GEMM with the loop body's row chains fused in -------------------------
// Y = X W^T over the group-quantized (or fp32) weights, for K = C (the rows of
// the residual stream), where X is produced in the prologue from whole rows:
//   pro 1: X = rms(a) * w1                                    (ln1 of loop 0)
//   pro 2: mid = res + rms(a) * w1 -> side;  X = rms(mid) * w2  (ln2)
//   pro 3: pre = res + rms(a) * w1;  x = rms(pre) * w2 -> side;  X = rms(x) * w3
//          (the end of one loop and ln1 of the next)
// A workgroup owns 16 rows; each of its 4 waves normalizes 4 of them (16 lanes
// per row, each RMSNorm exactly rmsnorm_fwd's formula with a 16-lane
// reduction), writes its rows into the LDS X block, and the column-tile-0
// workgroup stores the side output. The GEMM part is the LDS-staged forward
// (one contraction part per wave, 16-k weight runs per lane).
// PAIR: the weight holds [gate; up] (F rows each); waves 0-1 compute gate and
// waves 2-3 up for the same 32 columns, and the epilogue stores
// swiglu = gate * sigmoid(gate) * up (swiglu_fwd) instead of the projections.
struct DitGemmArgs {
    const float *a, *res, *w1, *w2, *w3;
    float* side;
    const void* W;
    const float* S;
    float* out;
    int M, N, K, G, groups, F;
    float eps;
    int pro;
    // Optional saves for the training forward (stored by the workgroups of
    // column tile 0; null = not stored): the normalized rows fed to the GEMM,
    // pro 3's first-stage rows (pre), each stage's rstd per row, and with
    // PAIR the gate and up projections before SwiGLU ([M, F] each).
    float *lnout, *side1, *rs1, *rs2, *rs3, *gate_out, *up_out;
};

using dgm_rows::add4;
using dgm_rows::norm4;
using dgm_rows::rstd16;

template <int BITS, bool PAIR, int J>
__global__ __launch_bounds__(kThreads) void dit_gemm_kernel(DitGemmArgs a, int tiles_i, int tiles_j, int per_xcd) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) float4 xs4[];   // [16][K/4] slots, swizzled
    const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (t >= tiles_i * tiles_j) return;
    const int ti = t / tiles_j, tj = t - ti * tiles_j;
    constexpr int TN = PAIR ? 32 : 64;
    const int i0 = ti * 16, j0 = tj * TN;
    const int K = a.K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;
    // K == 64 * J: J stages of 64 contraction indices.
    // -- weight row of this lane's column, all stages, issued first.
    int n;
    if constexpr (PAIR) n = (wave & 1) * 16 + r16 + j0, n = min(n, a.F - 1) + (wave >= 2 ? a.F : 0);
    else n = min(j0 + wave * 16 + r16, a.N - 1);
    uint32_t wc[J][BITS == 4 ? 2 : 4];
    float4 wf[J][BITS == 32 ? 4 : 1];
    float sc[J];
#pragma unroll
    for (int u = 0; u < J; ++u) {
        const int k = u * 64 + 16 * q4;
        if constexpr (BITS == 32) {
            const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.W) + size_t(n) * K + k);
#pragma unroll
            for (int e = 0; e < 4; ++e) wf[u][e] = p[e];
        } else if constexpr (BITS == 8) {
            const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(a.W) + size_t(n) * K + k);
            wc[u][0] = v.x; wc[u][1] = v.y; wc[u][2] = v.z; wc[u][3] = v.w;
            sc[u] = a.S[size_t(n) * a.groups + k / a.G];
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(a.W) + ((size_t(n) * K + k) >> 1));
            wc[u][0] = v.x; wc[u][1] = v.y;
            sc[u] = a.S[size_t(n) * a.groups + k / a.G];
        }
    }

    // -- prologue: rows 4*wave + q4, lane r16 holds chunks r16 + 16 j (J = K / 64).
    {
        const int row = 4 * wave + q4;
        const int gi = i0 + row;
        const size_t base = size_t(min(gi, a.M - 1)) * K;
        float4 v[J], rr[J], w1[J], w2[J], w3[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int c = 4 * (r16 + 16 * j);
            v[j] = *reinterpret_cast<const float4*>(a.a + base + c);
            w1[j] = *reinterpret_cast<const float4*>(a.w1 + c);
            if (a.pro >= 2) {
                rr[j] = *reinterpret_cast<const float4*>(a.res + base + c);
                w2[j] = *reinterpret_cast<const float4*>(a.w2 + c);
            }
            if (a.pro == 3) w3[j] = *reinterpret_cast<const float4*>(a.w3 + c);
        }
        const bool saver = tj == 0 && gi < a.M;   // this row's saves
        auto save_rows = [&](float* dst) {
#pragma unroll
            for (int j = 0; j < J; ++j) *reinterpret_cast<float4*>(dst + base + 4 * (r16 + 16 * j)) = v[j];
        };
        if (a.pro == 1 && a.side && saver) save_rows(a.side);   // the input rows
        float rs = rstd16<J>(v, K, a.eps);
        if (a.rs1 && saver && r16 == 0) a.rs1[gi] = rs;
#pragma unroll
        for (int j = 0; j < J; ++j) v[j] = norm4(v[j], rs, w1[j]);
        if (a.pro >= 2) {
#pragma unroll
            for (int j = 0; j < J; ++j) v[j] = add4(rr[j], v[j]);
            if (a.pro == 2 && saver) save_rows(a.side);
            if (a.pro == 3 && a.side1 && saver) save_rows(a.side1);
            rs = rstd16<J>(v, K, a.eps);
            if (a.rs2 && saver && r16 == 0) a.rs2[gi] = rs;
#pragma unroll
            for (int j = 0; j < J; ++j) v[j] = norm4(v[j], rs, w2[j]);
            if (a.pro == 3) {
                if (saver) save_rows(a.side);
                rs = rstd16<J>(v, K, a.eps);
                if (a.rs3 && saver && r16 == 0) a.rs3[gi] = rs;
#pragma unroll
                for (int j = 0; j < J; ++j) v[j] = norm4(v[j], rs, w3[j]);
            }
        }
        if (a.lnout && saver) save_rows(a.lnout);
        const int spr = K >> 2;
#pragma unroll
        for (int j = 0; j < J; ++j) xs4[row * spr + ((r16 + 16 * j) ^ (row & 15))] = v[j];
    }
    __syncthreads();

    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int spr = K >> 2;
    const float4* xrow = xs4 + r16 * spr;
#pragma unroll
    for (int u = 0; u < J; ++u) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 xv = xrow[(u * 16 + 4 * q4 + c) ^ r16];
            float bv[4];
            if constexpr (BITS == 32) {
                const float4 w = wf[u][c];
                bv[0] = w.x; bv[1] = w.y; bv[2] = w.z; bv[3] = w.w;
            } else if constexpr (BITS == 8) {
                const uint32_t w = wc[u][c];
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) bv[s2] = float(int(int8_t((w >> (8 * s2)) & 0xFF))) * sc[u];
            } else {
                const uint32_t w = wc[u][c >> 1] >> (16 * (c & 1));
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) {
                    const int nib = int((w >> (4 * s2)) & 0xF);
                    bv[s2] = float(nib >= 8 ? nib - 16 : nib) * sc[u];
                }
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.x, bv[0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.y, bv[1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.z, bv[2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.w, bv[3], acc, 0, 0, 0);
        }
    }

    // acc[r]: row 4*q4 + r, column r16 of this wave's 16.
    if constexpr (!PAIR) {
        const int j = j0 + wave * 16 + r16;
        if (j < a.N) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = i0 + 4 * q4 + r;
                if (i < a.M) a.out[size_t(i) * a.N + j] = acc[r];
            }
        }
    } else {
        __syncthreads();   // X no longer read: reuse LDS for the up half
        float* up = reinterpret_cast<float*>(xs4);   // [16][32]
        if (wave >= 2) {
#pragma unroll
            for (int r = 0; r < 4; ++r) up[(4 * q4 + r) * 32 + (wave - 2) * 16 + r16] = acc[r];
        }
        float* proj = wave < 2 ? a.gate_out : a.up_out;
        if (proj) {
            const int j = j0 + (wave & 1) * 16 + r16;
            if (j < a.F) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int i = i0 + 4 * q4 + r;
                    if (i < a.M) proj[size_t(i) * a.F + j] = acc[r];
                }
            }
        }
        __syncthreads();
        if (wave < 2) {
            const int j = j0 + wave * 16 + r16;
            if (j < a.F) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int i = i0 + 4 * q4 + r;
                    if (i < a.M) {
                        const float z = acc[r];
                        const float act = z * silu_sigmoid(z);
                        a.out[size_t(i) * a.F + j] = act * up[(4 * q4 + r) * 32 + wave * 16 + r16];
                    }
                }
            }
        }
    }
}

template <int BITS, bool PAIR, int J>
void launch_dit_gemm_j(const DitGemmArgs& a, hipStream_t st) {
    constexpr int TN = PAIR ? 32 : 64;
    const int ti = int(dgm::ceil_div(a.M, 16)), tj = int(dgm::ceil_div(PAIR ? a.F : a.N, TN));
    const int64_t nt = int64_t(ti) * tj;
    const int per = int((nt + 7) / 8);
    hipLaunchKernelGGL((dit_gemm_kernel<BITS, PAIR, J>), dim3(unsigned(per) * 8u), dim3(kThreads),
                       size_t(16) * a.K * sizeof(float), st, a, ti, tj, per);
}

template <int BITS, bool PAIR>
int launch_dit_gemm_b(dgm_gpu* g, const DitGemmArgs& a) {
    switch (a.K / 64) {
        case 1: launch_dit_gemm_j<BITS, PAIR, 1>(a, g->stream); break;
        case 2: launch_dit_gemm_j<BITS, PAIR, 2>(a, g->stream); break;
        case 3: launch_dit_gemm_j<BITS, PAIR, 3>(a, g->stream); break;
        case 4: launch_dit_gemm_j<BITS, PAIR, 4>(a, g->stream); break;
        case 6: launch_dit_gemm_j<BITS, PAIR, 6>(a, g->stream); break;
        case 8: launch_dit_gemm_j<BITS, PAIR, 8>(a, g->stream); break;
        default: return dgm::fail(g, DGM_ERR_UNSUPPORTED, "dit_forward: fused projection needs C in {64,...,512}");
    }
    return dgm::check_launch(g, "dit_forward fused gemm");
}

int launch_dit_gemm(dgm_gpu* g, int bits, bool pair, const DitGemmArgs& a) {
    if (bits == 8) return pair ? launch_dit_gemm_b<8, true>(g, a) : launch_dit_gemm_b<8, false>(g, a);
    if (bits == 4) return pair ? launch_dit_gemm_b<4, true>(g, a) : launch_dit_gemm_b<4, false>(g, a);
    return pair ? launch_dit_gemm_b<32, true>(g, a) : launch_dit_gemm_b<32, false>(g, a);
}

// The fused path's conditions: C a multiple of 64 with C / 64 in {1,2,3,4,6,8},
// groups holding a 16-wide run, weights aligned for 8- / 16-byte loads.
bool dit_fused_ok(const dgm_dit_cfg* c, const dgm_dit_weights* w) {
    const int jb = c->C / 64;
    if (c->C % 64 != 0 || !(jb == 1 || jb == 2 || jb == 3 || jb == 4 || jb == 6 || jb == 8)) return false;
    if (c->bits == 32) return dgm::aligned(w->wq.w, 16) && dgm::aligned(w->wgate.w, 16);
    if (c->group % 16 != 0) return false;
    const size_t al = c->bits == 8 ? 16 : 8;
    return dgm::aligned(w->wq.q, al) && dgm::aligned(w->wgate.q, al) && dgm::aligned(w->n1, 16) &&
           dgm::aligned(w->n1b, 16) && dgm::aligned(w->n2, 16) && dgm::aligned(w->n2b, 16) &&
           dgm::aligned(w->nf, 16);
}

// ---- the block orchestrator (src/DiT.swift:520-550) ---------------------------------
// Workspace (floats, each piece 256-byte aligned):
//   ln1 [M,C] | qkv0 [M,C+2D] | qkv1 [M,C+2D] | scores [B,H,T,T] | probs [B,H,T,T]
//   | av [M,C] | attn [M,C] | mid [M,C] | ln2 [M,C] | gu [M,2F] | sw [M,F] | mlp [M,C]
//   | pre [M,C] | rstd [M]
// qkv0 holds loop 0's projections (its v columns are the value-residual
// source of later loops); later loops use qkv1.
enum Buf { LN1, QKV0, QKV1, SCORES, PROBS, AV, ATTN, MID, LN2, GU, SW, MLP, PRE, RSTD, NBUF };

void dit_sizes(const dgm_dit_cfg* c, int64_t* sz) {
    const int64_t M = int64_t(c->B) * c->T, C = c->C, F = c->F, KV = c->D;
    const int64_t att = int64_t(c->B) * c->H * c->T * c->T;
    const int64_t s[NBUF] = {M * C, M * (C + 2 * KV), M * (C + 2 * KV), att, att, M * C, M * C, M * C, M * C,
                             M * 2 * F, M * F, M * C, M * C, M};
    for (int i = 0; i < NBUF; ++i) sz[i] = s[i];
}

int64_t dit_workspace_floats(const dgm_dit_cfg* c) {
    int64_t sz[NBUF], total = 0;
    dit_sizes(c, sz);
    for (int i = 0; i < NBUF; ++i) total += (sz[i] + 63) & ~int64_t(63);   // 256-byte aligned pieces
    return total;
}

int launch_row_fuse(dgm_gpu* g, const float* a, const float* res, float* mid, float* out2, float* out3,
                    const float* w1, const float* w2, const float* w3, float* rstd, int64_t rows, int64_t cols,
                    float eps, float* rstd1 = nullptr) {
    if (rows == 0 || cols == 0) return DGM_OK;
    hipLaunchKernelGGL(row_fuse_kernel, dim3(unsigned((rows + 3) / 4)), dim3(kThreads), 0, g->stream, a, res, mid,
                       out2, out3, w1, w2, w3, rstd, rstd1, int(rows), int(cols), eps);
    return dgm::check_launch(g, "dit_forward row_fuse");
}

int launch_swiglu_rows(dgm_gpu* g, const float* gate, const float* up, float* y, int64_t rows, int64_t F,
                       int64_t ldg, int64_t ldu) {
    const int64_t n = rows * F;
    if (n == 0) return DGM_OK;
    hipLaunchKernelGGL(swiglu_rows_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, gate, up, y, int(rows),
                       int(F), int(ldg), int(ldu));
    return dgm::check_launch(g, "dit_forward swiglu");
}

// Byte offset between two linears' codes / scales when laid out back to back.
bool follows(const dgm_dit_linear& first, const dgm_dit_linear& next, int64_t rows, int64_t K, int bits, int G) {
    if (bits == 32) return next.w == first.w + rows * K;
    const int64_t code_bytes = bits == 4 ? rows * K / 2 : rows * K;
    return static_cast<const uint8_t*>(next.q) == static_cast<const uint8_t*>(first.q) + code_bytes &&
           next.scale == first.scale + rows * (K / G);
}

}  // namespace

namespace dgm {

bool dit_linear_follows(const dgm_dit_linear& first, const dgm_dit_linear& next, int64_t rows, int64_t K, int bits,
                        int G) {
    return follows(first, next, rows, K, bits, G);
}

// Scratch of the fused training forward: loop 0's and the current loop's
// [q | k | v] rows and the scores the attention kernel writes.
int64_t dit_train_scratch_floats(const dgm_dit_cfg* c) {
    const int64_t M = int64_t(c->B) * c->T, QKV = c->C + 2 * int64_t(c->D);
    return 2 * ((M * QKV + 63) & ~int64_t(63)) + int64_t(c->B) * c->H * c->T * c->T;
}

int dit_forward_train_fused(dgm_gpu* g, const dgm_dit_cfg* c, const dgm_dit_weights* w, const float* cosv,
                            const float* sinv, float* x, const DitSaves* saves, float* scratch,
                            int64_t scratch_floats) {
    const int B = c->B, T = c->T, H = c->H, D = c->D, bits = c->bits, G = c->group;
    const int64_t M = int64_t(B) * T, C = c->C, F = c->F, KV = D, QKV = C + 2 * KV;
    if (!follows(w->wq, w->wk, C, C, bits, G) || !follows(w->wk, w->wv, KV, C, bits, G) ||
        !follows(w->wgate, w->wup, F, C, bits, G) || !dit_fused_ok(c, w) || !attn_mfma_ok(T, D) ||
        c->C > 64 * kRowMax || scratch_floats < dit_train_scratch_floats(c) || !aligned(x, 16) ||
        !aligned(scratch, 16) || !aligned(cosv, 16) || !aligned(sinv, 16))
        return kNotFused;
    for (int l = 0; l < c->loops; ++l) {
        const DitSaves& S = saves[l];
        for (const float* p : {S.x, S.ln1, S.attn, S.mid, S.ln2, S.mlp, S.pre, S.q, S.k, S.v, S.av})
            if (!aligned(p, 16)) return kNotFused;
    }
    float* qkv0 = scratch;
    float* qkv1 = qkv0 + ((M * QKV + 63) & ~int64_t(63));
    float* scores = qkv1 + ((M * QKV + 63) & ~int64_t(63));
#define DGM_TRY(expr)                \
    do {                             \
        int _r = (expr);             \
        if (_r != DGM_OK) return _r; \
    } while (0)
    auto pgemm = [&](const dgm_dit_linear& L, bool pair, int pro, const float* a_in, const float* res,
                     const float* n_a, const float* n_b, const float* n_c, float* side, float* out, int64_t N,
                     DitGemmArgs d) -> int {
        d.a = a_in; d.res = res; d.w1 = n_a; d.w2 = n_b; d.w3 = n_c; d.side = side;
        d.W = bits == 32 ? static_cast<const void*>(L.w) : L.q;
        d.S = L.scale;
        d.out = out;
        d.M = int(M); d.N = int(N); d.K = int(C); d.G = bits == 32 ? 1 : G;
        d.groups = bits == 32 ? 0 : int(C / G);
        d.F = int(F); d.eps = c->eps; d.pro = pro;
        return launch_dit_gemm(g, bits, pair, d);
    };
    auto gemm = [&](const dgm_dit_linear& L, const float* in, float* out, int64_t N, int64_t K) -> int {
        dgm_GemmP gp{uint32_t(M), uint32_t(N), uint32_t(K), 0u, uint32_t(bits == 32 ? 0 : G), 0, 0, 0};
        int r = gemm_check_sizes(g, "dit_forward_train", &gp, bits);
        if (r) return r;
        const void* wt = bits == 32 ? static_cast<const void*>(L.w) : L.q;
        r = gemm_f32_fwd(g, bits, wt, L.scale, in, nullptr, out, &gp);
        if (r) return r;
        return check_launch(g, "dit_forward_train gemm");
    };
    for (int l = 0; l < c->loops; ++l) {
        const DitSaves& S = saves[l];
        float* qkv = l == 0 ? qkv0 : qkv1;
        DitGemmArgs d{};
        d.lnout = S.ln1;
        if (l == 0) {   // x (saved as loop 0's input) -> ln1 = rms(x) * n1
            d.rs1 = S.r1;
            DGM_TRY(pgemm(w->wq, false, 1, x, nullptr, w->n1, nullptr, nullptr, S.x, qkv, QKV, d));
        } else {        // pre = mid + rms(mlp) * n2b; x = rms(pre) * nf; ln1 = rms(x) * n1
            const DitSaves& P = saves[l - 1];
            d.side1 = P.pre; d.rs1 = P.r2b; d.rs2 = P.rf; d.rs3 = S.r1;
            DGM_TRY(pgemm(w->wq, false, 3, P.mlp, P.mid, w->n2b, w->nf, w->n1, S.x, qkv, QKV, d));
        }
        AttnArgs aa{};
        aa.q = qkv; aa.k = qkv + C; aa.v = qkv + C + KV; aa.vfirst = qkv0 + C + KV;
        aa.cosv = cosv; aa.sinv = sinv;
        aa.scores = scores; aa.probs = S.probs; aa.av = S.av;
        aa.B = B; aa.T = T; aa.H = H; aa.D = D;
        aa.q_ld = aa.kv_ld = aa.vf_ld = int(QKV); aa.av_ld = int(C);
        aa.kv_heads = 1;
        aa.scale = 1.0f / sqrtf(float(D));
        aa.ca = 1.0f - c->mix; aa.cb = c->mix;
        aa.causal = 0; aa.rope = 1; aa.vmix = l > 0;
        aa.qo = S.q; aa.ko = S.k; aa.vo = S.v; aa.o_ld = int(C);
        DGM_TRY(launch_attn_mfma(g, aa));
        DGM_TRY(gemm(w->wo, S.av, S.attn, C, C));
        // mid = x + rms(attn) * n1b; ln2 = rms(mid) * n2; gate, up; sw = swiglu(gate, up)
        DitGemmArgs d2{};
        d2.lnout = S.ln2; d2.rs1 = S.r1b; d2.rs2 = S.r2; d2.gate_out = S.gate; d2.up_out = S.up;
        DGM_TRY(pgemm(w->wgate, true, 2, S.attn, S.x, w->n1b, w->n2, nullptr, S.mid, S.sw, 2 * F, d2));
        DGM_TRY(gemm(w->wdown, S.sw, S.mlp, C, F));
    }
    if (c->loops > 0) {   // pre = mid + rms(mlp) * n2b; x = rms(pre) * nf
        const DitSaves& P = saves[c->loops - 1];
        DGM_TRY(launch_row_fuse(g, P.mlp, P.mid, P.pre, x, nullptr, w->n2b, w->nf, nullptr, P.rf, M, C, c->eps,
                                P.r2b));
    }
#undef DGM_TRY
    return DGM_OK;
}

}  // namespace dgm

extern "C" {

// ---- GPU.swift-style entry points (src/GPU.swift:212-410) -------------------------

int dgm_rmsFwd(dgm_gpu* g, const float* x, float* y, float* rstd, const float* weight, int64_t rows,
               int64_t cols, float eps) {
    int rc = dgm::enter(g, "rmsnorm_fwd");
    if (rc) return rc;
    if (rows < 0 || cols < 0 || rows > dgm::kMaxIndex || cols > dgm::kMaxIndex || bad_count(rows * cols))
        return dgm::fail(g, DGM_ERR_ARG, "rmsFwd: bad sizes rows=%lld cols=%lld", (long long)rows, (long long)cols);
    if (rows && cols && (!x || !y || !weight)) return dgm::fail(g, DGM_ERR_ARG, "rmsFwd: null buffer");
    return launch_rms(g, x, y, rstd, weight, rows, cols, eps);
}

int dgm_ropeFwd(dgm_gpu* g, const float* x, float* y, const float* cosv, const float* sinv, int64_t B,
                int64_t T, int64_t H, int64_t D) {
    int rc = dgm::enter(g, "rope_fwd");
    if (rc) return rc;
    rc = check_bthd(g, "ropeFwd", B, T, H, D);
    if (rc) return rc;
    if (D % 2 != 0) return dgm::fail(g, DGM_ERR_SHAPE, "ropeFwd: head dim %lld must be even", (long long)D);
    if (B * T * H * D && (!x || !y || !cosv || !sinv)) return dgm::fail(g, DGM_ERR_ARG, "ropeFwd: null buffer");
    return launch_rope(g, x, y, cosv, sinv, int(B), int(T), int(H), int(D));
}

int dgm_repeatHeads(dgm_gpu* g, const float* src, float* dst, int64_t B, int64_t T, int64_t H, int64_t D) {
    int rc = dgm::enter(g, "repeat_heads");
    if (rc) return rc;
    rc = check_bthd(g, "repeatHeads", B, T, H, D);
    if (rc) return rc;
    if (B * T * H * D && (!src || !dst)) return dgm::fail(g, DGM_ERR_ARG, "repeatHeads: null buffer");
    return launch_repeat(g, src, dst, int(B), int(T), int(H), int(D));
}

int dgm_attnFwd(dgm_gpu* g, const float* q, const float* k, const float* v, float* scores, float* probs,
                float* av, int64_t B, int64_t T, int64_t H, int64_t D, int causal) {
    int rc = dgm::enter(g, "attn_fwd");
    if (rc) return rc;
    rc = check_bthd(g, "attnFwd", B, T, H, D);
    if (rc) return rc;
    if (B * T * H * D && (!q || !k || !v || !scores || !probs || !av))
        return dgm::fail(g, DGM_ERR_ARG, "attnFwd: null buffer");
    if (attn_lds_bytes(int(T), int(D)) > 160 * 1024)
        return dgm::fail(g, DGM_ERR_UNSUPPORTED, "attnFwd: T*D = %lld exceeds the LDS-resident kernel",
                         (long long)(T * D));
    return launch_attn(g, q, k, v, scores, probs, av, int(B), int(T), int(H), int(D), causal ? 1 : 0);
}

int dgm_swigluFwd(dgm_gpu* g, const float* gate, const float* up, float* y, int64_t n) {
    int rc = dgm::enter(g, "swiglu_fwd");
    if (rc) return rc;
    if (bad_count(n)) return dgm::fail(g, DGM_ERR_ARG, "swigluFwd: bad count");
    if (n && (!gate || !up || !y)) return dgm::fail(g, DGM_ERR_ARG, "swigluFwd: null buffer");
    return launch_swiglu(g, gate, up, y, n);
}

int dgm_add(dgm_gpu* g, const float* a, const float* b, float* y, int64_t n) {
    int rc = dgm::enter(g, "add_f");
    if (rc) return rc;
    if (bad_count(n)) return dgm::fail(g, DGM_ERR_ARG, "add: bad count");
    if (n && (!a || !b || !y)) return dgm::fail(g, DGM_ERR_ARG, "add: null buffer");
    return launch_add(g, a, b, y, n);
}

int dgm_mix(dgm_gpu* g, const float* a, const float* b, float* y, int64_t n, float ca, float cb) {
    int rc = dgm::enter(g, "mix_f");
    if (rc) return rc;
    if (bad_count(n)) return dgm::fail(g, DGM_ERR_ARG, "mix: bad count");
    if (n && (!a || !b || !y)) return dgm::fail(g, DGM_ERR_ARG, "mix: null buffer");
    return launch_mix(g, a, b, y, n, ca, cb);
}

int dgm_copy(dgm_gpu* g, const float* x, float* y, int64_t n) {
    int rc = dgm::enter(g, "copy_f");
    if (rc) return rc;
    if (bad_count(n)) return dgm::fail(g, DGM_ERR_ARG, "copy: bad count");
    if (n && (!x || !y)) return dgm::fail(g, DGM_ERR_ARG, "copy: null buffer");
    return launch_copy(g, x, y, n);
}

// ---- ropeTables (src/Macro.swift:509-530), host side --------------------------------

int dgm_ropeTables(int64_t maxT, int64_t dim, float theta, float* cos_t, float* sin_t) {
    if (maxT < 0 || dim < 0 || dim % 2 != 0 || maxT > dgm::kMaxIndex || dim > dgm::kMaxIndex ||
        maxT * dim > (int64_t(1) << 40))
        return DGM_ERR_ARG;
    if (maxT * dim == 0) return DGM_OK;
    if (!cos_t || !sin_t) return DGM_ERR_ARG;
    const int64_t half = dim / 2;
    for (int64_t t = 0; t < maxT; ++t) {
        for (int64_t i = 0; i < half; ++i) {
            const float e = float(2 * i) / float(dim);
            const float inv = ::powf(theta, -e);
            const float f = float(t) * inv;
            const float c = ::cosf(f), s = ::sinf(f);
            cos_t[t * dim + i] = c;
            cos_t[t * dim + i + half] = c;
            sin_t[t * dim + i] = s;
            sin_t[t * dim + i + half] = s;
        }
    }
    return DGM_OK;
}

// ---- block forward ------------------------------------------------------------------

int64_t dgm_dit_workspace_floats(const dgm_dit_cfg* c) { return c ? dit_workspace_floats(c) : -1; }

int dgm_dit_forward(dgm_gpu* g, const dgm_dit_cfg* c, const dgm_dit_weights* w, const float* cosv,
                    const float* sinv, float* x, float* ws, int64_t ws_floats) {
    int rc = dgm::enter(g, "dit_forward");
    if (rc) return rc;
    if (!c || !w || !x || !ws || !cosv || !sinv) return dgm::fail(g, DGM_ERR_ARG, "dit_forward: null argument");
    if (!dgm::aligned(x, 16) || !dgm::aligned(ws, 16) || !dgm::aligned(cosv, 16) || !dgm::aligned(sinv, 16))
        return dgm::fail(g, DGM_ERR_ARG, "dit_forward: x, ws and the RoPE tables must be 16-byte aligned");
    if (c->bits != 4 && c->bits != 8 && c->bits != 32)
        return dgm::fail(g, DGM_ERR_BITS, "dit_forward: unsupported bits %d", c->bits);
    if (c->B <= 0 || c->T <= 0 || c->C <= 0 || c->F <= 0 || c->H <= 0 || c->D <= 0 || c->loops < 0 ||
        c->H * c->D != c->C || c->D % 2 != 0)
        return dgm::fail(g, DGM_ERR_SHAPE, "dit_forward: bad config (C must be H*D, D even)");
    if (c->C > 64 * kRowMax)
        return dgm::fail(g, DGM_ERR_UNSUPPORTED, "dit_forward: embd %d above %d", c->C, 64 * kRowMax);
    if (c->bits != 32 && (c->group <= 0 || c->C % c->group != 0 || c->F % c->group != 0 ||
                          (c->bits == 4 && c->group % 2 != 0)))
        return dgm::fail(g, DGM_ERR_SHAPE, "dit_forward: C and F must be multiples of an (even for int4) group");
    if (!attn_mfma_ok(c->T, c->D))
        return dgm::fail(g, DGM_ERR_UNSUPPORTED,
                         "dit_forward: tokens %d and head dim %d must be multiples of 16 (LDS-resident attention)",
                         c->T, c->D);
    if (int64_t(c->B) * c->T * (c->C + 2 * c->F) > (int64_t(1) << 31))
        return dgm::fail(g, DGM_ERR_UNSUPPORTED, "dit_forward: activations beyond 2^31 elements");
    if (ws_floats < dit_workspace_floats(c)) return dgm::fail(g, DGM_ERR_ARG, "dit_forward: workspace too small");
    const dgm_dit_linear* lins[7] = {&w->wq, &w->wk, &w->wv, &w->wo, &w->wgate, &w->wup, &w->wdown};
    for (const dgm_dit_linear* L : lins)
        if (c->bits == 32 ? !L->w : (!L->q || !L->scale)) return dgm::fail(g, DGM_ERR_ARG, "dit_forward: null weight");
    if (!w->n1 || !w->n1b || !w->n2 || !w->n2b || !w->nf) return dgm::fail(g, DGM_ERR_ARG, "dit_forward: null norm");

    int64_t sz[NBUF];
    float* p[NBUF];
    dit_sizes(c, sz);
    float* cur = ws;
    for (int i = 0; i < NBUF; ++i) {
        p[i] = cur;
        cur += (sz[i] + 63) & ~int64_t(63);
    }
    // Three launches per loop when the shape is built for it: the wdown
    // slabs take the gu | sw pieces (contiguous), loop 0's v the qkv0 piece,
    // q | k | v the qkv1 piece, and mid alternates between the mid and pre
    // pieces.
    if (dgm::dit_loop_ok(c, w) && dgm::dit_loop_part_floats(c) <= (p[SW] - p[GU]) + sz[SW]) {
        const int64_t MC = int64_t(c->B) * c->T * c->C, MD = int64_t(c->B) * c->T * c->D;
        const dgm::DitLoopBufs buf{p[GU], p[QKV0], p[QKV1], p[QKV1] + MC, p[QKV1] + MC + MD,
                                   {p[MID], p[PRE]}, p[LN2], p[PROBS]};
        return dgm::dit_forward_loops(g, c, w, cosv, sinv, x, buf, nullptr);
    }
    const int B = c->B, T = c->T, H = c->H, D = c->D, bits = c->bits, G = c->group;
    const int64_t M = int64_t(B) * T, C = c->C, F = c->F, KV = D, QKV = C + 2 * KV;
    // Back-to-back weights run as one GEMM: [wq; wk; wv] and [wgate; wup].
    const bool fuse_qkv = follows(w->wq, w->wk, C, C, bits, G) && follows(w->wk, w->wv, KV, C, bits, G);
    const bool fuse_gu = follows(w->wgate, w->wup, F, C, bits, G);

    auto gemm = [&](const dgm_dit_linear& L, const float* in, float* out, int64_t N, int64_t K) -> int {
        dgm_GemmP gp{uint32_t(M), uint32_t(N), uint32_t(K), 0u, uint32_t(bits == 32 ? 0 : G), 0, 0, 0};
        int r = dgm::gemm_check_sizes(g, "dit_forward", &gp, bits);
        if (r) return r;
        const void* wt = bits == 32 ? static_cast<const void*>(L.w) : L.q;
        r = dgm::gemm_f32_fwd(g, bits, wt, L.scale, in, nullptr, out, &gp);
        if (r) return r;
        return dgm::check_launch(g, "dit_forward gemm");
    };
#define DGM_TRY(expr)                \
    do {                             \
        int _r = (expr);             \
        if (_r != DGM_OK) return _r; \
    } while (0)
    if (fuse_qkv && fuse_gu && dit_fused_ok(c, w)) {
        // Five launches per loop: [row chain +] qkv projection, attention, wo,
        // [row chain +] gate/up with SwiGLU, wdown; one row chain at the end.
        auto pgemm = [&](const dgm_dit_linear& L, bool pair, int pro, const float* a_in, const float* res,
                         const float* n_a, const float* n_b, const float* n_c, float* side, float* out,
                         int64_t N) -> int {
            DitGemmArgs d{};
            d.a = a_in; d.res = res; d.w1 = n_a; d.w2 = n_b; d.w3 = n_c; d.side = side;
            d.W = bits == 32 ? static_cast<const void*>(L.w) : L.q;
            d.S = L.scale;
            d.out = out;
            d.M = int(M); d.N = int(N); d.K = int(C); d.G = bits == 32 ? 1 : G;
            d.groups = bits == 32 ? 0 : int(C / G);
            d.F = int(F); d.eps = c->eps; d.pro = pro;
            return launch_dit_gemm(g, bits, pair, d);
        };
        for (int loop = 0; loop < c->loops; ++loop) {
            float* qkv = p[loop == 0 ? QKV0 : QKV1];
            if (loop == 0)
                DGM_TRY(pgemm(w->wq, false, 1, x, nullptr, w->n1, nullptr, nullptr, nullptr, qkv, QKV));
            else   // x = rms(mid + rms(mlp) * n2b) * nf; ln1 = rms(x) * n1
                DGM_TRY(pgemm(w->wq, false, 3, p[MLP], p[MID], w->n2b, w->nf, w->n1, x, qkv, QKV));
            AttnArgs aa{};
            aa.q = qkv; aa.k = qkv + C; aa.v = qkv + C + KV; aa.vfirst = p[QKV0] + C + KV;
            aa.cosv = cosv; aa.sinv = sinv;
            aa.scores = p[SCORES]; aa.probs = p[PROBS]; aa.av = p[AV];
            aa.B = B; aa.T = T; aa.H = H; aa.D = D;
            aa.q_ld = aa.kv_ld = aa.vf_ld = int(QKV); aa.av_ld = int(C);
            aa.kv_heads = 1;
            aa.scale = 1.0f / sqrtf(float(D));
            aa.ca = 1.0f - c->mix; aa.cb = c->mix;
            aa.causal = 0; aa.rope = 1; aa.vmix = loop > 0;
            DGM_TRY(launch_attn_mfma(g, aa));
            DGM_TRY(gemm(w->wo, p[AV], p[ATTN], C, C));
            // mid = x + rms(attn) * n1b; ln2 = rms(mid) * n2; sw = swiglu(ln2 Wg^T, ln2 Wu^T)
            DGM_TRY(pgemm(w->wgate, true, 2, p[ATTN], x, w->n1b, w->n2, nullptr, p[MID], p[SW], 2 * F));
            DGM_TRY(gemm(w->wdown, p[SW], p[MLP], C, F));
        }
        if (c->loops > 0)
            DGM_TRY(launch_row_fuse(g, p[MLP], p[MID], p[PRE], x, nullptr, w->n2b, w->nf, nullptr, p[RSTD], M, C,
                                    c->eps));
        return DGM_OK;
    }
    DGM_TRY(launch_rms(g, x, p[LN1], p[RSTD], w->n1, M, C, c->eps));
    for (int loop = 0; loop < c->loops; ++loop) {
        float* qkv = p[loop == 0 ? QKV0 : QKV1];
        // q / k / v projections; fused: rows of qkv are [q | k | v], else three blocks.
        const float *q, *k, *v;
        int q_ld, kv_ld, v_ld;
        if (fuse_qkv) {
            DGM_TRY(gemm(w->wq, p[LN1], qkv, QKV, C));
            q = qkv; k = qkv + C; v = qkv + C + KV;
            q_ld = kv_ld = v_ld = int(QKV);
        } else {
            DGM_TRY(gemm(w->wq, p[LN1], qkv, C, C));
            DGM_TRY(gemm(w->wk, p[LN1], qkv + M * C, KV, C));
            DGM_TRY(gemm(w->wv, p[LN1], qkv + M * (C + KV), KV, C));
            q = qkv; k = qkv + M * C; v = qkv + M * (C + KV);
            q_ld = int(C); kv_ld = v_ld = int(KV);
        }
        const float* vfirst = fuse_qkv ? p[QKV0] + C + KV : p[QKV0] + M * (C + KV);
        // value residual (mix), RoPE on q and k, one KV head for all heads, full attention.
        {
            AttnArgs aa{};
            aa.q = q; aa.k = k; aa.v = v; aa.vfirst = vfirst; aa.cosv = cosv; aa.sinv = sinv;
            aa.scores = p[SCORES]; aa.probs = p[PROBS]; aa.av = p[AV];
            aa.B = B; aa.T = T; aa.H = H; aa.D = D;
            aa.q_ld = q_ld; aa.kv_ld = kv_ld; aa.vf_ld = v_ld; aa.av_ld = int(C);
            aa.kv_heads = 1;
            aa.scale = 1.0f / sqrtf(float(D));
            aa.ca = 1.0f - c->mix; aa.cb = c->mix;
            aa.causal = 0; aa.rope = 1; aa.vmix = loop > 0;
            (void)v_ld;   // == kv_ld in both layouts
            DGM_TRY(launch_attn_mfma(g, aa));
        }
        DGM_TRY(gemm(w->wo, p[AV], p[ATTN], C, C));
        // mid = x + rms(attn) * n1b; ln2 = rms(mid) * n2
        DGM_TRY(launch_row_fuse(g, p[ATTN], x, p[MID], p[LN2], nullptr, w->n1b, w->n2, nullptr, p[RSTD], M, C,
                                c->eps));
        if (fuse_gu) {
            DGM_TRY(gemm(w->wgate, p[LN2], p[GU], 2 * F, C));
            DGM_TRY(launch_swiglu_rows(g, p[GU], p[GU] + F, p[SW], M, F, 2 * F, 2 * F));
        } else {
            DGM_TRY(gemm(w->wgate, p[LN2], p[GU], F, C));
            DGM_TRY(gemm(w->wup, p[LN2], p[GU] + M * F, F, C));
            DGM_TRY(launch_swiglu_rows(g, p[GU], p[GU] + M * F, p[SW], M, F, F, F));
        }
        DGM_TRY(gemm(w->wdown, p[SW], p[MLP], C, F));
        // pre = mid + rms(mlp) * n2b; x = rms(pre) * nf; next ln1 = rms(x) * n1
        const bool more = loop + 1 < c->loops;
        DGM_TRY(launch_row_fuse(g, p[MLP], p[MID], p[PRE], x, more ? p[LN1] : nullptr, w->n2b, w->nf,
                                more ? w->n1 : nullptr, p[RSTD], M, C, c->eps));
    }
#undef DGM_TRY
    return DGM_OK;
}

}  // extern "C"
