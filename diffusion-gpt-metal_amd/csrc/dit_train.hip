// Training step of the looped DiT block (src/DiT.swift:505-626) on gfx950:
// the backward kernels of the block's non-GEMM pieces, their GPU.swift-style
// C entry points, a forward that saves every loop's activations, and the
// block backward that accumulates the weight and norm gradients.
//
// Kernels (semantics of metal/kernels.metal, cited per kernel; fp contraction
// off, each product and sum rounded as in the reference's separate
// operations):
//  * rms_bwd: dx (one wave per row; the row's sum(dy*w*x) is a wave reduction,
//    fp32, a different order than the reference's sequential loop) and
//    dweight (16 waves per 64 columns, partial sums added in wave order, then
//    into dweight: the weight is shared by every loop) in one launch, dx
//    optionally added to a residual gradient; rms_bwd_chain runs up to three
//    of them back to back per row (the block backward's consecutive norms).
//  * attention backward: for T % 8 == 0 two launches over 8-row blocks of
//    each head (query rows: dP, dS, dQ; key rows: dV, dK); else one workgroup
//    per (batch, head) with the head in LDS (T and D multiples of 4,
//    (4TD + 2T^2) floats of LDS), or the reference's five passes with one lane
//    per output. All sum in the reference's order and are bitwise the
//    oracle's.
//  * rope_bwd, swiglu_bwd, sum_heads, acc_f, acc_scale_f: elementwise;
//    qkv_grad: sum_heads, rope_bwd and the value-residual steps of the q / k /
//    v gradients in one launch, one wave per token row.
//  * swiglu_bwd and qkv_grad can write [dgate | dup] and [dq | dk | dv] rows,
//    the output gradient of the stacked [gate; up] and [q; k; v] linears.
// The block's GEMMs are the library's: dgm_gemmNT and dgm_gemmBwd (gemmDWAcc +
// gemmDX in one launch; for wdown with the SwiGLU backward applied to its dX,
// dgm::gemm_bwd_swiglu) on the fp32 masters (bits 32, as the reference's DiT) or on
// the group-quantized codes (bits 8 / 4: forward on the codes, dX through the
// dequantized codes, dW into the fp32 master gradient: the straight-through
// estimator of src/GPT.swift's backward).
#include <cmath>

#include "common.hpp"
#include "dit_rows.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 256;

// Sum over the wave on DPP and permlane swaps; every lane gets the same bits.
__device__ __forceinline__ float wave_sum(float v) { return dgm_rows::wave64_sum(v); }

constexpr int kDwWaves = 16;

// ---- rmsnorm backward (metal/kernels.metal:827-868), dx and dweight in one launch --
// Workgroups [0, ndx) take 16 rows each for dx: one wave per row, the row's
// sum(dy*w*x) a wave reduction (fp32, a different order than the reference's
// sequential loop). The others take 64 columns each for dweight += sum over
// rows: wave w sums rows w, w+16, ... and the 16 partial sums are added in
// wave order, then added into dweight (the weight is shared by every loop). With
// `add`, dx[r, c] = add[r, c] + the row's dx (an acc_f of the result; add may
// alias dx).
__global__ __launch_bounds__(64 * kDwWaves) void rms_bwd_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ rstd,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ dy, float* dx,
                                                                const float* add, float* __restrict__ dweight,
                                                                int rows, int cols, int ndx) {
    __shared__ float part[kDwWaves][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (int(blockIdx.x) < ndx) {
        const int row = blockIdx.x * kDwWaves + wave;
        if (row >= rows) return;
        const float* xr = x + size_t(row) * cols;
        const float* gr = dy + size_t(row) * cols;
        float pt = 0.0f;
        for (int c = lane; c < cols; c += 64) {
            const float dyhat = gr[c] * w[c];
            pt += dyhat * xr[c];
        }
        const float meanDyX = wave_sum(pt) / float(cols);
        const float rs = rstd[row];
        const float rs3 = rs * rs * rs;
        float* o = dx + size_t(row) * cols;
        const float* ad = add ? add + size_t(row) * cols : nullptr;
        for (int c = lane; c < cols; c += 64) {
            const float dyhat = gr[c] * w[c];
            const float v = rs * dyhat - xr[c] * rs3 * meanDyX;
            o[c] = ad ? ad[c] + v : v;
        }
        return;
    }
    const int c = (int(blockIdx.x) - ndx) * 64 + lane;
    float acc = 0.0f;
    if (c < cols) {
        int r = wave;
        for (; r + 7 * kDwWaves < rows; r += 8 * kDwWaves) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int rr = r + u * kDwWaves;
                v[u] = dy[size_t(rr) * cols + c] * x[size_t(rr) * cols + c] * rstd[rr];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += v[u];
        }
        for (; r < rows; r += kDwWaves) acc += dy[size_t(r) * cols + c] * x[size_t(r) * cols + c] * rstd[r];
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && c < cols) {
        float tot = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < kDwWaves; ++w2) tot += part[w2][lane];
        dweight[c] += tot;
    }
}

// ---- chained rmsnorm backwards in one launch (the DiT backward's runs) -----------
// Stage 0 is rms_bwd above: out = [add +] dx of (x, r, w, dy), its weight
// gradient dw0 += sum over rows by the direct workgroups. Each further stage
// takes the previous stage's out as its dy, computed by the same wave from
// values held in registers (so a stage's add may alias its out). A further
// stage's weight gradient needs the previous out of every row, so each dx
// workgroup writes its sums over its 16 rows (in row order) to
// part[block][cols], and a later launch adds the blocks in order into the
// gradient: pin[p] / dwp[p] name such pending partial sums (npin blocks),
// reduced here by their own workgroups. Row arithmetic is rms_bwd's;
// cols <= 256.
constexpr int kChainCols = 256;
constexpr int kChainStages = 3;
struct RmsStage {
    const float *x, *r, *w;
    float* out;
    const float* add;
    float* part;   // stages >= 1
};
struct RmsChainArgs {
    const float* dy;
    RmsStage st[kChainStages];
    int nst;
    float* dw0;
    const float* pin[2];
    float* dwp[2];
    int npend, npin;
    int rows, cols, ndx, ndw, ndd;   // ndd: stage 0's weight-gradient workgroups (8 columns each)
    dgm_dw::DwTileArgs dw;           // a linear's dW run beside the chain (it reads none of its outputs)
    int dw_tiles, dw_tiles_n;        // its 32 x 16 tiles, one per workgroup after the others
};

__global__ __launch_bounds__(64 * kDwWaves) void rms_bwd_chain_kernel(RmsChainArgs a) {
    static_assert(kDwWaves == dgm_dw::kHostedWaves, "one dW tile per workgroup");
    // part[kDwWaves][kChainCols] for the chain, 32 KB for a dW tile.
    constexpr int kDwFloats = dgm_dw::kHostedWaves * 2 * 16 * 16;
    __shared__ __align__(16) float lds[kDwWaves * kChainCols > kDwFloats ? kDwWaves * kChainCols : kDwFloats];
    float (*part)[kChainCols] = reinterpret_cast<float (*)[kChainCols]>(lds);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cols = a.cols, rows = a.rows;
    constexpr int NPL = kChainCols / 64;
    const int blk = int(blockIdx.x);
    if (blk < a.ndx) {
        const int row = blk * kDwWaves + wave;
        const bool live = row < rows;
        // Every stage's operands are loaded before the first stage computes,
        // so the chain waits for one round of loads, not one per stage.
        float g[NPL];   // the stage's dy, then its out
        float xv[kChainStages][NPL], wv[kChainStages][NPL], av[kChainStages][NPL], rv[kChainStages];
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int c = lane + 64 * i;
            g[i] = live && c < cols ? a.dy[size_t(row) * cols + c] : 0.0f;
        }
#pragma unroll
        for (int s = 0; s < kChainStages; ++s) {
            const RmsStage& S = a.st[s];
            const bool on = live && s < a.nst;
            rv[s] = on ? S.r[row] : 0.0f;
#pragma unroll
            for (int i = 0; i < NPL; ++i) {
                const int c = lane + 64 * i;
                const bool in = on && c < cols;
                xv[s][i] = in ? S.x[size_t(row) * cols + c] : 0.0f;
                wv[s][i] = in ? S.w[c] : 0.0f;
                av[s][i] = in && S.add ? S.add[size_t(row) * cols + c] : 0.0f;
            }
        }
#pragma unroll
        for (int s = 0; s < kChainStages; ++s) {
            if (s >= a.nst) break;
            const RmsStage& S = a.st[s];
            if (live) {
                float pt = 0.0f;
#pragma unroll
                for (int i = 0; i < NPL; ++i) {
                    const int c = lane + 64 * i;
                    if (c < cols) pt += (g[i] * wv[s][i]) * xv[s][i];
                }
                const float meanDyX = wave_sum(pt) / float(cols);
                const float rs = rv[s];
                const float rs3 = rs * rs * rs;
                float* o = S.out + size_t(row) * cols;
#pragma unroll
                for (int i = 0; i < NPL; ++i) {
                    const int c = lane + 64 * i;
                    if (c < cols) {
                        if (s > 0) part[wave][c] = g[i] * xv[s][i] * rs;   // this stage's dy * xhat
                        const float dyhat = g[i] * wv[s][i];
                        const float v = rs * dyhat - xv[s][i] * rs3 * meanDyX;
                        g[i] = S.add ? av[s][i] + v : v;
                        o[c] = g[i];
                    }
                }
            } else if (s > 0) {
                for (int c = lane; c < cols; c += 64) part[wave][c] = 0.0f;
            }
            if (s > 0) {
                __syncthreads();
                for (int c = threadIdx.x; c < cols; c += 64 * kDwWaves) {
                    float tot = 0.0f;
#pragma unroll
                    for (int w2 = 0; w2 < kDwWaves; ++w2) tot += part[w2][c];
                    S.part[size_t(blk) * cols + c] = tot;
                }
                __syncthreads();
            }
        }
        return;
    }
    // Stage 0's weight gradient: 8 columns per workgroup; lane (column c0 +
    // lane % 8, row phase lane / 8) of wave w sums rows 8 w + phase + 128 u in
    // order, all its loads in flight at once (one round trip, like the dx
    // workgroups: with 64 columns per workgroup and 32 rows per lane in two
    // rounds these workgroups finished last, ~8 us per training step), then
    // the 128 partial sums of a column are added in a fixed order (wave, then
    // phase).
    const int rest = blk - a.ndx;
    if (rest < a.ndd) {
        const int c = rest * 8 + (lane % 8), ph = lane / 8;
        float acc = 0.0f;
        if (c < cols) {
            const float* x = a.st[0].x;
            const float* r1 = a.st[0].r;
            for (int r0 = 8 * wave + ph; r0 < rows; r0 += 128 * 8) {   // 8 rows' loads in flight
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int rr = r0 + 128 * u;
                    v[u] = rr < rows ? a.dy[size_t(rr) * cols + c] * x[size_t(rr) * cols + c] * r1[rr] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) acc += v[u];
            }
        }
        part[wave][lane] = acc;
        __syncthreads();
        if (wave == 0 && ph == 0 && c < cols) {
            float tot = 0.0f;
            for (int w2 = 0; w2 < kDwWaves; ++w2)
#pragma unroll
                for (int p2 = 0; p2 < 8; ++p2) tot += part[w2][8 * p2 + lane];
            a.dw0[c] += tot;
        }
        return;
    }
    const int pr = rest - a.ndd;
    if (pr >= a.ndw * a.npend) {
        dgm_dw::dw_tile<2, dgm_dw::kPairCH, dgm_dw::kHostedWaves>(a.dw, true, pr - a.ndw * a.npend, a.dw_tiles_n,
                                                                  wave, int(threadIdx.x),
                                                                  reinterpret_cast<float (*)[2][16][16]>(lds));
        return;
    }
    // The pending partial sums: 64 columns per workgroup.
    const int pi = pr / a.ndw;
    const int c = (pr % a.ndw) * 64 + lane;
    float acc = 0.0f;
    if (c < cols) {
        const float* pin = a.pin[pi];
        for (int b2 = wave; b2 < a.npin; b2 += kDwWaves) acc += pin[size_t(b2) * cols + c];
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && c < cols) {
        float tot = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < kDwWaves; ++w2) tot += part[w2][lane];
        a.dwp[pi][c] += tot;
    }
}

// ---- attention backward (metal/kernels.metal:508-612) -----------------------------
// q, k, v, dout, dq, dk, dv: [B, T, H, D]; probs, dprobs, dscores: [B, H, T, T].
struct AttnBwdArgs {
    const float *q, *k, *v, *probs, *dout;
    float *dq, *dk, *dv, *dprobs, *dscores;
    int B, T, H, D;
    float scale;
};

__global__ __launch_bounds__(kThreads) void attn_bwd_dv_kernel(AttnBwdArgs a) {
    const int64_t idx = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t total = int64_t(a.B) * a.T * a.H * a.D;
    if (idx >= total) return;
    const int d = int(idx % a.D);
    const int h = int((idx / a.D) % a.H);
    const int s = int((idx / (int64_t(a.D) * a.H)) % a.T);
    const int b = int(idx / (int64_t(a.D) * a.H * a.T));
    const float* pr = a.probs + (int64_t(b) * a.H + h) * a.T * a.T + s;
    const float* g = a.dout + (int64_t(b) * a.T * a.H + h) * a.D + d;
    float acc = 0.0f;
    for (int t = 0; t < a.T; ++t) acc += pr[int64_t(t) * a.T] * g[int64_t(t) * a.H * a.D];
    a.dv[idx] = acc;
}

__global__ __launch_bounds__(kThreads) void attn_bwd_dp_kernel(AttnBwdArgs a) {
    const int64_t idx = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t TT = int64_t(a.T) * a.T;
    if (idx >= int64_t(a.B) * a.H * TT) return;
    const int s = int(idx % a.T);
    const int t = int((idx / a.T) % a.T);
    const int h = int((idx / TT) % a.H);
    const int b = int(idx / (TT * a.H));
    const float* g = a.dout + ((int64_t(b) * a.T + t) * a.H + h) * a.D;
    const float* vv = a.v + ((int64_t(b) * a.T + s) * a.H + h) * a.D;
    float acc = 0.0f;
    for (int d = 0; d < a.D; ++d) acc += g[d] * vv[d];
    a.dprobs[idx] = acc;
}

__global__ __launch_bounds__(kThreads) void attn_softmax_bwd_kernel(AttnBwdArgs a) {
    const int64_t row = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (row >= int64_t(a.B) * a.H * a.T) return;
    const float* pr = a.probs + row * a.T;
    const float* g = a.dprobs + row * a.T;
    float* o = a.dscores + row * a.T;
    float dot = 0.0f;
    for (int i = 0; i < a.T; ++i) dot += g[i] * pr[i];
    for (int i = 0; i < a.T; ++i) o[i] = pr[i] * (g[i] - dot);
}

template <bool DQ>
__global__ __launch_bounds__(kThreads) void attn_bwd_dqk_kernel(AttnBwdArgs a) {
    // DQ: dq[b,t,h,d] = scale * sum_s ds[b,h,t,s] k[b,s,h,d]
    // else dk[b,s,h,d] = scale * sum_t ds[b,h,t,s] q[b,t,h,d]
    const int64_t idx = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t total = int64_t(a.B) * a.T * a.H * a.D;
    if (idx >= total) return;
    const int d = int(idx % a.D);
    const int h = int((idx / a.D) % a.H);
    const int r = int((idx / (int64_t(a.D) * a.H)) % a.T);
    const int b = int(idx / (int64_t(a.D) * a.H * a.T));
    const float* ds = a.dscores + (int64_t(b) * a.H + h) * a.T * a.T;
    const float* src = (DQ ? a.k : a.q) + (int64_t(b) * a.T * a.H + h) * a.D + d;
    float acc = 0.0f;
    for (int u = 0; u < a.T; ++u) {
        const float gval = DQ ? ds[int64_t(r) * a.T + u] : ds[int64_t(u) * a.T + r];
        acc += gval * src[int64_t(u) * a.H * a.D];
    }
    (DQ ? a.dq : a.dk)[idx] = acc * a.scale;
}

// ---- fused attention backward: one workgroup per (batch, head) -------------------
// The head's Q, K, dO rows, V transposed and its probability matrix P are
// staged in LDS once; dV = P^T dO and dP = dO V^T, the softmax backward
// dS = P (dP - rowdot), then dQ = scale dS K and dK = scale dS^T Q. 16 waves
// (four per SIMD, so one wave's LDS latency hides behind the others' work);
// each product gives a lane 2 x 2 outputs and runs its contraction loop
// unrolled by 4. Every sum runs over the contraction index in increasing
// order from +0.0f, the reference kernels' order, including the softmax
// row dot (lanes form the products, one lane adds them in order): bitwise
// the five separate passes. LDS: (4 T D + 2 T T) floats.
constexpr int kAbThreads = 1024;

// out(r0, c0, acc) receives rows r0, r0+1 x columns c0, c0+1; A2(r, k) the
// A values of rows r, r+1 at k; B2(k, c) the B values of columns c, c+1.
template <int NT = kAbThreads, typename FA, typename FB, typename FO>
__device__ __forceinline__ void tiled_product(int rows, int cols, int kdim, FA A2, FB B2, FO out) {
    const int tc = cols / 2;
    const int ntiles = (rows / 2) * tc;
    for (int tile = threadIdx.x; tile < ntiles; tile += NT) {
        const int r0 = (tile / tc) * 2, c0 = (tile % tc) * 2;
        float a00 = 0.0f, a01 = 0.0f, a10 = 0.0f, a11 = 0.0f;
        for (int k = 0; k < kdim; k += 4) {
            float2 a[4], b[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a[u] = A2(r0, k + u);
                b[u] = B2(k + u, c0);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a00 += a[u].x * b[u].x;
                a01 += a[u].x * b[u].y;
                a10 += a[u].y * b[u].x;
                a11 += a[u].y * b[u].y;
            }
        }
        out(r0, c0, a00, a01, a10, a11);
    }
}

__global__ __launch_bounds__(kAbThreads) void attn_bwd_fused_kernel(AttnBwdArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int T = a.T, D = a.D, H = a.H;
    const int b = blockIdx.x / H, h = blockIdx.x % H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* Q = lds;            // [T][D]
    float* K = Q + T * D;      // [T][D]
    float* Vt = K + T * D;     // [D][T]
    float* G = Vt + T * D;     // dO [T][D]
    float* P = G + T * D;      // [T][T]
    float* S = P + T * T;      // dP, then dS [T][T]
    const int64_t row_stride = int64_t(H) * D;
    const int64_t head0 = (int64_t(b) * T * H + h) * D;     // [b, 0, h, 0]
    const int64_t pm0 = (int64_t(b) * H + h) * T * T;         // [b, h, 0, 0]
    // Stage the head's rows (D % 4 == 0: 16-byte loads), V transposed, and P.
    const int d4 = D / 4;
    for (int i = threadIdx.x; i < T * d4; i += kAbThreads) {
        const int t = i / d4, c = (i % d4) * 4;
        const int64_t off = head0 + t * row_stride + c;
        *reinterpret_cast<float4*>(Q + t * D + c) = *reinterpret_cast<const float4*>(a.q + off);
        *reinterpret_cast<float4*>(K + t * D + c) = *reinterpret_cast<const float4*>(a.k + off);
        *reinterpret_cast<float4*>(G + t * D + c) = *reinterpret_cast<const float4*>(a.dout + off);
        const float4 v = *reinterpret_cast<const float4*>(a.v + off);
        Vt[(c + 0) * T + t] = v.x;
        Vt[(c + 1) * T + t] = v.y;
        Vt[(c + 2) * T + t] = v.z;
        Vt[(c + 3) * T + t] = v.w;
    }
    for (int i = threadIdx.x; i < T * T / 4; i += kAbThreads)
        reinterpret_cast<float4*>(P)[i] = reinterpret_cast<const float4*>(a.probs + pm0)[i];
    __syncthreads();
    auto f2 = [](const float* p) { return *reinterpret_cast<const float2*>(p); };
    auto col2 = [](const float* p, int stride) { return make_float2(p[0], p[stride]); };
    auto store2 = [&](float* base, int r0, int c0, float a00, float a01, float a10, float a11) {
        *reinterpret_cast<float2*>(base + head0 + r0 * row_stride + c0) = make_float2(a00, a01);
        *reinterpret_cast<float2*>(base + head0 + (r0 + 1) * row_stride + c0) = make_float2(a10, a11);
    };
    // dV[s][d] = sum_t P[t][s] dO[t][d]  (attn_bwd_dv)
    tiled_product(
        T, D, T, [&](int s0, int t) { return f2(P + t * T + s0); }, [&](int t, int d0) { return f2(G + t * D + d0); },
        [&](int s0, int d0, float a00, float a01, float a10, float a11) { store2(a.dv, s0, d0, a00, a01, a10, a11); });
    // dP[t][s] = sum_d dO[t][d] V[s][d]  (attn_bwd_dp)
    tiled_product(
        T, T, D, [&](int t0, int d) { return col2(G + t0 * D + d, D); }, [&](int d, int s0) { return f2(Vt + d * T + s0); },
        [&](int t0, int s0, float a00, float a01, float a10, float a11) {
            *reinterpret_cast<float2*>(S + t0 * T + s0) = make_float2(a00, a01);
            *reinterpret_cast<float2*>(S + (t0 + 1) * T + s0) = make_float2(a10, a11);
            *reinterpret_cast<float2*>(a.dprobs + pm0 + t0 * T + s0) = make_float2(a00, a01);
            *reinterpret_cast<float2*>(a.dprobs + pm0 + (t0 + 1) * T + s0) = make_float2(a10, a11);
        });
    __syncthreads();
    // dS[t][i] = P[t][i] (dP[t][i] - sum_i dP[t][i] P[t][i])  (attn_softmax_bwd):
    // one wave per row; lane l holds i = l, l+64, ...; the dot is added in i order.
    for (int t = wave; t < T; t += kAbThreads / 64) {
        float dot = 0.0f;
        for (int i0 = 0; i0 < T; i0 += 64) {
            const int i = i0 + lane;
            const float prod = i < T ? S[t * T + i] * P[t * T + i] : 0.0f;
            const int n = T - i0 < 64 ? T - i0 : 64;
            for (int j = 0; j < n; ++j) dot += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(prod), j));
        }
        for (int i = lane; i < T; i += 64) {
            const float ds = P[t * T + i] * (S[t * T + i] - dot);
            S[t * T + i] = ds;
            a.dscores[pm0 + t * T + i] = ds;
        }
    }
    __syncthreads();
    // dQ[t][d] = scale * sum_s dS[t][s] K[s][d]  (attn_bwd_dq)
    tiled_product(
        T, D, T, [&](int t0, int s) { return col2(S + t0 * T + s, T); }, [&](int s, int d0) { return f2(K + s * D + d0); },
        [&](int t0, int d0, float a00, float a01, float a10, float a11) {
            store2(a.dq, t0, d0, a00 * a.scale, a01 * a.scale, a10 * a.scale, a11 * a.scale);
        });
    // dK[s][d] = scale * sum_t dS[t][s] Q[t][d]  (attn_bwd_dk)
    tiled_product(
        T, D, T, [&](int s0, int t) { return f2(S + t * T + s0); }, [&](int t, int d0) { return f2(Q + t * D + d0); },
        [&](int s0, int d0, float a00, float a01, float a10, float a11) {
            store2(a.dk, s0, d0, a00 * a.scale, a01 * a.scale, a10 * a.scale, a11 * a.scale);
        });
}

// ---- split attention backward: 8-row blocks of a head in two launches ------------
// The fused kernel gives each (batch, head) one workgroup: 32 workgroups at the
// DiT's shape. Here a head's work is cut into blocks of 8 rows, with the same
// per-element arithmetic and summation orders (results bitwise those of the
// fused kernel):
//  * rows kernel, workgroup (b, h, query block): dP = dO V^T and the softmax
//    backward dS for its 8 query rows, then dQ = scale dS K; dP and dS go to
//    dprobs / dscores;
//  * keys kernel, workgroup (b, h, key block): dV = P^T dO and
//    dK = scale dS^T Q for its 8 key rows, reading dS from dscores.
// Both are bound by latency (global loads, then short LDS contractions): every
// thread issues all of its loads before its first LDS store, so staging is one
// round trip, and the products give one output per thread (sum over the
// contraction index in increasing order from +0.0f).
constexpr int kAsThreads = 1024;
constexpr int kAsRows = 8;

size_t attn_split_rows_lds(int T, int D) {
    return size_t(2 * kAsRows * T + kAsRows * D + (2 * T + 1) * D) * sizeof(float);
}
size_t attn_split_keys_lds(int T, int D) { return size_t(2 * kAsRows * T + 2 * T * D) * sizeof(float); }

// out(r, c, v) for r < rows, c < cols, v = sum_k A(r, k) * B(k, c); one output per thread.
template <typename FA, typename FB, typename FO>
__device__ __forceinline__ void split_product(int rows, int cols, int kdim, FA A, FB B, FO out) {
    for (int e = threadIdx.x; e < rows * cols; e += kAsThreads) {
        const int r = e / cols, c = e % cols;
        float acc = 0.0f;
        int k = 0;
        for (; k + 4 <= kdim; k += 4) {
            float x[4], y[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                x[u] = A(r, k + u);
                y[u] = B(k + u, c);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) acc += x[u] * y[u];
        }
        for (; k < kdim; ++k) acc += A(r, k) * B(k, c);
        out(r, c, acc);
    }
}

__global__ __launch_bounds__(kAsThreads) void attn_bwd_rows_kernel(AttnBwdArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int T = a.T, D = a.D, H = a.H;
    const int nblk = T / kAsRows;
    const int bh = blockIdx.x / nblk, t0 = (blockIdx.x % nblk) * kAsRows;
    const int b = bh / H, h = bh % H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* Gr = lds;                 // dO rows [kAsRows][D]
    float* Vt = Gr + kAsRows * D;    // [D][T + 1] (padded: the transposing stores spread over the banks)
    float* Kf = Vt + (T + 1) * D;    // [T][D]
    float* Pr = Kf + T * D;          // P rows [kAsRows][T]
    float* S = Pr + kAsRows * T;     // dP, then dS rows [kAsRows][T]
    const int64_t row_stride = int64_t(H) * D;
    const int64_t head0 = (int64_t(b) * T * H + h) * D;
    const int64_t pm0 = (int64_t(b) * H + h) * T * T + int64_t(t0) * T;   // row t0 of P, dP, dS
    const int d4 = D / 4, nkv = T * d4, ng = kAsRows * d4, np = kAsRows * T / 4;
    const int nmax = max(nkv, max(ng, np));
    for (int i = threadIdx.x; i < nmax; i += kAsThreads) {
        float4 kk{}, vv{}, gg{}, pp{};
        const int t = i / d4, c = (i % d4) * 4;
        if (i < nkv) {
            const int64_t off = head0 + t * row_stride + c;
            kk = *reinterpret_cast<const float4*>(a.k + off);
            vv = *reinterpret_cast<const float4*>(a.v + off);
        }
        if (i < ng) gg = *reinterpret_cast<const float4*>(a.dout + head0 + (t0 + t) * row_stride + c);
        if (i < np) pp = reinterpret_cast<const float4*>(a.probs + pm0)[i];
        if (i < nkv) {
            *reinterpret_cast<float4*>(Kf + t * D + c) = kk;
            Vt[(c + 0) * (T + 1) + t] = vv.x;
            Vt[(c + 1) * (T + 1) + t] = vv.y;
            Vt[(c + 2) * (T + 1) + t] = vv.z;
            Vt[(c + 3) * (T + 1) + t] = vv.w;
        }
        if (i < ng) *reinterpret_cast<float4*>(Gr + t * D + c) = gg;
        if (i < np) reinterpret_cast<float4*>(Pr)[i] = pp;
    }
    __syncthreads();
    // dP[t][s] = sum_d dO[t][d] V[s][d]
    split_product(
        kAsRows, T, D, [&](int r, int d) { return Gr[r * D + d]; }, [&](int d, int s) { return Vt[d * (T + 1) + s]; },
        [&](int r, int s, float v) {
            S[r * T + s] = v;
            a.dprobs[pm0 + r * T + s] = v;
        });
    __syncthreads();
    // dS rows: lane 0 of the row's wave forms the row dot in i order (the
    // products rounded, then added, as the fused kernel), then the wave
    // applies it.
    for (int r = wave; r < kAsRows; r += kAsThreads / 64) {
        float dot = 0.0f;
        if (lane == 0) {
            const float* sr = S + r * T;
            const float* pr = Pr + r * T;
            int i = 0;
            for (; i + 8 <= T; i += 8) {
                float x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) x[u] = sr[i + u] * pr[i + u];
#pragma unroll
                for (int u = 0; u < 8; ++u) dot += x[u];
            }
            for (; i < T; ++i) dot += sr[i] * pr[i];
        }
        dot = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(dot)));
        for (int i = lane; i < T; i += 64) {
            const float ds = Pr[r * T + i] * (S[r * T + i] - dot);
            S[r * T + i] = ds;
            a.dscores[pm0 + r * T + i] = ds;
        }
    }
    __syncthreads();
    // dQ[t][d] = scale * sum_s dS[t][s] K[s][d]
    split_product(
        kAsRows, D, T, [&](int r, int s) { return S[r * T + s]; }, [&](int s, int d) { return Kf[s * D + d]; },
        [&](int r, int d, float v) { a.dq[head0 + (t0 + r) * row_stride + d] = v * a.scale; });
}

__global__ __launch_bounds__(kAsThreads) void attn_bwd_keys_kernel(AttnBwdArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int T = a.T, D = a.D, H = a.H;
    const int nblk = T / kAsRows;
    const int bh = blockIdx.x / nblk, s0 = (blockIdx.x % nblk) * kAsRows;
    const int b = bh / H, h = bh % H;
    float* G = lds;                  // dO [T][D]
    float* Qf = G + T * D;           // [T][D]
    float* Pc = Qf + T * D;          // P[:, s0 .. s0+kAsRows) as [T][kAsRows]
    float* Sc = Pc + T * kAsRows;    // dS[:, s0 .. s0+kAsRows) as [T][kAsRows]
    const int64_t row_stride = int64_t(H) * D;
    const int64_t head0 = (int64_t(b) * T * H + h) * D;
    const int64_t pm0 = (int64_t(b) * H + h) * T * T + s0;
    const int d4 = D / 4, nq = T * d4, c4 = kAsRows / 4, npc = T * c4;
    const int nmax = max(nq, npc);
    for (int i = threadIdx.x; i < nmax; i += kAsThreads) {
        float4 gg{}, qq{}, pp{}, ss{};
        const int t = i / d4, c = (i % d4) * 4;
        const int tp = i / c4, cp = (i % c4) * 4;
        if (i < nq) {
            const int64_t off = head0 + t * row_stride + c;
            gg = *reinterpret_cast<const float4*>(a.dout + off);
            qq = *reinterpret_cast<const float4*>(a.q + off);
        }
        if (i < npc) {
            pp = *reinterpret_cast<const float4*>(a.probs + pm0 + tp * T + cp);
            ss = *reinterpret_cast<const float4*>(a.dscores + pm0 + tp * T + cp);
        }
        if (i < nq) {
            *reinterpret_cast<float4*>(G + t * D + c) = gg;
            *reinterpret_cast<float4*>(Qf + t * D + c) = qq;
        }
        if (i < npc) {
            *reinterpret_cast<float4*>(Pc + tp * kAsRows + cp) = pp;
            *reinterpret_cast<float4*>(Sc + tp * kAsRows + cp) = ss;
        }
    }
    __syncthreads();
    // dV[s][d] = sum_t P[t][s] dO[t][d] and dK[s][d] = scale * sum_t dS[t][s] Q[t][d]:
    // one list of 2 x kAsRows x D outputs, dV first.
    const int nout = kAsRows * D;
    for (int e = threadIdx.x; e < 2 * nout; e += kAsThreads) {
        const bool isk = e >= nout;
        const int r = (isk ? e - nout : e) / D, d = (isk ? e - nout : e) % D;
        const float* A = (isk ? Sc : Pc) + r;
        const float* Bm = (isk ? Qf : G) + d;
        float acc = 0.0f;
        int t = 0;
        for (; t + 4 <= T; t += 4) {
            float x[4], y[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                x[u] = A[(t + u) * kAsRows];
                y[u] = Bm[(t + u) * D];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) acc += x[u] * y[u];
        }
        for (; t < T; ++t) acc += A[t * kAsRows] * Bm[t * D];
        float* o = (isk ? a.dk : a.dv) + head0 + (s0 + r) * row_stride + d;
        *o = isk ? acc * a.scale : acc;
    }
}

bool attn_split_ok(const AttnBwdArgs& a) {
    return a.T % kAsRows == 0 && a.D % 4 == 0 && attn_split_rows_lds(a.T, a.D) <= 64 * 1024 &&
           attn_split_keys_lds(a.T, a.D) <= 64 * 1024 && dgm::aligned(a.q, 16) && dgm::aligned(a.k, 16) &&
           dgm::aligned(a.v, 16) && dgm::aligned(a.dout, 16) && dgm::aligned(a.probs, 16) &&
           dgm::aligned(a.dscores, 16);
}

size_t attn_bwd_fused_lds(int T, int D) { return (size_t(4) * T * D + size_t(2) * T * T) * sizeof(float); }

bool attn_bwd_fused_ok(const AttnBwdArgs& a) {
    return a.T % 4 == 0 && a.D % 4 == 0 && attn_bwd_fused_lds(a.T, a.D) <= 160 * 1024 &&
           dgm::aligned(a.q, 16) && dgm::aligned(a.k, 16) && dgm::aligned(a.v, 16) && dgm::aligned(a.dout, 16) &&
           dgm::aligned(a.probs, 16) && dgm::aligned(a.dq, 16) && dgm::aligned(a.dk, 16) && dgm::aligned(a.dv, 16) &&
           dgm::aligned(a.dprobs, 16);
}

// ---- rope_bwd (metal/kernels.metal:891-909) --------------------------------------
__global__ __launch_bounds__(kThreads) void rope_bwd_kernel(const float* __restrict__ dy, float* __restrict__ dx,
                                                            const float* __restrict__ cosv,
                                                            const float* __restrict__ sinv, int B, int T, int H,
                                                            int D) {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= int64_t(B) * T * H * D) return;
    const int d = int(i % D);
    const int mid = D >> 1;
    const int t = int((i / (int64_t(H) * D)) % T);
    const float c = cosv[t * D + d], s = sinv[t * D + d];
    if (d < mid) dx[i] = dy[i] * c + dy[i + mid] * s;
    else dx[i] = dy[i] * c - dy[i - mid] * s;
}

// ---- swiglu_bwd (metal/kernels.metal:932-949) ------------------------------------
// Outputs in rows of ldo floats (ldo == F: the contiguous [n] layout; 2F with
// dup = dgate + F: the [dgate | dup] rows of a fused [gate; up] projection).
__global__ __launch_bounds__(kThreads) void swiglu_bwd_kernel(const float* __restrict__ gate,
                                                              const float* __restrict__ up,
                                                              const float* __restrict__ dy, float* dgate, float* dup,
                                                              int64_t n, int64_t F, int64_t ldo) {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    const int64_t o = ldo == F ? i : (i / F) * ldo + i % F;
    dgm::swiglu_bwd_value(gate[i], up[i], dy[i], dgate[o], dup[o]);
}

// ---- gradients of q / k / v before their projections, one wave per token row ----
// From the attention's dq, dk, dv ([B*T, H*D]): dq through RoPE (rope_bwd);
// dk summed over heads (sum_heads) then through RoPE with one head; dv summed
// over heads, then through the value residual: loop 0 (vmix == 0) dvpre =
// dv1 + dfirst (copy_f, acc_f), later loops dvpre = mix(dv1, dv1, 1 - mix, 0)
// and dfirst += mix * dv1 (mix_f, acc_scale_f). Every element is computed
// with those kernels' formulas in their order, so the outputs equal the
// sequence bitwise. Each output has its own row stride (the three blocks of
// [q | k | v] rows, or three separate buffers).
__global__ __launch_bounds__(kThreads) void qkv_grad_kernel(const float* __restrict__ dq, const float* __restrict__ dk,
                                                            const float* __restrict__ dv,
                                                            const float* __restrict__ cosv,
                                                            const float* __restrict__ sinv, float* oq, int ldq,
                                                            float* ok, int ldk, float* ov, int ldv,
                                                            float* __restrict__ dfirst, int rows, int T, int H, int D,
                                                            int vmix, float ca, float mixc) {
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int t = row % T, C = H * D, mid = D >> 1;
    const float* q = dq + size_t(row) * C;
    const float* cr = cosv + size_t(t) * D;
    const float* sr = sinv + size_t(t) * D;
    for (int e = lane; e < C; e += 64) {
        const int d = e % D;
        const float c = cr[d], s = sr[d];
        oq[size_t(row) * ldq + e] = d < mid ? q[e] * c + q[e + mid] * s : q[e] * c - q[e - mid] * s;
    }
    const float* kr = dk + size_t(row) * C;
    const float* vr = dv + size_t(row) * C;
    for (int d = lane; d < D; d += 64) {
        const int pd = d < mid ? d + mid : d - mid;
        float a = 0.0f, b = 0.0f, v = 0.0f;
        int h = 0;
        for (; h + 4 <= H; h += 4) {   // loads of four heads in flight, sums in head order
            float ka[4], kb[4], vv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                ka[u] = kr[(h + u) * D + d];
                kb[u] = kr[(h + u) * D + pd];
                vv[u] = vr[(h + u) * D + d];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a += ka[u];
                b += kb[u];
                v += vv[u];
            }
        }
        for (; h < H; ++h) {
            a += kr[h * D + d];
            b += kr[h * D + pd];
            v += vr[h * D + d];
        }
        const float c = cr[d], s = sr[d];
        ok[size_t(row) * ldk + d] = d < mid ? a * c + b * s : a * c - b * s;
        float* f = dfirst + size_t(row) * D + d;
        if (vmix == 0) {
            ov[size_t(row) * ldv + d] = v + *f;
        } else {
            const float p = ca * v;
            const float r = 0.0f * v;
            ov[size_t(row) * ldv + d] = p + r;
            *f += mixc * v;
        }
    }
}

// ---- sum_heads (metal/kernels.metal:995-1010) --------------------------------------
__global__ __launch_bounds__(kThreads) void sum_heads_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                             int B, int T, int H, int D) {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= int64_t(B) * T * D) return;
    const int d = int(i % D);
    const int64_t bt = i / D;
    const float* p = src + bt * H * D + d;
    float acc = 0.0f;
    for (int h = 0; h < H; ++h) acc += p[int64_t(h) * D];
    dst[i] = acc;
}

// ---- acc_f / acc_scale_f (metal/kernels.metal:429-436, 970-977) --------------------
template <bool SCALED>
__global__ __launch_bounds__(kThreads) void acc_kernel(float* __restrict__ a, const float* __restrict__ b, int64_t n,
                                                       float s) {
    const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    if (SCALED) a[i] += s * b[i];
    else a[i] += b[i];
}

inline unsigned blocks_for(int64_t n) { return unsigned((n + kThreads - 1) / kThreads); }
bool bad_count(int64_t n) { return n < 0 || n > dgm::kMaxIndex; }

// dx must not alias x or dy; `add` may alias dx.
int launch_rms_bwd(dgm_gpu* g, const float* x, const float* rstd, const float* w, const float* dy, float* dx,
                   float* dweight, int64_t rows, int64_t cols, const float* add = nullptr) {
    if (rows == 0 || cols == 0) return DGM_OK;
    const int ndx = int((rows + kDwWaves - 1) / kDwWaves), ndw = int((cols + 63) / 64);
    hipLaunchKernelGGL(rms_bwd_kernel, dim3(unsigned(ndx + ndw)), dim3(64 * kDwWaves), 0, g->stream, x, rstd, w, dy,
                       dx, add, dweight, int(rows), int(cols), ndx);
    return dgm::check_launch(g, "rms_bwd");
}

// a.ndx / a.ndw / a.ndd are filled in here; a.dw_tiles (0: none) and a.dw_tiles_n by the caller.
int launch_rms_chain(dgm_gpu* g, RmsChainArgs a) {
    if (a.rows == 0 || a.cols == 0) return DGM_OK;
    a.ndx = (a.rows + kDwWaves - 1) / kDwWaves;
    a.ndw = (a.cols + 63) / 64;
    a.ndd = (a.cols + 7) / 8;
    hipLaunchKernelGGL(rms_bwd_chain_kernel, dim3(unsigned(a.ndx + a.ndd + a.ndw * a.npend + a.dw_tiles)),
                       dim3(64 * kDwWaves), 0, g->stream, a);
    return dgm::check_launch(g, "rms_bwd");
}

int launch_attn_bwd(dgm_gpu* g, const AttnBwdArgs& a) {
    const int64_t n = int64_t(a.B) * a.T * a.H * a.D, tt = int64_t(a.B) * a.H * a.T * a.T;
    if (n == 0) return DGM_OK;
    if (attn_split_ok(a)) {
        const unsigned grid = unsigned(a.B * a.H * (a.T / kAsRows));
        hipLaunchKernelGGL(attn_bwd_rows_kernel, dim3(grid), dim3(kAsThreads), attn_split_rows_lds(a.T, a.D),
                           g->stream, a);
        hipLaunchKernelGGL(attn_bwd_keys_kernel, dim3(grid), dim3(kAsThreads), attn_split_keys_lds(a.T, a.D),
                           g->stream, a);
        return dgm::check_launch(g, "attn_bwd");
    }
    if (attn_bwd_fused_ok(a)) {
        const size_t lds = attn_bwd_fused_lds(a.T, a.D);
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_bwd_fused_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess)
            return dgm::fail(g, DGM_ERR_HIP, "attn_bwd: cannot reserve %zu bytes of LDS: %s", lds,
                             hipGetErrorString(e));
        hipLaunchKernelGGL(attn_bwd_fused_kernel, dim3(unsigned(a.B * a.H)), dim3(kAbThreads), lds, g->stream, a);
        return dgm::check_launch(g, "attn_bwd");
    }
    hipLaunchKernelGGL(attn_bwd_dv_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, a);
    hipLaunchKernelGGL(attn_bwd_dp_kernel, dim3(blocks_for(tt)), dim3(kThreads), 0, g->stream, a);
    hipLaunchKernelGGL(attn_softmax_bwd_kernel, dim3(blocks_for(int64_t(a.B) * a.H * a.T)), dim3(kThreads), 0,
                       g->stream, a);
    hipLaunchKernelGGL(attn_bwd_dqk_kernel<true>, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, a);
    hipLaunchKernelGGL(attn_bwd_dqk_kernel<false>, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, a);
    return dgm::check_launch(g, "attn_bwd");
}

int launch_rope_bwd(dgm_gpu* g, const float* dy, float* dx, const float* c, const float* s, int B, int T, int H,
                    int D) {
    const int64_t n = int64_t(B) * T * H * D;
    if (n == 0) return DGM_OK;
    hipLaunchKernelGGL(rope_bwd_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, dy, dx, c, s, B, T, H, D);
    return dgm::check_launch(g, "rope_bwd");
}

int launch_swiglu_bwd(dgm_gpu* g, const float* gate, const float* up, const float* dy, float* dgate, float* dup,
                      int64_t n, int64_t F = 0, int64_t ldo = 0) {
    if (n == 0) return DGM_OK;
    if (ldo == 0) F = ldo = n;
    hipLaunchKernelGGL(swiglu_bwd_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, gate, up, dy, dgate,
                       dup, n, F, ldo);
    return dgm::check_launch(g, "swiglu_bwd");
}

int launch_qkv_grad(dgm_gpu* g, const float* dq, const float* dk, const float* dv, const float* c, const float* s,
                    float* oq, int ldq, float* ok, int ldk, float* ov, int ldv, float* dfirst, int B, int T, int H,
                    int D, bool first_loop, float mix) {
    const int rows = B * T;
    if (rows == 0 || H == 0 || D == 0) return DGM_OK;
    constexpr int per = kThreads / 64;
    hipLaunchKernelGGL(qkv_grad_kernel, dim3(unsigned((rows + per - 1) / per)), dim3(kThreads), 0, g->stream, dq, dk,
                       dv, c, s, oq, ldq, ok, ldk, ov, ldv, dfirst, rows, T, H, D, first_loop ? 0 : 1, 1.0f - mix,
                       mix);
    return dgm::check_launch(g, "qkv_grad");
}

int launch_sum_heads(dgm_gpu* g, const float* src, float* dst, int B, int T, int H, int D) {
    const int64_t n = int64_t(B) * T * D;
    if (n == 0) return DGM_OK;
    hipLaunchKernelGGL(sum_heads_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, src, dst, B, T, H, D);
    return dgm::check_launch(g, "sum_heads");
}

int launch_acc(dgm_gpu* g, float* a, const float* b, int64_t n, float s, bool scaled) {
    if (n == 0) return DGM_OK;
    if (scaled)
        hipLaunchKernelGGL(acc_kernel<true>, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, a, b, n, s);
    else
        hipLaunchKernelGGL(acc_kernel<false>, dim3(blocks_for(n)), dim3(kThreads), 0, g->stream, a, b, n, s);
    return dgm::check_launch(g, scaled ? "acc_scale_f" : "acc_f");
}

int check_bthd(dgm_gpu* g, const char* name, int64_t B, int64_t T, int64_t H, int64_t D) {
    if (B < 0 || T < 0 || H < 0 || D < 0) return dgm::fail(g, DGM_ERR_ARG, "%s: negative size", name);
    if (bad_count(B * T * H * D) || bad_count(B * H * T * T))
        return dgm::fail(g, DGM_ERR_UNSUPPORTED, "%s: sizes beyond 2^31 elements", name);
    return DGM_OK;
}

// ---- block layout ----------------------------------------------------------------
// Saved activations of one loop (the reference's Acts, src/DiT.swift:260-300),
// then the forward's shared scratch.
enum { A_X, A_LN1, A_R1, A_Q, A_K, A_V, A_PROBS, A_AV, A_ATTN, A_R1B, A_MID, A_LN2, A_R2, A_GATE, A_UP, A_SW,
       A_MLP, A_R2B, A_PRE, A_RF, A_COUNT };
// F_PART: the three-launch loop's wdown slabs (empty when the shape is not built for it).
enum { F_QPRE, F_KPRE, F_VPRE, F_VFIRST, F_VMIX, F_KROT, F_SCORES, F_T1, F_PART, F_COUNT };
// Backward scratch.
// B_DG, B_DU back to back hold [M, 2F] rows [dgate | dup] and B_QPRE, B_KPRE,
// B_DVPRE [M, C + 2 KV] rows [dq | dk | dv] when the linears are fused.
// B_RPA / B_RPB / B_RPC: per-16-row-block sums of the chained RMSNorm
// backwards' later-stage weight gradients (n2b, n1b, nf), reduced by the next
// chain launch.
enum { B_T1, B_T2, B_DLN, B_DSW, B_DG, B_DU, B_DAV, B_DQ, B_DK, B_DV, B_DPROBS, B_DSCORES, B_DK1, B_DV1,
       B_DFIRST, B_QPRE, B_KPRE, B_DVPRE, B_RPA, B_RPB, B_RPC, B_CT, B_ST, B_COUNT };
// B_CT / B_ST: the four stacked linears' codes (int8) and scales transposed
// for the bf16 dX of gemm_bwd_fold ([wq; wk; wv], wo, [wgate; wup], wdown in
// that order), empty when the backward does not use it.

inline int64_t pad64(int64_t n) { return (n + 63) & ~int64_t(63); }

// The four stacked linears of the bf16-dX backward: (N, K) of [wq; wk; wv],
// wo, [wgate; wup], wdown; false when the config does not take it.
bool fold_shapes(const dgm_dit_cfg* c, int (*nk)[2]) {
    if (!c || (c->bits != 8 && c->bits != 4) || c->B <= 0 || c->T <= 0) return false;
    const int M = c->B * c->T, C = c->C, F = c->F, KV = c->D;
    const int v[4][2] = {{C + 2 * KV, C}, {C, C}, {2 * F, C}, {C, F}};
    for (int i = 0; i < 4; ++i) {
        if (!dgm::bwd_fold_ok(M, v[i][0], v[i][1], c->group)) return false;
        nk[i][0] = v[i][0];
        nk[i][1] = v[i][1];
    }
    return true;
}

// Bytes of transposed codes and floats of transposed scales (each linear's
// block padded to 256 bytes).
void fold_sizes(const dgm_dit_cfg* c, int64_t* code_bytes, int64_t* scale_floats) {
    int nk[4][2];
    *code_bytes = *scale_floats = 0;
    if (!fold_shapes(c, nk)) return;
    for (int i = 0; i < 4; ++i) {
        *code_bytes += (int64_t(nk[i][0]) * nk[i][1] + 255) & ~int64_t(255);
        *scale_floats += pad64(int64_t(nk[i][0]) * (nk[i][1] / c->group));
    }
}

void act_sizes(const dgm_dit_cfg* c, int64_t* a, int64_t* f) {
    const int64_t M = int64_t(c->B) * c->T, C = c->C, F = c->F, KV = c->D;
    const int64_t att = int64_t(c->B) * c->H * c->T * c->T;
    const int64_t av[A_COUNT] = {M * C, M * C, M, M * C, M * C, M * C, att, M * C, M * C, M,
                                 M * C, M * C, M, M * F, M * F, M * F, M * C, M, M * C, M};
    const int64_t fv[F_COUNT] = {M * C, M * KV, M * KV, M * KV, M * KV, M * KV, att, M * C,
                                 dgm::dit_loop_part_floats(c)};
    for (int i = 0; i < A_COUNT; ++i) a[i] = pad64(av[i]);
    for (int i = 0; i < F_COUNT; ++i) f[i] = pad64(fv[i]);
}

void bwd_sizes(const dgm_dit_cfg* c, int64_t* b) {
    const int64_t M = int64_t(c->B) * c->T, C = c->C, F = c->F, KV = c->D;
    const int64_t att = int64_t(c->B) * c->H * c->T * c->T;
    const int64_t RP = (M + kDwWaves - 1) / kDwWaves * C;
    int64_t ct = 0, st = 0;
    fold_sizes(c, &ct, &st);
    const int64_t bv[B_COUNT] = {M * C, M * C, M * C, M * F, M * F, M * F, M * C,  M * C,  M * C, M * C,
                                 att,   att,   M * KV, M * KV, M * KV, M * C, M * KV, M * KV, RP,    RP,
                                 RP,    (ct + 3) / 4, st};
    for (int i = 0; i < B_COUNT; ++i) b[i] = pad64(bv[i]);
}

int64_t acts_floats(const dgm_dit_cfg* c) {
    int64_t a[A_COUNT], f[F_COUNT], per = 0, tot = 0;
    act_sizes(c, a, f);
    for (int i = 0; i < A_COUNT; ++i) per += a[i];
    for (int i = 0; i < F_COUNT; ++i) tot += f[i];
    return per * c->loops + tot;
}

int64_t bwd_floats(const dgm_dit_cfg* c) {
    int64_t b[B_COUNT], tot = 0;
    bwd_sizes(c, b);
    for (int i = 0; i < B_COUNT; ++i) tot += b[i];
    return tot;
}

// Shared validation of the block entry points.
int check_cfg(dgm_gpu* g, const char* name, const dgm_dit_cfg* c, const dgm_dit_weights* w, bool need_master) {
    if (!c || !w) return dgm::fail(g, DGM_ERR_ARG, "%s: null argument", name);
    if (c->bits != 4 && c->bits != 8 && c->bits != 32)
        return dgm::fail(g, DGM_ERR_BITS, "%s: unsupported bits %d", name, c->bits);
    if (c->B <= 0 || c->T <= 0 || c->C <= 0 || c->F <= 0 || c->H <= 0 || c->D <= 0 || c->loops < 0 ||
        c->loops > 64 || c->H * c->D != c->C || c->D % 2 != 0)
        return dgm::fail(g, DGM_ERR_SHAPE, "%s: bad config (C must be H*D, D even, loops <= 64)", name);
    if (c->bits != 32 && (c->group <= 0 || c->C % c->group != 0 || c->F % c->group != 0 ||
                          (c->bits == 4 && c->group % 2 != 0)))
        return dgm::fail(g, DGM_ERR_SHAPE, "%s: C and F must be multiples of an (even for int4) group", name);
    if (bad_count(int64_t(c->B) * c->T * (c->C + 2 * c->F)) || bad_count(int64_t(c->B) * c->H * c->T * c->T))
        return dgm::fail(g, DGM_ERR_UNSUPPORTED, "%s: activations beyond 2^31 elements", name);
    const dgm_dit_linear* lins[7] = {&w->wq, &w->wk, &w->wv, &w->wo, &w->wgate, &w->wup, &w->wdown};
    for (const dgm_dit_linear* L : lins) {
        if (c->bits == 32 ? !L->w : (!L->q || !L->scale)) return dgm::fail(g, DGM_ERR_ARG, "%s: null weight", name);
        (void)need_master;
    }
    if (!w->n1 || !w->n1b || !w->n2 || !w->n2b || !w->nf) return dgm::fail(g, DGM_ERR_ARG, "%s: null norm", name);
    return DGM_OK;
}

}  // namespace

#define DGM_TRY(expr)                \
    do {                             \
        int _r = (expr);             \
        if (_r != DGM_OK) return _r; \
    } while (0)

extern "C" {

int dgm_rmsBwd(dgm_gpu* g, const float* x, const float* rstd, const float* weight, const float* dy, float* dx,
               float* dweight, int64_t rows, int64_t cols, float eps) {
    (void)eps;   // GPU.rmsBwd passes eps; the backward uses the saved rstd
    int rc = dgm::enter(g, "rmsnorm_bwd");
    if (rc) return rc;
    if (rows < 0 || cols < 0 || bad_count(rows * cols)) return dgm::fail(g, DGM_ERR_ARG, "rmsBwd: bad sizes");
    if (rows * cols && (!x || !rstd || !weight || !dy || !dx || !dweight))
        return dgm::fail(g, DGM_ERR_ARG, "rmsBwd: null buffer");
    return launch_rms_bwd(g, x, rstd, weight, dy, dx, dweight, rows, cols);
}

int dgm_attnBwd(dgm_gpu* g, const float* q, const float* k, const float* v, const float* probs, const float* dout,
                float* dq, float* dk, float* dv, float* dprobs, float* dscores, int64_t B, int64_t T, int64_t H,
                int64_t D) {
    int rc = dgm::enter(g, "attn_bwd");
    if (rc) return rc;
    DGM_TRY(check_bthd(g, "attnBwd", B, T, H, D));
    if (B * T * H * D && (!q || !k || !v || !probs || !dout || !dq || !dk || !dv || !dprobs || !dscores))
        return dgm::fail(g, DGM_ERR_ARG, "attnBwd: null buffer");
    AttnBwdArgs a{q, k, v, probs, dout, dq, dk, dv, dprobs, dscores, int(B), int(T), int(H), int(D),
                  D > 0 ? 1.0f / sqrtf(float(D)) : 0.0f};
    return launch_attn_bwd(g, a);
}

int dgm_ropeBwd(dgm_gpu* g, const float* dy, float* dx, const float* cos_t, const float* sin_t, int64_t B,
                int64_t T, int64_t H, int64_t D) {
    int rc = dgm::enter(g, "rope_bwd");
    if (rc) return rc;
    DGM_TRY(check_bthd(g, "ropeBwd", B, T, H, D));
    if (D % 2) return dgm::fail(g, DGM_ERR_SHAPE, "ropeBwd: head dim must be even");
    if (B * T * H * D && (!dy || !dx || !cos_t || !sin_t)) return dgm::fail(g, DGM_ERR_ARG, "ropeBwd: null buffer");
    return launch_rope_bwd(g, dy, dx, cos_t, sin_t, int(B), int(T), int(H), int(D));
}

int dgm_swigluBwd(dgm_gpu* g, const float* gate, const float* up, const float* dy, float* dgate, float* dup,
                  int64_t n) {
    int rc = dgm::enter(g, "swiglu_bwd");
    if (rc) return rc;
    if (bad_count(n)) return dgm::fail(g, DGM_ERR_ARG, "swigluBwd: bad count");
    if (n && (!gate || !up || !dy || !dgate || !dup)) return dgm::fail(g, DGM_ERR_ARG, "swigluBwd: null buffer");
    return launch_swiglu_bwd(g, gate, up, dy, dgate, dup, n);
}

int dgm_sumHeads(dgm_gpu* g, const float* src, float* dst, int64_t B, int64_t T, int64_t H, int64_t D) {
    int rc = dgm::enter(g, "sum_heads");
    if (rc) return rc;
    DGM_TRY(check_bthd(g, "sumHeads", B, T, H, D));
    if (B * T * D && (!src || !dst)) return dgm::fail(g, DGM_ERR_ARG, "sumHeads: null buffer");
    return launch_sum_heads(g, src, dst, int(B), int(T), int(H), int(D));
}

int dgm_acc(dgm_gpu* g, float* a, const float* b, int64_t n) {
    int rc = dgm::enter(g, "acc_f");
    if (rc) return rc;
    if (bad_count(n)) return dgm::fail(g, DGM_ERR_ARG, "acc: bad count");
    if (n && (!a || !b)) return dgm::fail(g, DGM_ERR_ARG, "acc: null buffer");
    return launch_acc(g, a, b, n, 1.0f, false);
}

int dgm_accScale(dgm_gpu* g, float* a, const float* b, int64_t n, float s) {
    int rc = dgm::enter(g, "acc_scale_f");
    if (rc) return rc;
    if (bad_count(n)) return dgm::fail(g, DGM_ERR_ARG, "accScale: bad count");
    if (n && (!a || !b)) return dgm::fail(g, DGM_ERR_ARG, "accScale: null buffer");
    return launch_acc(g, a, b, n, s, true);
}

int64_t dgm_dit_acts_floats(const dgm_dit_cfg* c) {
    if (!c || c->loops < 0 || c->B <= 0 || c->T <= 0) return -1;
    return acts_floats(c);
}

int64_t dgm_dit_backward_ws_floats(const dgm_dit_cfg* c) {
    if (!c || c->B <= 0 || c->T <= 0) return -1;
    return bwd_floats(c);
}

int dgm_dit_forward_train(dgm_gpu* g, const dgm_dit_cfg* c, const dgm_dit_weights* w, const float* cosv,
                          const float* sinv, float* x, float* acts, int64_t acts_n) {
    int rc = dgm::enter(g, "dit_forward_train");
    if (rc) return rc;
    DGM_TRY(check_cfg(g, "dit_forward_train", c, w, false));
    if (!x || !acts || !cosv || !sinv) return dgm::fail(g, DGM_ERR_ARG, "dit_forward_train: null buffer");
    if (acts_n < acts_floats(c)) return dgm::fail(g, DGM_ERR_ARG, "dit_forward_train: activation buffer too small");
    int64_t asz[A_COUNT], fsz[F_COUNT];
    act_sizes(c, asz, fsz);
    const int L = c->loops;
    float* cur = acts;
    auto A = [&](int l, int i) {
        float* p = acts;
        for (int j = 0; j < l; ++j)
            for (int k = 0; k < A_COUNT; ++k) p += asz[k];
        for (int k = 0; k < i; ++k) p += asz[k];
        return p;
    };
    for (int l = 0; l < L; ++l)
        for (int k = 0; k < A_COUNT; ++k) cur += asz[k];
    float* S[F_COUNT];
    for (int i = 0; i < F_COUNT; ++i) {
        S[i] = cur;
        cur += fsz[i];
    }
    // Fused loop-body kernels (five launches per loop, as the inference
    // forward) storing every activation the backward reads, when the weights
    // are laid out back to back; otherwise one kernel per wrapper below.
    {
        dgm::DitSaves sv[64];
        for (int l = 0; l < L; ++l) {
            sv[l] = dgm::DitSaves{A(l, A_X),   A(l, A_LN1), A(l, A_R1),   A(l, A_Q),   A(l, A_K),
                                  A(l, A_V),   A(l, A_PROBS), A(l, A_AV), A(l, A_ATTN), A(l, A_R1B),
                                  A(l, A_MID), A(l, A_LN2), A(l, A_R2),   A(l, A_GATE), A(l, A_UP),
                                  A(l, A_SW),  A(l, A_MLP), A(l, A_R2B),  A(l, A_PRE), A(l, A_RF)};
        }
        // Three launches per loop when the shape is built for it.
        bool loop2 = dgm::dit_loop_ok(c, w) && dgm::aligned(x, 16);
        for (int l = 0; loop2 && l < L; ++l)
            for (const float* p : {sv[l].x, sv[l].ln1, sv[l].mlp, sv[l].pre})
                if (!dgm::aligned(p, 16)) loop2 = false;
        if (loop2) {
            const dgm::DitLoopBufs buf{S[F_PART], S[F_VFIRST], nullptr, nullptr, nullptr, {nullptr, nullptr}, nullptr,
                                       nullptr};
            return dgm::dit_forward_loops(g, c, w, cosv, sinv, x, buf, sv);
        }
        int64_t fn = 0;
        for (int i = 0; i < F_PART; ++i) fn += fsz[i];
        const int r = dgm::dit_forward_train_fused(g, c, w, cosv, sinv, x, sv, S[0], fn);
        if (r != dgm::kNotFused) return r;
    }
    const int B = c->B, T = c->T, H = c->H, D = c->D, bits = c->bits, G = c->group;
    const int64_t M = int64_t(B) * T, C = c->C, F = c->F, KV = D, nC = M * C, nKV = M * KV;
    const float mix = c->mix;
    auto lin = [&](const dgm_dit_linear& Lw, const float* in, float* out, int64_t N, int64_t K) {
        return dgm_gemmNT(g, bits, Lw.w, Lw.q, Lw.scale, in, nullptr, out, M, N, K, bits == 32 ? 8 : G);
    };
    for (int l = 0; l < L; ++l) {
        float* X = A(l, A_X);
        if (l == 0) DGM_TRY(dgm_copy(g, x, X, nC));
        DGM_TRY(dgm_rmsFwd(g, X, A(l, A_LN1), A(l, A_R1), w->n1, M, C, c->eps));
        DGM_TRY(lin(w->wq, A(l, A_LN1), S[F_QPRE], C, C));
        DGM_TRY(lin(w->wk, A(l, A_LN1), S[F_KPRE], KV, C));
        DGM_TRY(lin(w->wv, A(l, A_LN1), S[F_VPRE], KV, C));
        if (l == 0) {
            DGM_TRY(dgm_copy(g, S[F_VPRE], S[F_VFIRST], nKV));
            DGM_TRY(dgm_repeatHeads(g, S[F_VPRE], A(l, A_V), B, T, H, D));
        } else {
            DGM_TRY(dgm_mix(g, S[F_VPRE], S[F_VFIRST], S[F_VMIX], nKV, 1.0f - mix, mix));
            DGM_TRY(dgm_repeatHeads(g, S[F_VMIX], A(l, A_V), B, T, H, D));
        }
        DGM_TRY(dgm_ropeFwd(g, S[F_QPRE], A(l, A_Q), cosv, sinv, B, T, H, D));
        DGM_TRY(dgm_ropeFwd(g, S[F_KPRE], S[F_KROT], cosv, sinv, B, T, 1, D));
        DGM_TRY(dgm_repeatHeads(g, S[F_KROT], A(l, A_K), B, T, H, D));
        DGM_TRY(dgm_attnFwd(g, A(l, A_Q), A(l, A_K), A(l, A_V), S[F_SCORES], A(l, A_PROBS), A(l, A_AV), B, T, H, D,
                            0));
        DGM_TRY(lin(w->wo, A(l, A_AV), A(l, A_ATTN), C, C));
        DGM_TRY(dgm_rmsFwd(g, A(l, A_ATTN), S[F_T1], A(l, A_R1B), w->n1b, M, C, c->eps));
        DGM_TRY(dgm_add(g, X, S[F_T1], A(l, A_MID), nC));
        DGM_TRY(dgm_rmsFwd(g, A(l, A_MID), A(l, A_LN2), A(l, A_R2), w->n2, M, C, c->eps));
        DGM_TRY(lin(w->wgate, A(l, A_LN2), A(l, A_GATE), F, C));
        DGM_TRY(lin(w->wup, A(l, A_LN2), A(l, A_UP), F, C));
        DGM_TRY(dgm_swigluFwd(g, A(l, A_GATE), A(l, A_UP), A(l, A_SW), M * F));
        DGM_TRY(lin(w->wdown, A(l, A_SW), A(l, A_MLP), C, F));
        DGM_TRY(dgm_rmsFwd(g, A(l, A_MLP), S[F_T1], A(l, A_R2B), w->n2b, M, C, c->eps));
        DGM_TRY(dgm_add(g, A(l, A_MID), S[F_T1], A(l, A_PRE), nC));
        DGM_TRY(dgm_rmsFwd(g, A(l, A_PRE), l + 1 < L ? A(l + 1, A_X) : x, A(l, A_RF), w->nf, M, C, c->eps));
    }
    return DGM_OK;
}

int dgm_dit_backward(dgm_gpu* g, const dgm_dit_cfg* c, const dgm_dit_weights* w, const dgm_dit_grads* gr,
                     const float* cosv, const float* sinv, const float* acts, int64_t acts_n, float* gx, float* ws,
                     int64_t ws_n) {
    int rc = dgm::enter(g, "dit_backward");
    if (rc) return rc;
    DGM_TRY(check_cfg(g, "dit_backward", c, w, true));
    if (!gr || !acts || !gx || !ws || !cosv || !sinv) return dgm::fail(g, DGM_ERR_ARG, "dit_backward: null buffer");
    float* const gws[7] = {gr->wq, gr->wk, gr->wv, gr->wo, gr->wgate, gr->wup, gr->wdown};
    float* const gns[5] = {gr->n1, gr->n1b, gr->n2, gr->n2b, gr->nf};
    for (float* p : gws)
        if (!p) return dgm::fail(g, DGM_ERR_ARG, "dit_backward: null weight gradient");
    for (float* p : gns)
        if (!p) return dgm::fail(g, DGM_ERR_ARG, "dit_backward: null norm gradient");
    if (acts_n < acts_floats(c)) return dgm::fail(g, DGM_ERR_ARG, "dit_backward: activation buffer too small");
    if (ws_n < bwd_floats(c)) return dgm::fail(g, DGM_ERR_ARG, "dit_backward: workspace too small");
    // The loop shapes' forward keeps k and v of the KV head only, which the
    // one-launch attention backward reads; it needs 16-byte aligned buffers.
    if (dgm::dit_loop_shape_ok(c) && !dgm::dit_attn_bwd_loop_ok(c, acts, ws))
        return dgm::fail(g, DGM_ERR_ARG, "dit_backward: acts and ws must be 16-byte aligned");
    int64_t asz[A_COUNT], fsz[F_COUNT], bsz[B_COUNT];
    act_sizes(c, asz, fsz);
    bwd_sizes(c, bsz);
    auto A = [&](int l, int i) {
        const float* p = acts;
        for (int j = 0; j < l; ++j)
            for (int k = 0; k < A_COUNT; ++k) p += asz[k];
        for (int k = 0; k < i; ++k) p += asz[k];
        return p;
    };
    float* S[B_COUNT];
    float* cur = ws;
    for (int i = 0; i < B_COUNT; ++i) {
        S[i] = cur;
        cur += bsz[i];
    }
    const int B = c->B, T = c->T, H = c->H, D = c->D, bits = c->bits, G = c->group;
    const int64_t M = int64_t(B) * T, C = c->C, F = c->F, KV = D, nC = M * C, nKV = M * KV;
    const float mix = c->mix;
    // dW accumulated into the fp32 gradient and dX through the linear (fp32
    // master for bits 32, dequantized codes for bits 8 / 4): the reference's
    // gemmDWAcc + gemmDX pair, one launch where the shapes allow.
    auto bwd = [&](const dgm_dit_linear& Lw, const float* dy, const float* in, float* out, float* dW, int64_t N,
                   int64_t K) {
        return dgm_gemmBwd(g, bits, Lw.w, Lw.q, Lw.scale, dy, in, out, dW, M, N, K, bits == 32 ? 8 : G, 1);
    };
    float *t1 = S[B_T1], *t2 = S[B_T2], *dln = S[B_DLN];
    // RMSNorm backward; with `add`, the residual gradient add (acc_f) that
    // follows it in the reference is done by the same launch.
    auto rms_bwd = [&](const float* xin, const float* rstd, const float* wt, const float* dy, float* dx,
                       float* dwt, const float* add) { return launch_rms_bwd(g, xin, rstd, wt, dy, dx, dwt, M, C, add); };
    // Where q / k / v (gate / up) weights and their gradients lie back to
    // back, one backward over the stacked [C + 2 KV, C] ([2F, C]) linear
    // replaces three (two) and the adds of their dX: dW rows are the same
    // sums, dX sums the same products in one chain.
    const bool qkv1 = dgm::dit_linear_follows(w->wq, w->wk, C, C, bits, G) &&
                      dgm::dit_linear_follows(w->wk, w->wv, KV, C, bits, G) && gr->wk == gr->wq + C * C &&
                      gr->wv == gr->wk + KV * C;
    const bool gu1 = dgm::dit_linear_follows(w->wgate, w->wup, F, C, bits, G) && gr->wup == gr->wgate + F * C;
    const int64_t QKV = qkv1 ? C + 2 * KV : 0;
    float* const qkvrow = S[B_QPRE];   // [M, C + 2 KV] rows when qkv1
    // dX on bf16 MFMA (gemm_bwd_fold) for the stacked linears: their codes
    // and scales transposed once here.
    int fnk[4][2];
    const size_t calign = bits == 8 ? 16 : 8;
    const bool fold = qkv1 && gu1 && fold_shapes(c, fnk) && dgm::aligned(ws, 16) && dgm::aligned(w->wq.q, calign) &&
                      dgm::aligned(w->wo.q, calign) && dgm::aligned(w->wgate.q, calign) &&
                      dgm::aligned(w->wdown.q, calign);
    const int8_t* fct[4] = {};
    const float* fst[4] = {};
    if (fold) {
        const dgm_dit_linear* lins[4] = {&w->wq, &w->wo, &w->wgate, &w->wdown};
        const void* Wp[4];
        const float* Sp[4];
        int8_t* ctp[4];
        float* stp[4];
        int Nn[4], Kk[4];
        int8_t* cc = reinterpret_cast<int8_t*>(S[B_CT]);
        float* sc = S[B_ST];
        for (int i = 0; i < 4; ++i) {
            Wp[i] = lins[i]->q;
            Sp[i] = lins[i]->scale;
            Nn[i] = fnk[i][0];
            Kk[i] = fnk[i][1];
            ctp[i] = cc;
            stp[i] = sc;
            fct[i] = cc;
            fst[i] = sc;
            cc += (int64_t(Nn[i]) * Kk[i] + 255) & ~int64_t(255);
            sc += pad64(int64_t(Nn[i]) * (Kk[i] / G));
        }
        DGM_TRY(dgm::wt_prep(g, bits, 4, Wp, Sp, Nn, Kk, G, ctp, stp));
    }
    // gemmBwd of stacked linear li (0 [wq; wk; wv], 1 wo, 2 [wgate; wup],
    // 3 wdown) on the bf16-dX pair when `fold`, else the fp32 pair.
    auto bwdf = [&](int li, const dgm_dit_linear& Lw, const float* dy, const float* in, float* out, float* dW,
                    int64_t N, int64_t K) -> int {
        if (fold) {
            const int r = dgm::gemm_bwd_fold(g, fct[li], fst[li], dy, in, out, dW, int(M), int(N), int(K), G, true,
                                             nullptr, nullptr);
            if (r != dgm::kNotFused) return r;
        }
        return bwd(Lw, dy, in, out, dW, N, K);
    };
    // The RMSNorm backwards that follow each other run as one chained launch
    // when C <= 256: nf + n2b, n2 + n1b, and n1 together with the next loop's
    // nf + n2b. A later stage's weight gradient is summed per row block (RPA:
    // n2b, RPB: n1b, RPC: nf) and added by the next chain launch.
    const bool chain = C <= kChainCols;
    const int nrb = int((M + kDwWaves - 1) / kDwWaves);
    auto stage = [](const float* x, const float* r, const float* wt, float* out, const float* add, float* part) {
        RmsStage st{};
        st.x = x; st.r = r; st.w = wt; st.out = out; st.add = add; st.part = part;
        return st;
    };
    auto run_chain = [&](const float* dy, float* dw0, int nst, const RmsStage* st, int npend, const float* pin0,
                         float* dwp0, const float* pin1, float* dwp1, const dgm_dw::DwTileArgs* dw = nullptr) {
        RmsChainArgs ra{};
        if (dw) {
            ra.dw = *dw;
            ra.dw_tiles = dgm_dw::dw_tiles(*dw);
            ra.dw_tiles_n = dgm_dw::dw_tiles_n(*dw);
        }
        ra.dy = dy; ra.dw0 = dw0; ra.nst = nst;
        for (int i = 0; i < nst; ++i) ra.st[i] = st[i];
        ra.npend = npend; ra.pin[0] = pin0; ra.dwp[0] = dwp0; ra.pin[1] = pin1; ra.dwp[1] = dwp1;
        ra.npin = nrb; ra.rows = int(M); ra.cols = int(C);
        return launch_rms_chain(g, ra);
    };
    // The one-launch attention backward writes dfirst in the first loop it
    // runs; the per-row gradient kernel adds to it, so it starts at zero.
    const bool attn1 = dgm::dit_attn_bwd_loop_ok(c, acts, ws);
    if (!attn1) DGM_TRY(dgm_zero(g, S[B_DFIRST], nKV));
    const int L = c->loops;
    // With the bf16-dX pair, the chained RMSNorm backwards and the one-launch
    // attention backward (which leaves the dq scratch unused), dL/dmlp lives
    // in that scratch until the loop's first chain launch, which runs wdown's
    // dW tiles beside its own work (it writes none of dL/dmlp, sw or that dW).
    const bool host_wd = fold && chain && attn1;
    float* const mlpd = host_wd ? S[B_DQ] : nullptr;
    float* dmlp = host_wd ? mlpd : t2;   // dL/dmlp of the loop about to run
    if (chain && L > 0) {
        const RmsStage st[2] = {stage(A(L - 1, A_PRE), A(L - 1, A_RF), w->nf, t1, nullptr, nullptr),
                                stage(A(L - 1, A_MLP), A(L - 1, A_R2B), w->n2b, dmlp, nullptr, S[B_RPA])};
        DGM_TRY(run_chain(gx, gr->nf, 2, st, 0, nullptr, nullptr, nullptr, nullptr));
    }
    for (int l = L - 1; l >= 0; --l) {
        if (!chain) {
            DGM_TRY(rms_bwd(A(l, A_PRE), A(l, A_RF), w->nf, gx, t1, gr->nf, nullptr));
            DGM_TRY(rms_bwd(A(l, A_MLP), A(l, A_R2B), w->n2b, t1, t2, gr->n2b, nullptr));
        }
        bool hwd = host_wd;
        const dgm_dw::DwTileArgs dwd{dmlp, A(l, A_SW), gr->wdown, int(M), int(C), int(F), 1};
        if (gu1) {
            // wdown's backward with the SwiGLU backward in its dX epilogue,
            // else the two launches.
            const int r = fold ? dgm::gemm_bwd_fold(g, fct[3], fst[3], dmlp, A(l, A_SW), S[B_DG],
                                                    hwd ? nullptr : gr->wdown, int(M), int(C), int(F), G, true,
                                                    A(l, A_GATE), A(l, A_UP))
                               : dgm::gemm_bwd_swiglu(g, bits, w->wdown.w, w->wdown.q, w->wdown.scale, dmlp,
                                                      A(l, A_SW), A(l, A_GATE), A(l, A_UP), S[B_DG], gr->wdown, M, C,
                                                      F, bits == 32 ? 8 : G);
            if (r == dgm::kNotFused) {
                hwd = false;
                DGM_TRY(bwd(w->wdown, dmlp, A(l, A_SW), S[B_DSW], gr->wdown, C, F));
                DGM_TRY(launch_swiglu_bwd(g, A(l, A_GATE), A(l, A_UP), S[B_DSW], S[B_DG], S[B_DG] + F, M * F, F,
                                          2 * F));
            } else {
                DGM_TRY(r);
            }
            DGM_TRY(bwdf(2, w->wgate, S[B_DG], A(l, A_LN2), t2, gr->wgate, 2 * F, C));
        } else {
            DGM_TRY(bwd(w->wdown, dmlp, A(l, A_SW), S[B_DSW], gr->wdown, C, F));
            DGM_TRY(launch_swiglu_bwd(g, A(l, A_GATE), A(l, A_UP), S[B_DSW], S[B_DG], S[B_DU], M * F));
            DGM_TRY(bwd(w->wgate, S[B_DG], A(l, A_LN2), t2, gr->wgate, F, C));
            DGM_TRY(bwd(w->wup, S[B_DU], A(l, A_LN2), dln, gr->wup, F, C));
            DGM_TRY(dgm_acc(g, t2, dln, nC));
        }
        // t1 += dx of n2; its n1b backward goes to dln (t2 is still being read
        // by the direct weight-gradient workgroups of the same launch).
        float* dattn = t2;
        if (chain) {
            const RmsStage st[2] = {stage(A(l, A_MID), A(l, A_R2), w->n2, t1, t1, nullptr),
                                    stage(A(l, A_ATTN), A(l, A_R1B), w->n1b, dln, nullptr, S[B_RPB])};
            if (l == L - 1)   // nf's gradient was direct in the first chain
                DGM_TRY(run_chain(t2, gr->n2, 2, st, 1, S[B_RPA], gr->n2b, nullptr, nullptr, hwd ? &dwd : nullptr));
            else
                DGM_TRY(run_chain(t2, gr->n2, 2, st, 2, S[B_RPA], gr->n2b, S[B_RPC], gr->nf, hwd ? &dwd : nullptr));
            dattn = dln;
        } else {
            DGM_TRY(rms_bwd(A(l, A_MID), A(l, A_R2), w->n2, t2, t1, gr->n2, t1));
            DGM_TRY(rms_bwd(A(l, A_ATTN), A(l, A_R1B), w->n1b, t1, t2, gr->n1b, nullptr));
        }
        // With the bf16-dX pair, the one-launch attention backward and the
        // chained RMSNorm backwards, the dW tiles of wo run in the attention
        // backward's launch and those of [wq; wk; wv] in the chain launch
        // after them, beside work that reads none of what they write and
        // writes none of what they read: their own launches are dX alone.
        const dgm_dw::DwTileArgs dwo{dattn, A(l, A_AV), gr->wo, int(M), int(C), int(C), 1};
        const dgm_dw::DwTileArgs dwq{qkvrow, A(l, A_LN1), gr->wq, int(M), int(QKV), int(C), 1};
        bool host_wo = fold && attn1 && chain, host_wq = host_wo;
        if (host_wo) {
            const int r = dgm::gemm_bwd_fold(g, fct[1], fst[1], dattn, A(l, A_AV), S[B_DAV], nullptr, int(M), int(C),
                                             int(C), G, true, nullptr, nullptr);
            if (r == dgm::kNotFused) host_wo = false;
            else DGM_TRY(r);
        }
        if (!host_wo) DGM_TRY(bwdf(1, w->wo, dattn, A(l, A_AV), S[B_DAV], gr->wo, C, C));
        // The attention backward with sum_heads of dk and dv, rope_bwd of dq
        // and dk and the value residual: one launch for the built shapes,
        // else attnBwd and the per-row gradient kernel.
        float *oq = qkv1 ? qkvrow : S[B_QPRE], *ok = qkv1 ? qkvrow + C : S[B_KPRE];
        float* ov = qkv1 ? qkvrow + C + KV : S[B_DVPRE];
        const int ldq = qkv1 ? int(QKV) : int(C), ldkv = qkv1 ? int(QKV) : int(KV);
        if (attn1) {
            const int ra = dgm::dit_attn_bwd_loop(g, c, A(l, A_Q), A(l, A_K), A(l, A_V), A(l, A_PROBS), A(l, A_AV),
                                                  S[B_DAV], cosv, sinv, oq, ldq, ok, ov, ldkv, S[B_DFIRST], l == 0,
                                                  l == L - 1, host_wo ? &dwo : nullptr);
            if (ra == dgm::kNotFused)
                return dgm::fail(g, DGM_ERR_UNSUPPORTED, "dit_backward: attention backward shape changed");
            DGM_TRY(ra);
        } else {
            DGM_TRY(dgm_attnBwd(g, A(l, A_Q), A(l, A_K), A(l, A_V), A(l, A_PROBS), S[B_DAV], S[B_DQ], S[B_DK],
                                S[B_DV], S[B_DPROBS], S[B_DSCORES], B, T, H, D));
            DGM_TRY(launch_qkv_grad(g, S[B_DQ], S[B_DK], S[B_DV], cosv, sinv, oq, ldq, ok, ldkv, ov, ldkv,
                                    S[B_DFIRST], B, T, H, D, l == 0, mix));
        }
        if (host_wq) {
            const int r = dgm::gemm_bwd_fold(g, fct[0], fst[0], qkvrow, A(l, A_LN1), t2, nullptr, int(M), int(QKV),
                                             int(C), G, true, nullptr, nullptr);
            if (r == dgm::kNotFused) host_wq = false;
            else DGM_TRY(r);
        }
        if (host_wq) {
            // dX done; its dW runs in the chain launch below.
        } else if (qkv1) {
            DGM_TRY(bwdf(0, w->wq, qkvrow, A(l, A_LN1), t2, gr->wq, QKV, C));
        } else {
            DGM_TRY(bwd(w->wq, S[B_QPRE], A(l, A_LN1), t2, gr->wq, C, C));
            DGM_TRY(bwd(w->wk, S[B_KPRE], A(l, A_LN1), dln, gr->wk, KV, C));
            DGM_TRY(dgm_acc(g, t2, dln, nC));
            DGM_TRY(bwd(w->wv, S[B_DVPRE], A(l, A_LN1), dln, gr->wv, KV, C));
            DGM_TRY(dgm_acc(g, t2, dln, nC));
        }
        if (chain) {
            // gx = t1 + dx of n1 (and the pending n1b sums); below loop 0 the
            // next loop's nf and n2b backwards follow in the same launch, its
            // dL/dmlp going to the dq scratch when wdown's dW is hosted, else
            // to dln (t2 is read by the direct workgroups).
            if (l > 0) {
                const RmsStage st[3] = {stage(A(l, A_X), A(l, A_R1), w->n1, gx, t1, nullptr),
                                        stage(A(l - 1, A_PRE), A(l - 1, A_RF), w->nf, t1, nullptr, S[B_RPC]),
                                        stage(A(l - 1, A_MLP), A(l - 1, A_R2B), w->n2b, host_wd ? mlpd : dln,
                                              nullptr, S[B_RPA])};
                DGM_TRY(run_chain(t2, gr->n1, 3, st, 1, S[B_RPB], gr->n1b, nullptr, nullptr, host_wq ? &dwq : nullptr));
                dmlp = host_wd ? mlpd : dln;
            } else {
                const RmsStage st[1] = {stage(A(l, A_X), A(l, A_R1), w->n1, gx, t1, nullptr)};
                DGM_TRY(run_chain(t2, gr->n1, 1, st, 1, S[B_RPB], gr->n1b, nullptr, nullptr, host_wq ? &dwq : nullptr));
            }
        } else {
            DGM_TRY(rms_bwd(A(l, A_X), A(l, A_R1), w->n1, t2, gx, gr->n1, t1));   // gx = t1 + dx
        }
    }
    return DGM_OK;
}

}  // extern "C"
#undef DGM_TRY
