// Looped DiT block forward in three launches per loop (src/DiT.swift:520-550),
// for the block shapes it is built for: int8 / int4 linears with group 32,
// one KV head, C a multiple of 64, F a multiple of the mlp slice (96 or 128 columns).
//
//  * loop_row_kernel: one workgroup of 16 waves per (8 rows, column group);
//    waves 8 .. 15 own a row each, waves 0 .. ntile-1 the group's projection
//    tiles (16 x 16, the MFMA's other 8 rows computed and dropped). The row
//    chain that closes the previous loop
//    (mlp = the previous loop's wdown slabs added in slab order;
//    pre = mid + rms(mlp)*n2b; x = rms(pre)*nf; loop 0: x = the input), then
//    ln1 = rms(x)*n1, and the group's columns of the [wq; wk; wv] projection
//    (HG query heads, or k | v), with RoPE on q and k and the value residual
//    on v.
//  * loop_attn_kernel: one workgroup of 16 waves per (sequence b, 16 query
//    rows, head pair, quarter of wo's output columns): scores, row softmax and
//    P.V of the pair's two heads on fp32 MFMA (the stages of attn_mfma_kernel
//    in dit.hip, each query head against the one KV head), then the pair's
//    share of av . wo^T (its 2D contraction columns) for the quarter's output
//    columns into the pair's slab; the mlp kernel adds the pairs' slabs in
//    order.
//  * loop_mlp_kernel: one workgroup of SL / 16 waves per (16 rows, slice of SL
//    SwiGLU columns): the row chain mid = x + rms(attn)*n1b and ln2 =
//    rms(mid)*n2 of its 16 rows (stored by the slice-0 workgroup), gate and up
//    of those columns, SwiGLU, and the slice's
//    share of wdown (its sum over the slice's SL contraction indices) into
//    slab `slice` of [P][M][C], P = F / SL.
//  * loop_tail_kernel after the last loop: the closing row chain.
// A sequence's workgroups run on one XCD (block b + 8 j), where the previous
// launch left its rows.
//
// Projections run on v_mfma_f32_16x16x32_bf16 with exact operands: a code is
// an integer of at most 8 bits (exact in bf16), and every activation is split
// into three bf16 pieces hi + mid + lo whose sum is the fp32 value exactly
// (hi: the top 8 significand bits, mid: the next 8 of the remainder, lo: what
// is left, at most 8 bits). Every product is exact; each 32-k group's sum is
// accumulated in fp32 (lo, mid, then hi pieces) and multiplied by the group's
// scale. RoPE, softmax, SwiGLU and the row chains use the standalone kernels'
// formulas (the chains' rstd with the hardware inverse square root, the
// softmax's and SwiGLU's exponentials as the hardware 2^x of x log2 e, within
// a few ulp of expf), so results agree with the oracle to fp32 rounding of
// the sums.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "dit_rows.hpp"

namespace {

using dgm_rows::add4;
using dgm_rows::norm4;
using dgm_rows::row16_max;
using dgm_rows::row16_sum;
using dgm_rows::wave64_sum;
using dgm_rows::rstd16;
using dgm_rows::silu_sigmoid;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// SwiGLU columns per mlp workgroup (16 per wave): 128, or 96 when that gives
// at most one workgroup per CU of the MI355X's 256 where 128 would leave CUs
// idle. A workgroup's weight codes set the kernel's time (a CU receives them
// at a bounded rate): at c3, 96 columns bring 55 KB of codes to each of 256
// CUs instead of 74 KB to each of 192. The choice depends on the shape alone,
// so the workspace size does too.
constexpr int kSlice = 128;
constexpr int64_t kSliceCus = 256;
constexpr int kRowTile = 8;           // rows per loop_row_kernel workgroup
int slice_cols(const dgm_dit_cfg* c) {
    const int64_t tiles = int64_t(c->B) * c->T / 16;
    if (c->F % 96 == 0 && tiles * (c->F / 96) <= kSliceCus && tiles * (c->F / kSlice) < kSliceCus) return 96;
    return kSlice;
}

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// x = h + m + l exactly; each piece has a zero low half (a bf16 value).
__device__ __forceinline__ void split3(float x, float& h, float& m, float& l) {
    h = __uint_as_float(__float_as_uint(x) & 0xFFFF0000u);
    const float r = x - h;
    m = __uint_as_float(__float_as_uint(r) & 0xFFFF0000u);
    l = r - m;
}

// Pieces of 4 consecutive values into planes P (hi), P + ps (mid), P + 2 ps
// (lo) at element o (o % 4 == 0).
__device__ __forceinline__ void put4(__bf16* P, int ps, int o, float4 v) {
    float h[4], m[4], l[4];
    split3(v.x, h[0], m[0], l[0]);
    split3(v.y, h[1], m[1], l[1]);
    split3(v.z, h[2], m[2], l[2]);
    split3(v.w, h[3], m[3], l[3]);
    *reinterpret_cast<uint2*>(P + o) = make_uint2(pk_bf16(h[0], h[1]), pk_bf16(h[2], h[3]));
    *reinterpret_cast<uint2*>(P + ps + o) = make_uint2(pk_bf16(m[0], m[1]), pk_bf16(m[2], m[3]));
    *reinterpret_cast<uint2*>(P + 2 * ps + o) = make_uint2(pk_bf16(l[0], l[1]), pk_bf16(l[2], l[3]));
}

__device__ __forceinline__ void put1(__bf16* P, int ps, int o, float v) {
    float h, m, l;
    split3(v, h, m, l);
    uint16_t* Q = reinterpret_cast<uint16_t*>(P);
    Q[o] = uint16_t(__float_as_uint(h) >> 16);
    Q[ps + o] = uint16_t(__float_as_uint(m) >> 16);
    Q[2 * ps + o] = uint16_t(__float_as_uint(l) >> 16);
}

// 8 consecutive codes k .. k+7 of weight row `row` ([rows, K] row-major):
// int8 as 8 bytes, int4 as 8 nibbles (low nibble first) in .x.
template <int BITS>
__device__ __forceinline__ uint2 codes_at(const void* W, size_t row, int K, int k) {
    if constexpr (BITS == 8) {
        return *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(W) + row * size_t(K) + k);
    } else {
        const uint8_t* p = static_cast<const uint8_t*>(W) + ((row * size_t(K) + size_t(k)) >> 1);
        return make_uint2(*reinterpret_cast<const uint32_t*>(p), 0u);
    }
}

template <int BITS>
__device__ __forceinline__ bf16x8 codes_bf16(uint2 w) {
    u32x4 r;
    if constexpr (BITS == 8) {
        r.x = pk_bf16(float(int8_t(w.x)), float(int8_t(w.x >> 8)));
        r.y = pk_bf16(float(int8_t(w.x >> 16)), float(int8_t(w.x >> 24)));
        r.z = pk_bf16(float(int8_t(w.y)), float(int8_t(w.y >> 8)));
        r.w = pk_bf16(float(int8_t(w.y >> 16)), float(int8_t(w.y >> 24)));
    } else {
        const uint32_t v = w.x;
        auto nib = [v](int i) { return float(int32_t(v << (28 - 4 * i)) >> 28); };
        r.x = pk_bf16(nib(0), nib(1));
        r.y = pk_bf16(nib(2), nib(3));
        r.z = pk_bf16(nib(4), nib(5));
        r.w = pk_bf16(nib(6), nib(7));
    }
    return __builtin_bit_cast(bf16x8, r);
}

// One 32-k step of a 16x16 tile: sum over the three activation pieces of
// pieces x codes. `a` is this lane's 8 k of the hi plane (row r16, k 8*q4);
// the mid and lo planes follow at +ps and +2ps.
__device__ __forceinline__ f32x4 step3(const __bf16* a, int ps, bf16x8 b) {
    const bf16x8 lo = *reinterpret_cast<const bf16x8*>(a + 2 * ps);
    const bf16x8 mi = *reinterpret_cast<const bf16x8*>(a + ps);
    const bf16x8 hi = *reinterpret_cast<const bf16x8*>(a);
    f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, b, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mi, b, t, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, b, t, 0, 0, 0);
}

__device__ __forceinline__ f32x4 scale_add(f32x4 acc, f32x4 t, float s) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(t[e], s, acc[e]);
    return acc;
}

// 16x16 tile of A . B^T over n (n % 16 == 0) fp32 contraction indices, rows in
// LDS: a at (row r16, 4*q4) of A, b at (row r16, 4*q4) of B. fp32 MFMA.
__device__ __forceinline__ f32x4 dot_tile(const float* a, const float* b, int n) {
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int d0 = 0; d0 < n; d0 += 16) {
        const float4 x = *reinterpret_cast<const float4*>(a + d0);
        const float4 y = *reinterpret_cast<const float4*>(b + d0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, y.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, y.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, y.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, y.w, acc, 0, 0, 0);
    }
    return acc;
}

// rstd of one row held by a whole wave, one float4 per lane (columns 4 lane ..
// 4 lane + 3; lanes past the row's end hold zeros): 1 / sqrt(mean(x^2) + eps).
// The mean is a product with 1/cols and the inverse square root the hardware
// one (v_rsq_f32, within 1 ulp), not the IEEE divide and square root of the
// standalone rmsnorm_fwd: the row chains here are VALU-bound, and the results
// stay within a few ulp of the correctly rounded formula.
template <int COLS>
__device__ __forceinline__ float rstd_row(float4 v, float eps) {
#pragma clang fp contract(off)
    float ss = v.x * v.x;
    ss += v.y * v.y;
    ss += v.z * v.z;
    ss += v.w * v.w;
    ss = wave64_sum(ss);
    const float mean = ss * (1.0f / float(COLS));
    return __builtin_amdgcn_rsqf(mean + eps);
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// Barrier for LDS hand-over only: waits for this wave's LDS operations, not
// for its outstanding global loads or stores (each value loaded from global
// memory is waited for where it is used).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Sequence-major block order: block i runs on XCD i % 8; the blocks of
// sequence b (items per_seq of them) take XCD b % 8. Returns false for the
// padding blocks past the last sequence.
__device__ __forceinline__ bool seq_block(int B, int per_seq, int& b, int& item) {
    const int j = int(blockIdx.x >> 3);
    b = int(blockIdx.x & 7) + 8 * (j / per_seq);
    item = j % per_seq;
    return b < B;
}

// The KS group scales of one weight row (KS consecutive floats, 8-byte
// aligned when KS is even).
template <int KS>
__device__ __forceinline__ void load_scales(const float* p, float (&s)[KS]) {
    if constexpr (KS % 2 == 0) {
#pragma unroll
        for (int i = 0; i < KS / 2; ++i) {
            const float2 v = *reinterpret_cast<const float2*>(p + 2 * i);
            s[2 * i] = v.x;
            s[2 * i + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int i = 0; i < KS; ++i) s[i] = p[i];
    }
}

// ---- loop_row_kernel ------------------------------------------------------------------
// One workgroup of 16 waves per (16 rows, column group); wave w owns row w
// (64 lanes, columns lane + 64 u). Column groups: HG query heads each, then
// one group of k | v.
struct LoopRowArgs {
    const float* x;          // loop 0: the input rows [M, C]
    const float* part;       // later loops: the previous loop's wdown slabs [P][M][C]
    const float* mid_prev;   // later loops: the previous loop's mid [M, C]
    const float *n1, *n2b, *nf;
    const void* Wqkv;        // [C + 2D, C] codes of wq, wk, wv back to back
    const float* Sqkv;
    const float *cosv, *sinv;   // [T, D]
    float* vfirst;              // [M, D]: loop 0 stores its v, later loops mix it in
    float* q;                   // [M, C] after RoPE
    float *k, *v;               // rows of kv_ld floats: k after RoPE, v after the mix,
    int kv_ld, krep;            // each written to krep heads (columns h*D)
    float* xo;                  // this loop's x [M, C] (loop 0: a copy of the input), or null
    // Optional training saves: ln1 and its rstd; the previous loop's mlp,
    // pre and their rstd.
    float *sln1, *sr1, *pmlp, *ppre, *pr2b, *prf;
    int B, T, NG, HG;
    float eps, ca, cb;
};

// FIRST: the first loop (x from the input, v stored as the value residual);
// a compile-time flag, so that no branch splits the row loads into rounds.
template <int BITS, int KS, int DT, int NP, bool FIRST>
__global__ __launch_bounds__(1024) void loop_row_kernel(LoopRowArgs a) {
#pragma clang fp contract(off)
    constexpr int C = 32 * KS, D = 16 * DT, C4 = C / 4, LDA = C + 8, OLD = 2 * D + 4;
    static_assert(C4 <= 64, "one float4 of the row per lane");
    __shared__ __align__(16) __bf16 Ap[3 * 16 * LDA];
    __shared__ __align__(16) float os[16 * OLD];
    // kRowTile rows per workgroup: the rows' slab sums are most of what a
    // workgroup reads, so 8-row tiles (the MFMA's other 8 rows computed and
    // dropped) halve what each CU receives with twice the workgroups.
    constexpr int RT = kRowTile;
    static_assert(2 * DT <= 16 - RT, "the chain waves load no codes");
    int b, item;
    if (!seq_block(a.B, (a.T / RT) * a.NG, b, item)) return;
    const int g = item % a.NG;
    const size_t row0 = size_t(b) * a.T + size_t(item / a.NG) * RT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;
    const bool kvg = g == a.NG - 1;
    const int ntile = kvg ? 2 * DT : a.HG * DT;
    const int nbase = kvg ? C : g * a.HG * D;   // first weight row (output column) of the group

    // -- loads: waves 0 .. ntile-1 their projection tile's codes and scales;
    // waves 16-RT .. 15 a row each (lane l: columns 4l .. 4l+3), so no wave
    // waits for codes before its row chain (vmcnt counts in issue order).
    const int rw = wave - (16 - RT);   // this wave's row when >= 0
    const bool chainw = rw >= 0;
    const size_t row = row0 + (chainw ? rw : 0);
    const bool act = lane < C4;
    const int c0 = 4 * (act ? lane : C4 - 1);
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    uint2 wr[KS];
    float wsc[KS];
    if (wave < ntile) {
        const size_t n = size_t(nbase + wave * 16 + r16);
#pragma unroll
        for (int s = 0; s < KS; ++s) wr[s] = codes_at<BITS>(a.Wqkv, n, C, 32 * s + 8 * q4);
        load_scales<KS>(a.Sqkv + n * KS, wsc);
    }
    if (chainw) {
    const float4 w1 = ld4(a.n1 + c0);
    float4 y, mp, w2, w3;
    if constexpr (FIRST) {
        y = ld4(a.x + row * C + c0);
    } else {
        float4 pp[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) pp[p] = ld4(a.part + (size_t(p) * a.B * a.T + row) * C + c0);
        mp = ld4(a.mid_prev + row * C + c0);
        w2 = ld4(a.n2b + c0);
        w3 = ld4(a.nf + c0);
        y = pp[0];
#pragma unroll
        for (int p = 1; p < NP; ++p) y = add4(y, pp[p]);   // slab order
    }

    // -- the row chain (group 0 stores the row outputs), ln1 pieces into LDS.
    const bool saver = g == 0;
    float rs;
    if constexpr (!FIRST) {
        rs = rstd_row<C>(act ? y : z4, a.eps);   // rms(mlp)
        if (saver && act && a.pmlp) st4(a.pmlp + row * C + c0, y);
        if (saver && a.pr2b && lane == 0) a.pr2b[row] = rs;
        y = add4(mp, norm4(y, rs, w2));          // pre = mid + rms(mlp) * n2b
        if (saver && act && a.ppre) st4(a.ppre + row * C + c0, y);
        rs = rstd_row<C>(act ? y : z4, a.eps);   // rms(pre)
        if (saver && a.prf && lane == 0) a.prf[row] = rs;
        y = norm4(y, rs, w3);                    // x = rms(pre) * nf
    }
    if (saver && act && a.xo) st4(a.xo + row * C + c0, y);
    rs = rstd_row<C>(act ? y : z4, a.eps);       // ln1 = rms(x) * n1
    if (saver && a.sr1 && lane == 0) a.sr1[row] = rs;
    const float4 ln = norm4(y, rs, w1);
    if (saver && act && a.sln1) st4(a.sln1 + row * C + c0, ln);
    if (act) put4(Ap, 16 * LDA, rw * LDA + c0, ln);
    }
    lds_barrier();

    // -- the group's projection tiles (wave w: tile w).
    if (wave < ntile) {
        f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < KS; ++s)
            acc = scale_add(acc, step3(Ap + r16 * LDA + 32 * s + 8 * q4, 16 * LDA, codes_bf16<BITS>(wr[s])), wsc[s]);
#pragma unroll
        for (int e = 0; e < 4; ++e) os[(4 * q4 + e) * OLD + wave * 16 + r16] = acc[e];
    }
    lds_barrier();

    // -- RoPE of q / k (rope_fwd's formula), the value residual, stores.
    constexpr int half = D / 2;
    const int t0 = int(row0 % size_t(a.T));   // token position of row 0
    auto rope = [&](const float* src, int r, int d, float& ya, float& yb) {
        const float xa = src[d], xb = src[d + half];
        const int tok = t0 + r;
        const float c1 = a.cosv[tok * D + d], c2 = a.cosv[tok * D + d + half];
        const float s1 = a.sinv[tok * D + d], s2 = a.sinv[tok * D + d + half];
        const float p1 = xa * c1, r1 = -xb * s1;   // d < D/2: rot = -x[d + D/2]
        const float p2 = xb * c2, r2 = xa * s2;    // d >= D/2: rot = x[d - D/2]
        ya = p1 + r1;
        yb = p2 + r2;
    };
    if (!kvg) {
        const int np = RT * a.HG * half;
        for (int e = threadIdx.x; e < np; e += 1024) {
            const int r = e / (a.HG * half), rem = e - r * (a.HG * half), hh = rem / half, d = rem - hh * half;
            float ya, yb;
            rope(os + r * OLD + hh * D, r, d, ya, yb);
            float* o = a.q + (row0 + r) * C + nbase + hh * D;
            o[d] = ya;
            o[d + half] = yb;
        }
    } else {
        for (int e = threadIdx.x; e < RT * half; e += 1024) {
            const int r = e / half, d = e - r * half;
            float ya, yb;
            rope(os + r * OLD, r, d, ya, yb);
            float* o = a.k + (row0 + r) * a.kv_ld;
            for (int h = 0; h < a.krep; ++h) {
                o[h * D + d] = ya;
                o[h * D + d + half] = yb;
            }
        }
        for (int e = threadIdx.x; e < RT * D; e += 1024) {
            const int r = e / D, d = e - r * D;
            float vv = os[r * OLD + D + d];
            float* f = a.vfirst + (row0 + r) * D + d;
            if constexpr (FIRST) {
                *f = vv;
            } else {
                const float pa = a.ca * vv;
                const float pb = a.cb * *f;
                vv = pa + pb;
            }
            float* o = a.v + (row0 + r) * a.kv_ld;
            for (int h = 0; h < a.krep; ++h) o[h * D + d] = vv;
        }
    }
}

// ---- loop_attn_kernel -----------------------------------------------------------------
// One workgroup of 16 waves per (sequence b, 16 query rows).
struct LoopAttnArgs {
    const float* q;          // [M, C] after RoPE
    const float *k, *v;      // rows of kv_ld floats, the KV head at column 0
    int kv_ld;
    const void* Wo;          // [C, C]
    const float* So;
    float* attn;             // output [H/2][M][C]: av . wo^T over each head pair's columns
    int64_t slab;            // M C: floats between the head pairs' partial outputs
    float* probs;            // optional [B, H, T, T]
    float* sav;              // optional training save of av
    int B;
    float scale;
};

template <int KS, int TT, int DT>
struct AttnShape {
    static constexpr int C = 32 * KS, D = 16 * DT, H = C / D, T = 16 * TT;
    static constexpr int LDA = C + 8, QLD = C + 4, KLD = D + 4, VLD = T + 4;
    static constexpr int QS = 0, KO = QS + 16 * QLD * 4, VT = KO + T * KLD * 4;
    static constexpr int PS = VT + D * VLD * 4, AV = PS + H * 16 * VLD * 4, BYTES = AV + 3 * 16 * LDA * 2;
    // Workgroups per (sequence, 16 query rows): one per (head pair, quarter of
    // wo's output columns; a half when C/32 is odd).
    static constexpr int NHG = H / 2, NWH = KS % 2 == 0 ? 4 : 2, NWO = NWH * NHG, KSW = 2 * D / 32;
    static constexpr int OT = 2 * KS / NWH;   // wo output column tiles per workgroup
    static_assert(H % 2 == 0 && (2 * D) % 32 == 0 && KS <= 16, "head pairs of whole 32-k steps");
    static_assert(KS % 2 == 0 && C % D == 0 && TT >= 1 && C / 4 <= 64, "loop_attn shape");
    static_assert(BYTES <= 160 * 1024, "loop_attn LDS");
};

template <int BITS, int KS, int TT, int DT>
__global__ __launch_bounds__(1024) void loop_attn_kernel(LoopAttnArgs a) {
#pragma clang fp contract(off)
    using S = AttnShape<KS, TT, DT>;
    constexpr int C = S::C, D = S::D, H = S::H, T = S::T;
    constexpr int LDA = S::LDA, QLD = S::QLD, KLD = S::KLD, VLD = S::VLD;
    extern __shared__ __align__(16) unsigned char lds[];
    float* qs = reinterpret_cast<float*>(lds + S::QS);
    float* ks = reinterpret_cast<float*>(lds + S::KO);
    float* vt = reinterpret_cast<float*>(lds + S::VT);
    float* ps = reinterpret_cast<float*>(lds + S::PS);
    __bf16* Av = reinterpret_cast<__bf16*>(lds + S::AV);
    constexpr int NWO = S::NWO, KSW = S::KSW;
    int b, item;
    if (!seq_block(a.B, NWO * TT, b, item)) return;
    // Heads h0, h0 + 1 (their contraction columns k0 .. k0 + 2D of wo), wo's
    // output column tiles wh OT .. wh OT + OT-1.
    constexpr int NWH = S::NWH, OT = S::OT;
    const int qt = item / NWO, hg = (item % NWO) / NWH, wh = item % NWH;
    const int h0 = 2 * hg, k0 = h0 * D;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;
    const size_t seq0 = size_t(b) * T, own0 = seq0 + size_t(qt) * 16;

    // -- q (16 rows, the pair's columns), k, v (T rows), staged in LDS; the
    // wo codes of this wave's column tile over the pair's columns (waves
    // 0 .. OT-1) are issued after the staging, so that it does not wait for
    // them (a wave waits for its loads in issue order): they are needed only
    // by the last phase.
    constexpr int QC = 16 * 2 * D / 4, KC = T * D / 4;   // float4 chunks
    constexpr int RQ = (QC + 1023) / 1024, RK = (KC + 1023) / 1024;
    float4 qv[RQ], kv[RK], vv[RK];
#pragma unroll
    for (int i = 0; i < RQ; ++i) {
        const int e = min(tid + 1024 * i, QC - 1), r = e / (2 * D / 4), c4 = e - r * (2 * D / 4);
        qv[i] = ld4(a.q + (own0 + r) * C + k0 + 4 * c4);
    }
#pragma unroll
    for (int i = 0; i < RK; ++i) {
        const int e = min(tid + 1024 * i, KC - 1), t = e / (D / 4), c4 = e - t * (D / 4);
        kv[i] = ld4(a.k + (seq0 + t) * a.kv_ld + 4 * c4);
        vv[i] = ld4(a.v + (seq0 + t) * a.kv_ld + 4 * c4);
    }
#pragma unroll
    for (int i = 0; i < RQ; ++i) {
        const int e = tid + 1024 * i, r = e / (2 * D / 4), c4 = e - r * (2 * D / 4);
        if (e < QC) st4(qs + r * QLD + k0 + 4 * c4, qv[i]);
    }
#pragma unroll
    for (int i = 0; i < RK; ++i) {
        const int e = tid + 1024 * i, t = e / (D / 4), c4 = e - t * (D / 4);
        if (e < KC) {
            st4(ks + t * KLD + 4 * c4, kv[i]);
            vt[(4 * c4 + 0) * VLD + t] = vv[i].x;
            vt[(4 * c4 + 1) * VLD + t] = vv[i].y;
            vt[(4 * c4 + 2) * VLD + t] = vv[i].z;
            vt[(4 * c4 + 3) * VLD + t] = vv[i].w;
        }
    }
    const int ct = wh * OT + wave;   // this wave's wo column tile when wave < OT
    uint2 wo[KSW];
    float wos[KSW];
    if (wave < OT) {
#pragma unroll
        for (int s = 0; s < KSW; ++s) {
            wo[s] = codes_at<BITS>(a.Wo, size_t(ct * 16 + r16), C, k0 + 32 * s + 8 * q4);
            wos[s] = a.So[size_t(ct * 16 + r16) * KS + k0 / 32 + s];
        }
    }
    lds_barrier();

    // -- scores = (q . k) * scale per (head of the pair, 16 keys).
    for (int tile = wave; tile < 2 * TT; tile += 16) {
        const int hl = tile / TT, kt = tile - hl * TT;
        const f32x4 acc =
            dot_tile(qs + r16 * QLD + (h0 + hl) * D + 4 * q4, ks + (kt * 16 + r16) * KLD + 4 * q4, D);
#pragma unroll
        for (int e = 0; e < 4; ++e) ps[(hl * 16 + 4 * q4 + e) * VLD + kt * 16 + r16] = acc[e] * a.scale;
    }
    lds_barrier();

    // -- row softmax, 16 lanes per (head, query row): attn_softmax's max, sum
    // of exp and normalize (each exp computed once, on the hardware 2^x: the
    // library expf made this phase VALU-bound with 16 waves on 4 SIMDs).
    for (int rr = 4 * wave + q4; rr < 2 * 16; rr += 64) {
        float* rp = ps + rr * VLD;
        float ev[TT];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < TT; ++i) {
            ev[i] = rp[r16 + 16 * i];
            mx = fmaxf(mx, ev[i]);
        }
        mx = row16_max(mx);
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < TT; ++i) {
            ev[i] = __builtin_amdgcn_exp2f((ev[i] - mx) * 1.44269504088896341f);   // e^x = 2^(x log2 e)
            sum += ev[i];
        }
        sum = row16_sum(sum);
        const float inv = 1.0f / sum;
        float* po = a.probs && wh == 0
                        ? a.probs + ((size_t(b) * H + h0 + (rr >> 4)) * T + qt * 16 + (rr & 15)) * T
                        : nullptr;
#pragma unroll
        for (int i = 0; i < TT; ++i) {
            const float pv = ev[i] * inv;
            rp[r16 + 16 * i] = pv;
            if (po) po[r16 + 16 * i] = pv;
        }
    }
    lds_barrier();

    // -- av = P.V per (head of the pair, 16 columns), kept as bf16 pieces
    // (the pair's 2D columns) for wo.
    for (int tile = wave; tile < 2 * DT; tile += 16) {
        const int hl = tile / DT, dt = tile - hl * DT;
        const f32x4 acc = dot_tile(ps + (hl * 16 + r16) * VLD + 4 * q4, vt + (dt * 16 + r16) * VLD + 4 * q4, T);
        const int col = hl * D + dt * 16 + r16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 4 * q4 + e;
            if (a.sav && wh == 0) a.sav[(own0 + r) * C + k0 + col] = acc[e];
            put1(Av, 16 * LDA, r * LDA + col, acc[e]);
        }
    }
    lds_barrier();

    // -- the pair's share of attn = av . wo^T (its 2D contraction columns)
    // for this workgroup's output columns, into head-pair slab hg.
    if (wave < OT) {
        f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < KSW; ++s)
            acc = scale_add(acc, step3(Av + r16 * LDA + 32 * s + 8 * q4, 16 * LDA, codes_bf16<BITS>(wo[s])), wos[s]);
        float* o = a.attn + hg * a.slab;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[(own0 + 4 * q4 + e) * C + ct * 16 + r16] = acc[e];
    }
}

// swiglu_fwd's logistic (metal/kernels.metal:911-930), sign-split as
// silu_sigmoid, with the exponential as the hardware 2^x of x log2 e.
__device__ __forceinline__ float silu_sigmoid_hw(float z) {
#pragma clang fp contract(off)
    const float e = __builtin_amdgcn_exp2f(-fabsf(z) * 1.44269504088896341f);   // e^-|z|
    return z >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
}

// ---- loop_mlp_kernel ------------------------------------------------------------------
// One workgroup of SL / 16 waves per (16 rows, slice of SL SwiGLU columns).
// NHG (head pairs, the attention slabs to add) is a compile-time count, so
// that every slab load of a row is issued before the first add waits (a
// run-time count compiled to a loop that waited for each load in turn).
struct LoopMlpArgs {
    const float* attn;       // [NHG][M][C]: this loop's av . wo^T per head pair (summed in order here)
    int64_t slab;            // M C
    float* sattn;            // optional training save of the sum (slice-0 workgroups)
    const float* x;          // this loop's x [M, C] (the attention half's residual)
    const float *n1b, *n2;
    float* mid;              // output [M, C], stored by the slice-0 workgroups
    float *sln2, *sr1b, *sr2;   // optional training saves (slice-0 workgroups)
    float eps;
    const void* Wgu;         // [2F, C] codes of wgate, wup back to back
    const float* Sgu;
    const void* Wd;          // [C, F]
    const float* Sd;
    float* part;             // [P][M][C]
    float *sgate, *sup, *ssw;   // optional saves [M, F]
    int B, TT, M, F, P;
};

template <int BITS, int KS, int SL, int NHG>
__global__ __launch_bounds__(4 * SL) void loop_mlp_kernel(LoopMlpArgs a) {
#pragma clang fp contract(off)
    constexpr int C = 32 * KS, J = C / 64, LDA = C + 8, LDW = SL + 8, FKS = SL / 32;
    constexpr int NW = SL / 16;                 // waves
    constexpr int DPW = (2 * KS + NW - 1) / NW;   // wdown column tiles per wave
    static_assert(SL % 32 == 0 && NW >= 4, "whole 32-k steps; four waves run the row chains");
    __shared__ __align__(16) __bf16 Ah[3 * 16 * LDA];
    __shared__ __align__(16) __bf16 Sw[3 * 16 * LDW];
    int b, item;
    if (!seq_block(a.B, a.TT * a.P, b, item)) return;
    const int slice = item % a.P;
    const size_t row0 = (size_t(b) * a.TT + item / a.P) * 16;
    const int f0 = slice * SL;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;

    // attn and x rows and the norms (waves 0..3: row 4 wave + q4, lane r16
    // of the row: columns 4 (r16 + 16 j)), then the codes: gate / up column
    // tile `wave`, wdown column tiles wave, wave + NW, ...
    // The slabs are added only after the codes' loads are issued: adding
    // them first would hold those loads until the first slabs had landed.
    float4 xv[J], xs[NHG][J], xa[J], w1[J], w2[J];
    const size_t crow = row0 + 4 * wave + q4;
    if (wave < 4) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int c = 4 * (r16 + 16 * j);
#pragma unroll
            for (int h = 0; h < NHG; ++h) xs[h][j] = ld4(a.attn + h * a.slab + crow * C + c);
            xa[j] = ld4(a.x + crow * C + c);
            w1[j] = ld4(a.n1b + c);
            w2[j] = ld4(a.n2 + c);
        }
    }
    const size_t n = size_t(f0 + wave * 16 + r16);
    uint2 gw[KS], uw[KS];
    float gs[KS], us[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        gw[s] = codes_at<BITS>(a.Wgu, n, C, 32 * s + 8 * q4);
        uw[s] = codes_at<BITS>(a.Wgu, size_t(a.F) + n, C, 32 * s + 8 * q4);
    }
    load_scales<KS>(a.Sgu + n * KS, gs);
    load_scales<KS>(a.Sgu + (size_t(a.F) + n) * KS, us);
    const int fgroups = a.F / 32;
    uint2 dw[DPW][FKS];
    float dsc[DPW][FKS];
#pragma unroll
    for (int i = 0; i < DPW; ++i) {
        const int ct = wave + NW * i;
        if (ct < 2 * KS) {
#pragma unroll
            for (int s = 0; s < FKS; ++s) dw[i][s] = codes_at<BITS>(a.Wd, size_t(ct * 16 + r16), a.F, f0 + 32 * s + 8 * q4);
            load_scales<FKS>(a.Sd + size_t(ct * 16 + r16) * fgroups + f0 / 32, dsc[i]);
        }
    }
    // mid = x + rms(attn) * n1b; ln2 = rms(mid) * n2 (the loop kernels' rstd:
    // 1 / sqrt(mean(v^2) + eps) with the hardware inverse square root).
    if (wave < 4) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            xv[j] = xs[0][j];
#pragma unroll
            for (int h = 1; h < NHG; ++h) xv[j] = add4(xv[j], xs[h][j]);   // pair order
        }
        auto rstd = [&](const float4 (&v)[J]) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                ss += v[j].x * v[j].x;
                ss += v[j].y * v[j].y;
                ss += v[j].z * v[j].z;
                ss += v[j].w * v[j].w;
            }
            return __builtin_amdgcn_rsqf(row16_sum(ss) * (1.0f / float(C)) + a.eps);
        };
        const bool saver = slice == 0;
        if (saver && a.sattn) {
#pragma unroll
            for (int j = 0; j < J; ++j) st4(a.sattn + crow * C + 4 * (r16 + 16 * j), xv[j]);
        }
        const float rs1 = rstd(xv);
#pragma unroll
        for (int j = 0; j < J; ++j) xv[j] = add4(xa[j], norm4(xv[j], rs1, w1[j]));   // mid
        const float rs2 = rstd(xv);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int c = 4 * (r16 + 16 * j);
            if (saver) st4(a.mid + crow * C + c, xv[j]);
            xv[j] = norm4(xv[j], rs2, w2[j]);                                          // ln2
            if (saver && a.sln2) st4(a.sln2 + crow * C + c, xv[j]);
        }
        if (saver && r16 == 0 && a.sr1b) a.sr1b[crow] = rs1;
        if (saver && r16 == 0 && a.sr2) a.sr2[crow] = rs2;
#pragma unroll
        for (int j = 0; j < J; ++j) put4(Ah, 16 * LDA, (4 * wave + q4) * LDA + 4 * (r16 + 16 * j), xv[j]);
    }
    lds_barrier();

    // gate and up of this wave's 16 columns, SwiGLU (swiglu_fwd's formula).
    f32x4 ag = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, au = ag;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const __bf16* ap = Ah + r16 * LDA + 32 * s + 8 * q4;
        ag = scale_add(ag, step3(ap, 16 * LDA, codes_bf16<BITS>(gw[s])), gs[s]);
        au = scale_add(au, step3(ap, 16 * LDA, codes_bf16<BITS>(uw[s])), us[s]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int r = 4 * q4 + e;
        const float z = ag[e];
        const float act = z * silu_sigmoid_hw(z);
        const float sw = act * au[e];
        if (a.sgate) {
            const size_t o = (row0 + r) * a.F + f0 + wave * 16 + r16;
            a.sgate[o] = z;
            a.sup[o] = au[e];
            a.ssw[o] = sw;
        }
        put1(Sw, 16 * LDW, r * LDW + wave * 16 + r16, sw);
    }
    lds_barrier();

    // The slice's share of wdown: sw[:, f0 : f0 + SL] . wdown[:, f0 : f0 + SL]^T.
#pragma unroll
    for (int i = 0; i < DPW; ++i) {
        const int ct = wave + NW * i;
        if (ct >= 2 * KS) break;
        f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < FKS; ++s)
            acc = scale_add(acc, step3(Sw + r16 * LDW + 32 * s + 8 * q4, 16 * LDW, codes_bf16<BITS>(dw[i][s])),
                            dsc[i][s]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            a.part[(size_t(slice) * a.M + row0 + 4 * q4 + e) * C + ct * 16 + r16] = acc[e];
    }
}

// ---- loop_tail_kernel: the row chain after the last loop ------------------------------
// mlp = the slabs in slab order; pre = mid + rms(mlp)*n2b; x = rms(pre)*nf.
// One row per wave (lane l: columns 4l .. 4l+3), 4 rows per workgroup.
struct LoopTailArgs {
    const float* part;
    const float* mid;
    const float *n2b, *nf;
    float* x;
    float *pmlp, *ppre, *pr2b, *prf;   // optional saves of the last loop
    int M;
    float eps;
};

template <int C, int NP>
__global__ __launch_bounds__(256) void loop_tail_kernel(LoopTailArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const size_t row = size_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= size_t(a.M)) return;
    const bool act = lane < C / 4;
    const int c0 = 4 * (act ? lane : C / 4 - 1);
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 pp[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) pp[p] = ld4(a.part + (size_t(p) * a.M + row) * C + c0);
    const float4 m = ld4(a.mid + row * C + c0), w2 = ld4(a.n2b + c0), w3 = ld4(a.nf + c0);
    float4 y = pp[0];
#pragma unroll
    for (int p = 1; p < NP; ++p) y = add4(y, pp[p]);   // slab order
    if (act && a.pmlp) st4(a.pmlp + row * C + c0, y);
    float rs = rstd_row<C>(act ? y : z4, a.eps);
    if (a.pr2b && lane == 0) a.pr2b[row] = rs;
    y = add4(m, norm4(y, rs, w2));
    if (act && a.ppre) st4(a.ppre + row * C + c0, y);
    rs = rstd_row<C>(act ? y : z4, a.eps);
    if (a.prf && lane == 0) a.prf[row] = rs;
    if (act) st4(a.x + row * C + c0, norm4(y, rs, w3));
}

// ---- loop_attn_bwd_kernel: the attention backward of one loop --------------------------
// The reference's attention backward (metal/kernels.metal:508-612) followed by
// the DiT's sum_heads of dk and dv, rope_bwd of dq and dk and the value
// residual (src/DiT.swift:600-620), one launch. Per sequence b, 2 TT
// workgroups of 16 waves: the query side (item < TT) owns query rows
// 16 item .. and produces dq; the key side owns key rows and produces dk and
// dv of the single KV head (summed over the query heads). Both form
// dS = P * (dP - D) with D[h][t] = dO_h[t] . O_h[t], the row sum of dP * P
// (sum_s P[t][s] dO[t].V[s] = dO[t].O[t]), from the attention output O. The
// products run on fp32 MFMA.
struct LoopAttnBwdArgs {
    const float* q;          // [M, C] after RoPE
    const float *k, *v;      // [M, C] repeated to every head: the KV head is columns 0 .. D-1
    const float* probs;      // [B, H, T, T]
    const float* o;          // [M, C] the attention output (av)
    const float* dout;       // [M, C] dL/d(av)
    const float *cosv, *sinv;
    float* dq;               // rows of ldq floats: gradient of q before RoPE
    int ldq;
    float *dk, *dv;          // rows of ldkv floats: of k before RoPE, of v before the value mix
    int ldkv;
    float* dfirst;           // [M, D]: the value-residual source's gradient
    int B, vmix;
    int fresh;               // dfirst holds nothing yet (the first loop the backward runs)
    float ca, mixc, scale;
    int own;                 // workgroups of the attention backward; those past it run dW tiles
    dgm_dw::DwTileArgs dw;   // another linear's dW (32 x 16 tiles, one per workgroup)
    int dw_tiles, dw_tiles_n;
};

template <int KS, int TT, int DT>
struct AttnBwdShape {
    static constexpr int C = 32 * KS, D = 16 * DT, H = C / D, T = 16 * TT, HT = H * T, C4 = C / 4, D4 = D / 4;
    static constexpr int QLD = C + 4, KLD = D + 4, VLD = T + 4, SLD = HT + 4, XLD = 2 * D + 4;
    // query side (floats): G [16][QLD] | Vf [T][KLD] | Kt [D][VLD] | Pm [16H][VLD] | Dq [16H] | dqs [16][QLD]
    // (dqs first holds the [16][C4] partial dots of D)
    static constexpr int QG = 0, QV = QG + 16 * QLD, QK = QV + T * KLD, QP = QK + D * VLD, QD = QP + 16 * H * VLD,
                         QO = QD + 16 * H, QEND = QO + 16 * QLD;
    // key side: G [T][QLD] | Qs [T][QLD] | Vs [16][KLD] | Ps [16][SLD] | dSs [16][SLD] | Dk [HT]
    // (dSs first holds the [T][C4] partial dots; G | Qs last hold the [2][16][XLD] halves of dk | dv)
    static constexpr int KG = 0, KQ = KG + T * QLD, KV = KQ + T * QLD, KP = KV + 16 * KLD, KS_ = KP + 16 * SLD,
                         KD = KS_ + 16 * SLD, KEND = KD + HT;
    static constexpr int BYTES = 4 * (QEND > KEND ? QEND : KEND);
    static_assert(T * C4 <= 16 * SLD && 16 * C4 <= 16 * QLD && 2 * 16 * XLD <= 2 * T * QLD, "aliased LDS");
    static_assert(BYTES <= 160 * 1024, "loop_attn_bwd LDS");
    static_assert(H % 2 == 0, "two halves of the heads");
};

template <int KS, int TT, int DT>
__global__ __launch_bounds__(1024) void loop_attn_bwd_kernel(LoopAttnBwdArgs a) {
#pragma clang fp contract(off)
    using S = AttnBwdShape<KS, TT, DT>;
    if (int(blockIdx.x) >= a.own) {
        // One dW tile per workgroup over its sixteen waves (32 KB of the LDS).
        static_assert(dgm_dw::kHostedWaves == 16, "a 1024-thread workgroup per tile");
        extern __shared__ __align__(16) float lds_w[];
        dgm_dw::dw_tile<2, dgm_dw::kPairCH, dgm_dw::kHostedWaves>(
            a.dw, true, int(blockIdx.x) - a.own, a.dw_tiles_n, int(threadIdx.x >> 6), int(threadIdx.x),
            reinterpret_cast<float (*)[2][16][16]>(lds_w));
        return;
    }
    constexpr int C = S::C, D = S::D, H = S::H, T = S::T, HT = S::HT, C4 = S::C4, D4 = S::D4;
    constexpr int QLD = S::QLD, KLD = S::KLD, VLD = S::VLD, SLD = S::SLD, XLD = S::XLD, mid = D / 2;
    extern __shared__ __align__(16) float lds_f[];
    int b, item;
    if (!seq_block(a.B, 2 * TT, b, item)) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, q4 = lane >> 4;
    const size_t seq0 = size_t(b) * T;

    if (item < TT) {   // ---- query side: rows qt*16 ..
        const int qt = item;
        const size_t own0 = seq0 + size_t(qt) * 16;
        float* G = lds_f + S::QG;
        float* Vf = lds_f + S::QV;
        float* Kt = lds_f + S::QK;
        float* Pm = lds_f + S::QP;
        float* Dq = lds_f + S::QD;
        float* dqs = lds_f + S::QO;
        {
            constexpr int NG = 16 * C4, NV = T * D4, NP = 16 * H * (T / 4);
            static_assert(NG <= 1024 && NV <= 1024 && NP <= 1024, "one chunk per thread");
            float4 gv, ov, vv, kv, pv;
            const int r = tid / C4, c4 = tid - r * C4;
            const int t = tid / D4, d4 = tid - t * D4;
            const int pr = tid / (T / 4), pc = tid - pr * (T / 4);   // pr = h * 16 + row
            if (tid < NG) {
                gv = ld4(a.dout + (own0 + r) * C + 4 * c4);
                ov = ld4(a.o + (own0 + r) * C + 4 * c4);
            }
            if (tid < NV) {
                vv = ld4(a.v + (seq0 + t) * C + 4 * d4);
                kv = ld4(a.k + (seq0 + t) * C + 4 * d4);
            }
            if (tid < NP)
                pv = ld4(a.probs + ((size_t(b) * H + pr / 16) * T + qt * 16 + pr % 16) * T + 4 * pc);
            if (tid < NG) {
                st4(G + r * QLD + 4 * c4, gv);
                dqs[r * C4 + c4] = ((gv.x * ov.x + gv.y * ov.y) + gv.z * ov.z) + gv.w * ov.w;
            }
            if (tid < NV) {
                st4(Vf + t * KLD + 4 * d4, vv);
                Kt[(4 * d4 + 0) * VLD + t] = kv.x;
                Kt[(4 * d4 + 1) * VLD + t] = kv.y;
                Kt[(4 * d4 + 2) * VLD + t] = kv.z;
                Kt[(4 * d4 + 3) * VLD + t] = kv.w;
            }
            if (tid < NP) st4(Pm + pr * VLD + 4 * pc, pv);
        }
        lds_barrier();
        if (tid < 16 * H) {   // D[h][row] = sum of the head's partial dots, in chunk order
            const int h = tid / 16, r = tid % 16;
            float s = 0.0f;
            for (int j = 0; j < D4; ++j) s += dqs[r * C4 + h * D4 + j];
            Dq[tid] = s;
        }
        lds_barrier();
        // dS = P * (dP - D), dP[t][s] = dO_h[t] . V[s], per (head, 16 keys).
        for (int tile = wave; tile < H * TT; tile += 16) {
            const int h = tile / TT, kt = tile - h * TT;
            const f32x4 acc = dot_tile(G + r16 * QLD + h * D + 4 * q4, Vf + (kt * 16 + r16) * KLD + 4 * q4, D);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int pr = h * 16 + 4 * q4 + e;
                float* p = Pm + pr * VLD + kt * 16 + r16;
                *p = *p * (acc[e] - Dq[pr]);
            }
        }
        lds_barrier();
        // dq_h = scale * dS_h . K, per (head, 16 columns).
        for (int tile = wave; tile < H * DT; tile += 16) {
            const int h = tile / DT, dt = tile - h * DT;
            const f32x4 acc = dot_tile(Pm + (h * 16 + r16) * VLD + 4 * q4, Kt + (dt * 16 + r16) * VLD + 4 * q4, T);
#pragma unroll
            for (int e = 0; e < 4; ++e) dqs[(4 * q4 + e) * QLD + h * D + dt * 16 + r16] = acc[e] * a.scale;
        }
        lds_barrier();
        // rope_bwd (metal/kernels.metal:891-909).
        for (int e = tid; e < 16 * C; e += 1024) {
            const int r = e / C, col = e - r * C, d = col % D, t = qt * 16 + r;
            const float c = a.cosv[t * D + d], s = a.sinv[t * D + d];
            const float* row = dqs + r * QLD;
            a.dq[(own0 + r) * a.ldq + col] = d < mid ? row[col] * c + row[col + mid] * s : row[col] * c - row[col - mid] * s;
        }
        return;
    }

    // ---- key side: keys s0 ..
    const int s0 = (item - TT) * 16;
    float* G = lds_f + S::KG;
    float* Qs = lds_f + S::KQ;
    float* Vs = lds_f + S::KV;
    float* Ps = lds_f + S::KP;
    float* dSs = lds_f + S::KS_;
    float* Dk = lds_f + S::KD;
    {
        constexpr int NG = T * C4, NV = 16 * D4, NP = HT * 4;   // P: (h, t) rows of 16 keys = 4 float4
        constexpr int RG = (NG + 1023) / 1024;
        float4 gv[RG], ov[RG], qv[RG], vv, pv;
#pragma unroll
        for (int i = 0; i < RG; ++i) {
            const int e = min(tid + 1024 * i, NG - 1), t = e / C4, c4 = e - t * C4;
            gv[i] = ld4(a.dout + (seq0 + t) * C + 4 * c4);
            ov[i] = ld4(a.o + (seq0 + t) * C + 4 * c4);
            qv[i] = ld4(a.q + (seq0 + t) * C + 4 * c4);
        }
        const int vr = tid / D4, vd = tid - vr * D4;
        if (tid < NV) vv = ld4(a.v + (seq0 + s0 + vr) * C + 4 * vd);
        const int ph = tid / 4, pc = tid - ph * 4;   // ph = h * T + t
        if (tid < NP) pv = ld4(a.probs + ((size_t(b) * H + ph / T) * T + ph % T) * T + s0 + 4 * pc);
#pragma unroll
        for (int i = 0; i < RG; ++i) {
            const int e = tid + 1024 * i, t = e / C4, c4 = e - t * C4;
            if (e < NG) {
                st4(G + t * QLD + 4 * c4, gv[i]);
                st4(Qs + t * QLD + 4 * c4, qv[i]);
                dSs[t * C4 + c4] = ((gv[i].x * ov[i].x + gv[i].y * ov[i].y) + gv[i].z * ov[i].z) + gv[i].w * ov[i].w;
            }
        }
        if (tid < NV) st4(Vs + vr * KLD + 4 * vd, vv);
        if (tid < NP) {
            Ps[(4 * pc + 0) * SLD + ph] = pv.x;
            Ps[(4 * pc + 1) * SLD + ph] = pv.y;
            Ps[(4 * pc + 2) * SLD + ph] = pv.z;
            Ps[(4 * pc + 3) * SLD + ph] = pv.w;
        }
    }
    lds_barrier();
    for (int e = tid; e < HT; e += 1024) {   // D[h][t], e = h * T + t
        const int h = e / T, t = e - h * T;
        float s = 0.0f;
        for (int j = 0; j < D4; ++j) s += dSs[t * C4 + h * D4 + j];
        Dk[e] = s;
    }
    lds_barrier();
    // dS^T[s][(h, t)] = P * (dP - D), dP^T[s][t] = V[s] . dO_h[t], per (head, 16 queries).
    for (int tile = wave; tile < H * TT; tile += 16) {
        const int h = tile / TT, tt = tile - h * TT;
        const f32x4 acc = dot_tile(Vs + r16 * KLD + 4 * q4, G + (tt * 16 + r16) * QLD + h * D + 4 * q4, D);
        const int ht = h * T + tt * 16 + r16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int o = (4 * q4 + e) * SLD + ht;
            dSs[o] = Ps[o] * (acc[e] - Dk[ht]);
        }
    }
    lds_barrier();
    // dk = sum_(h,t) dS^T[s][(h,t)] Q_h[t], dv = sum_(h,t) P^T[s][(h,t)] dO_h[t]:
    // items (dk | dv, 16 columns, half of the heads).
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int item2 = wave;
    const bool busy = item2 < 4 * DT;
    const int which = item2 / (2 * DT), dt = (item2 / 2) % DT, half = item2 % 2;
    if (busy) {
        const float* A = (which == 0 ? dSs : Ps) + r16 * SLD;
        const float* X = which == 0 ? Qs : G;
        const int d = dt * 16 + r16;
        for (int k0 = half * (HT / 2); k0 < (half + 1) * (HT / 2); k0 += 16) {
            const float4 av = ld4(A + k0 + 4 * q4);
            const int h = k0 / T, t = k0 - h * T + 4 * q4;
            const float* xb = X + t * QLD + h * D + d;
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, xb[0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, xb[QLD], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, xb[2 * QLD], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, xb[3 * QLD], acc, 0, 0, 0);
        }
    }
    lds_barrier();   // G and Qs are no longer read: the halves go where they were
    float* st = G;   // [2][16][XLD]: columns 0 .. D-1 dk, D .. 2D-1 dv
    if (busy) {
#pragma unroll
        for (int e = 0; e < 4; ++e) st[(half * 16 + 4 * q4 + e) * XLD + which * D + dt * 16 + r16] = acc[e];
    }
    lds_barrier();
    // rope_bwd of dk (one head), the value residual of dv.
    for (int e = tid; e < 16 * mid; e += 1024) {
        const int s = e / mid, d = e - s * mid, t = s0 + s;
        const float x0 = (st[s * XLD + d] + st[(16 + s) * XLD + d]) * a.scale;
        const float x1 = (st[s * XLD + d + mid] + st[(16 + s) * XLD + d + mid]) * a.scale;
        float* o = a.dk + (seq0 + t) * a.ldkv;
        o[d] = x0 * a.cosv[t * D + d] + x1 * a.sinv[t * D + d];
        o[d + mid] = x1 * a.cosv[t * D + d + mid] - x0 * a.sinv[t * D + d + mid];
    }
    for (int e = tid; e < 16 * D; e += 1024) {
        const int s = e / D, d = e - s * D;
        const size_t row = seq0 + s0 + s;
        const float v = st[s * XLD + D + d] + st[(16 + s) * XLD + D + d];
        float* f = a.dfirst + row * D + d;
        const float f0 = a.fresh ? 0.0f : *f;
        if (a.vmix == 0) {
            a.dv[row * a.ldkv + d] = v + f0;
        } else {
            const float p = a.ca * v;
            const float r = 0.0f * v;
            a.dv[row * a.ldkv + d] = p + r;
            *f = f0 + a.mixc * v;
        }
    }
}

// ---- host side -------------------------------------------------------------------------
template <int BITS, int KS, int TT, int DT, int NP, int SL>
int run_loops(dgm_gpu* g, const dgm_dit_cfg* c, const dgm_dit_weights* w, const float* cosv, const float* sinv,
              float* x, const dgm::DitLoopBufs& buf, const dgm::DitSaves* sv) {
    using S = AttnShape<KS, TT, DT>;
    const int B = c->B, L = c->loops, T = S::T, H = S::H, D = S::D, C = S::C;
    const int M = B * T;
    const int gb = 8 * ((B + 7) / 8);   // blocks of sequence b run on XCD b % 8
    const int HG = H % 2 == 0 ? 2 : 1, NG = H / HG + 1;
    auto attn_k = loop_attn_kernel<BITS, KS, TT, DT>;
    if (S::BYTES > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_k),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, S::BYTES);
        if (e != hipSuccess)
            return dgm::fail(g, DGM_ERR_HIP, "dit_forward: cannot reserve %d bytes of LDS: %s", S::BYTES,
                             hipGetErrorString(e));
    }
    // mid alternates between two buffers (a loop reads the previous loop's
    // mid while writing its own), or is saved per loop; q / k / v are the
    // training saves ([M, C] rows; k and v hold the KV head in columns
    // 0 .. D-1, which is all the backward of these shapes reads) or the
    // inference buffers (k, v as [M, D]).
    auto mid_of = [&](int l) { return sv ? sv[l].mid : buf.mid[l & 1]; };
    for (int l = 0; l < L; ++l) {
        float* q = sv ? sv[l].q : buf.q;
        float* k = sv ? sv[l].k : buf.k;
        float* v = sv ? sv[l].v : buf.v;
        const int kv_ld = sv ? C : D;
        float* xl = sv ? sv[l].x : x;   // this loop's x, the residual of its attention half

        LoopRowArgs ra{};
        ra.x = x;
        ra.part = buf.part;
        ra.mid_prev = l > 0 ? mid_of(l - 1) : nullptr;
        ra.n1 = w->n1; ra.n2b = w->n2b; ra.nf = w->nf;
        ra.Wqkv = w->wq.q; ra.Sqkv = w->wq.scale;
        ra.cosv = cosv; ra.sinv = sinv;
        ra.vfirst = buf.vfirst;
        ra.q = q; ra.k = k; ra.v = v; ra.kv_ld = kv_ld; ra.krep = 1;   // the KV head only (columns 0 .. D-1)
        ra.xo = (sv || l > 0) ? xl : nullptr;
        if (sv) {
            ra.sln1 = sv[l].ln1; ra.sr1 = sv[l].r1;
            if (l > 0) { ra.pmlp = sv[l - 1].mlp; ra.ppre = sv[l - 1].pre; ra.pr2b = sv[l - 1].r2b; ra.prf = sv[l - 1].rf; }
        }
        ra.B = B; ra.T = T; ra.NG = NG; ra.HG = HG;
        ra.eps = c->eps; ra.ca = 1.0f - c->mix; ra.cb = c->mix;
        const dim3 rgrid(unsigned(gb * (T / kRowTile) * NG));
        if (l == 0) hipLaunchKernelGGL((loop_row_kernel<BITS, KS, DT, NP, true>), rgrid, dim3(1024), 0, g->stream, ra);
        else hipLaunchKernelGGL((loop_row_kernel<BITS, KS, DT, NP, false>), rgrid, dim3(1024), 0, g->stream, ra);
        DGM_LAUNCH_CHECK(g, "dit_forward loop_row");

        // The head pairs' partial attn slabs follow the wdown slabs.
        float* attn = buf.part + int64_t(NP) * M * C;
        LoopAttnArgs aa{};
        aa.q = q; aa.k = k; aa.v = v; aa.kv_ld = kv_ld;
        aa.Wo = w->wo.q; aa.So = w->wo.scale;
        aa.attn = attn; aa.slab = int64_t(M) * C;
        aa.probs = sv ? sv[l].probs : (l == L - 1 ? buf.probs_last : nullptr);
        if (sv) aa.sav = sv[l].av;
        aa.B = B; aa.scale = 1.0f / sqrtf(float(D));
        hipLaunchKernelGGL(attn_k, dim3(unsigned(gb * TT * S::NWO)), dim3(1024), size_t(S::BYTES), g->stream, aa);
        DGM_LAUNCH_CHECK(g, "dit_forward loop_attn");

        LoopMlpArgs ma{};
        ma.attn = attn; ma.slab = int64_t(M) * C; ma.x = xl; ma.n1b = w->n1b; ma.n2 = w->n2;
        if (sv) ma.sattn = sv[l].attn;
        ma.mid = mid_of(l);
        if (sv) { ma.sln2 = sv[l].ln2; ma.sr1b = sv[l].r1b; ma.sr2 = sv[l].r2; }
        ma.eps = c->eps;
        ma.Wgu = w->wgate.q; ma.Sgu = w->wgate.scale;
        ma.Wd = w->wdown.q; ma.Sd = w->wdown.scale;
        ma.part = buf.part;
        if (sv) { ma.sgate = sv[l].gate; ma.sup = sv[l].up; ma.ssw = sv[l].sw; }
        ma.B = B; ma.TT = TT; ma.M = M; ma.F = c->F; ma.P = NP;
        hipLaunchKernelGGL((loop_mlp_kernel<BITS, KS, SL, S::NHG>), dim3(unsigned(gb * TT * NP)), dim3(4 * SL), 0, g->stream,
                           ma);
        DGM_LAUNCH_CHECK(g, "dit_forward loop_mlp");
    }
    if (L > 0) {
        LoopTailArgs ta{};
        ta.part = buf.part;
        ta.mid = mid_of(L - 1);
        ta.n2b = w->n2b; ta.nf = w->nf;
        ta.x = x;
        if (sv) { ta.pmlp = sv[L - 1].mlp; ta.ppre = sv[L - 1].pre; ta.pr2b = sv[L - 1].r2b; ta.prf = sv[L - 1].rf; }
        ta.M = M;
        ta.eps = c->eps;
        hipLaunchKernelGGL((loop_tail_kernel<32 * KS, NP>), dim3(unsigned((M + 3) / 4)), dim3(256), 0, g->stream, ta);
        DGM_LAUNCH_CHECK(g, "dit_forward loop_tail");
    }
    return DGM_OK;
}

// The built shapes: (C / 32, T / 16, D / 16, F / SL, SL).
template <int BITS>
int dispatch(dgm_gpu* g, const dgm_dit_cfg* c, const dgm_dit_weights* w, const float* cosv, const float* sinv,
             float* x, const dgm::DitLoopBufs& buf, const dgm::DitSaves* sv) {
    const int sl = slice_cols(c);
    const int ks = c->C / 32, tt = c->T / 16, dt = c->D / 16, np = c->F / sl;
    if (ks == 6 && tt == 4 && dt == 3 && np == 8 && sl == 96)
        return run_loops<BITS, 6, 4, 3, 8, 96>(g, c, w, cosv, sinv, x, buf, sv);
    if (ks == 6 && tt == 4 && dt == 3 && np == 6 && sl == 128)
        return run_loops<BITS, 6, 4, 3, 6, 128>(g, c, w, cosv, sinv, x, buf, sv);
    if (ks == 2 && tt == 1 && dt == 1 && np == 1 && sl == 128)
        return run_loops<BITS, 2, 1, 1, 1, 128>(g, c, w, cosv, sinv, x, buf, sv);
    return dgm::fail(g, DGM_ERR_UNSUPPORTED, "dit_forward: no loop kernels built for this shape");
}

bool shape_built(const dgm_dit_cfg* c) {
    const int sl = slice_cols(c);
    const int ks = c->C / 32, tt = c->T / 16, dt = c->D / 16, np = c->F / sl;
    return (ks == 6 && tt == 4 && dt == 3 && ((np == 8 && sl == 96) || (np == 6 && sl == 128))) ||
           (ks == 2 && tt == 1 && dt == 1 && np == 1 && sl == 128);
}


template <int KS, int TT, int DT>
int run_attn_bwd(dgm_gpu* g, LoopAttnBwdArgs a) {
    using S = AttnBwdShape<KS, TT, DT>;
    auto k = loop_attn_bwd_kernel<KS, TT, DT>;
    // The dW workgroups use 32 KB of the same dynamic LDS.
    constexpr int kDwLds = dgm_dw::kHostedWaves * 2 * 16 * 16 * 4;
    const int bytes = a.dw_tiles > 0 && S::BYTES < kDwLds ? kDwLds : S::BYTES;
    if (bytes > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess)
            return dgm::fail(g, DGM_ERR_HIP, "dit_backward: cannot reserve %d bytes of LDS: %s", bytes,
                             hipGetErrorString(e));
    }
    a.own = 8 * ((a.B + 7) / 8) * 2 * TT;
    hipLaunchKernelGGL(k, dim3(unsigned(a.own + a.dw_tiles)), dim3(1024), size_t(bytes), g->stream, a);
    return dgm::check_launch(g, "dit_backward loop_attn_bwd");
}

}  // namespace

namespace dgm {

bool dit_loop_shape_ok(const dgm_dit_cfg* c) {
    if (!c || (c->bits != 8 && c->bits != 4) || c->group != 32 || c->loops < 0 || c->B <= 0) return false;
    if (c->C % 64 != 0 || c->D % 16 != 0 || c->H * c->D != c->C || c->T % 16 != 0) return false;
    if (c->F <= 0 || c->F % slice_cols(c) != 0) return false;
    return shape_built(c);
}

// The wdown slabs (F / SL) and the attention's head-pair slabs (H / 2).
int64_t dit_loop_part_floats(const dgm_dit_cfg* c) {
    if (!dit_loop_shape_ok(c)) return 0;
    return int64_t(c->F / slice_cols(c) + c->H / 2) * c->B * c->T * c->C;
}

bool dit_loop_ok(const dgm_dit_cfg* c, const dgm_dit_weights* w) {
    if (!dit_loop_shape_ok(c)) return false;
    const int64_t C = c->C, F = c->F, KV = c->D;
    if (!dit_linear_follows(w->wq, w->wk, C, C, c->bits, c->group) ||
        !dit_linear_follows(w->wk, w->wv, KV, C, c->bits, c->group) ||
        !dit_linear_follows(w->wgate, w->wup, F, C, c->bits, c->group))
        return false;
    const size_t al = c->bits == 8 ? 8 : 4;
    return aligned(w->wq.q, al) && aligned(w->wo.q, al) && aligned(w->wgate.q, al) && aligned(w->wdown.q, al) &&
           aligned(w->wq.scale, 8) && aligned(w->wo.scale, 8) && aligned(w->wgate.scale, 8) &&
           aligned(w->wdown.scale, 8) && aligned(w->n1, 16) && aligned(w->n1b, 16) && aligned(w->n2, 16) &&
           aligned(w->n2b, 16) && aligned(w->nf, 16);
}

int dit_forward_loops(dgm_gpu* g, const dgm_dit_cfg* c, const dgm_dit_weights* w, const float* cosv,
                      const float* sinv, float* x, const DitLoopBufs& buf, const DitSaves* saves) {
    return c->bits == 8 ? dispatch<8>(g, c, w, cosv, sinv, x, buf, saves)
                        : dispatch<4>(g, c, w, cosv, sinv, x, buf, saves);
}


bool dit_attn_bwd_loop_ok(const dgm_dit_cfg* c, const float* acts, const float* ws) {
    const int ks = c->C / 32, tt = c->T / 16, dt = c->D / 16;
    return dit_loop_shape_ok(c) && ((ks == 6 && tt == 4 && dt == 3) || (ks == 2 && tt == 1 && dt == 1)) &&
           aligned(acts, 16) && aligned(ws, 16);
}

int dit_attn_bwd_loop(dgm_gpu* g, const dgm_dit_cfg* c, const float* q, const float* k, const float* v,
                      const float* probs, const float* o, const float* dout, const float* cosv, const float* sinv,
                      float* dq, int ldq, float* dk, float* dv, int ldkv, float* dfirst, bool first, bool fresh,
                      const dgm_dw::DwTileArgs* dw) {
    if (!dit_attn_bwd_loop_ok(c, q, dout)) return kNotFused;
    LoopAttnBwdArgs a{};
    if (dw) {
        a.dw = *dw;
        a.dw_tiles = dgm_dw::dw_tiles(*dw);
        a.dw_tiles_n = dgm_dw::dw_tiles_n(*dw);
    }
    a.q = q; a.k = k; a.v = v; a.probs = probs; a.o = o; a.dout = dout; a.cosv = cosv; a.sinv = sinv;
    a.dq = dq; a.ldq = ldq; a.dk = dk; a.dv = dv; a.ldkv = ldkv; a.dfirst = dfirst;
    a.B = c->B; a.vmix = first ? 0 : 1; a.fresh = fresh ? 1 : 0; a.ca = 1.0f - c->mix; a.mixc = c->mix;
    a.scale = 1.0f / sqrtf(float(c->D));
    const int ks = c->C / 32, tt = c->T / 16, dt = c->D / 16;
    if (ks == 6 && tt == 4 && dt == 3) return run_attn_bwd<6, 4, 3>(g, a);
    if (ks == 2 && tt == 1 && dt == 1) return run_attn_bwd<2, 1, 1>(g, a);
    return kNotFused;
}

}  // namespace dgm
