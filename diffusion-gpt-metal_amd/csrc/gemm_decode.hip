// Decode-shaped (M <= 64) dequant-fused group-quant forward on f16 MFMA
// (gfx950):
//
//   Y[m,n] = sum_g S[n,g] * sum_{k in g} code[n,k] * X[m,k]  (+ bias[n])
//
// The per-group scale multiplies an fp32 partial of exact code * x products
// (the reference's own order: group partial, scale, bias last;
// metal/kernels.metal:152-209). The codes enter the MFMA unscaled: int4 and
// int8 codes are exact in f16.
//
// Activations are split into f16 pieces against a power-of-two factor per
// (row, block of k):
//     x' = x * 2^e,  max|x'| over the block in [2^14, 2^15),
//     x' = h1 + h2 + r,  h1 = f16(x'), h2 = f16(x' - h1),  |r| <= 2^-22 |x'|
// (plus the f16 subnormal floor, 2^-39 of the block maximum). Two pieces are
// the fp32 mode (bar 1e-5): every element keeps ~22 bits of its own
// magnitude, so an outlier costs nothing outside its block. One piece is the
// reduced-precision mode (bar 1e-2). The products h * code are exact in the
// MFMA's fp32 accumulation; the block partial is rescaled exactly by 2^-e
// before the group scale.
//
// Reduced-precision int4 instead takes bf16(x) with its own exponent (no
// factor) against the codes entered as 128 + (code + 8), exact in bf16; the
// offset 136 leaves inside each block's fp32 partial (see below).
//
// Two kernels:
//  * M <= 16 (decode_small_kernel, further down): one launch; every
//    workgroup converts the activations it needs in registers.
//  * 16 < M <= 64 (decode_kernel): a prepare kernel writes the pieces once,
//    fragment-major: for each MFMA step (32 k), row tile and piece, the 64
//    lanes' 16-byte A fragments form one contiguous 1 KB, so every activation
//    load is a whole-line 1 KB read. A row block holding a non-finite value
//    is stored as NaN, so that output row is NaN (bf16: the value itself;
//    an infinity meets the offset term's opposite infinity and gives NaN).
//    For bf16 the prepare pass also writes, per (block, row), the fp32 term
//    -136 * sum of the block's bf16(x); a block's MFMA chain starts from it,
//    so the offset is removed before the group scale, exactly whenever the
//    sums are exact (one-hot or small-integer activations).
//
// Weights (both kernels). A workgroup owns 64 whole rows of W (64 output
// columns) and all of K; its compute waves split K, so each weight is
// converted once per workgroup. A separate wave only streams W global -> LDS
// with direct-to-LDS loads into a ring, several intervals ahead: the weight
// stream needs a long lead (HBM latency plus this workgroup's share of the
// bandwidth) and the activations a short one; a wave's load counter retires
// in issue order, so one wave issuing both would make every activation wait
// for the younger weight loads. One barrier per interval hands the weights
// from the stream wave to the compute waves. 16-byte slots are XOR-swizzled
// by row (slot = piece ^ (row & 7)), which keeps the fragment reads free of
// bank conflicts.
//
// Code -> f16 without a convert instruction: offset-binary codes (sign bit
// flipped) are placed under the exponent of 1024.0 (0x6400) by one v_bitop3,
// giving 1024 + code + bias exactly, and one packed f16 FMA removes the bias
// (a nibble held in bits 4-7 is 16 times larger and is scaled by 1/16 in the
// same FMA). int4: 9 VALU ops per 8 weights; int8: 5 per 4.
//
// Loads are issued as inline asm and waited for by hand: every step issues
// the same sequence, so each wait count is a compile-time constant, and
// nothing waits for loads issued after the data it needs. The waves' fp32
// partials are summed in LDS in a fixed order at the end (deterministic
// results).
#include "common.hpp"
#include "decode_codes.hpp"

#include <atomic>
#include <type_traits>

// Set (to 1) by a decode workgroup whose bounded hand-over wait gave up;
// read and cleared by dgm_end (decode_wait_check). One per device.
__device__ uint32_t g_wait_gave_up;

namespace {

using namespace dgm_codes;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int DEC_COLS = 64;                 // W rows (output columns) per workgroup
constexpr int DEC_SLOTS = 4;                 // intervals (4 chunks each) in the weight ring
constexpr int DEC_CHUNK = DEC_COLS * 128;    // bytes of one chunk (64 rows x 128 B)
constexpr int DEC_KW = 4;                    // compute waves splitting K
constexpr int DEC_LDS = DEC_SLOTS * 4 * DEC_CHUNK;   // 128 KB

template <int BITS>
struct DecShape {
    static constexpr int KB = BITS == 4 ? 128 : 64;   // k per 64-byte block of a weight row
    static constexpr int SPB = KB / 32;               // MFMA steps (32 k) per block
    static constexpr int SPC = 2 * SPB;               // steps per chunk
    static constexpr int KL = KB / 4;                 // k of a block per lane group (q)
};


// ---- prepare: X -> f16 pieces (fragment-major) + exponent per (block, row)
//
// One wave per (row tile, block): lane (q = lane / 16, c = lane % 16) owns
// row 16 mt + c and the KL consecutive k of lane group q, i.e. exactly the
// elements of its own fragments for the SPB steps of the block.
//
// Reduced-precision int4 (BITS 4, one piece) takes bf16 instead: the
// fragments hold bf16(x) (own exponent, no block factor), and in place of
// the exponents the prepare pass writes, per (block, row), the fp32 term
// -136 * sum over the block of bf16(x): the GEMM feeds the codes as
// 128 + (code + 8), exact in bf16, and this term removes the offset 136.
template <int BITS, int P>
__global__ __launch_bounds__(256) void decode_prep_kernel(const float* __restrict__ X, _Float16* __restrict__ XP,
                                                          int8_t* __restrict__ ex, float* __restrict__ corr, int M,
                                                          int K, int MT) {
    using SH = DecShape<BITS>;
    const int nblk = K / SH::KB;
    const int job = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (job >= MT * nblk) return;   // whole waves only
    const int blk = job % nblk, mt = job / nblk;
    const int lane = threadIdx.x & 63, q = lane >> 4, c = lane & 15;
    const int row = 16 * mt + c;
    float v[SH::KL];
    if (row < M) {
        const float4* src = reinterpret_cast<const float4*>(X + size_t(row) * K + size_t(blk) * SH::KB + SH::KL * q);
#pragma unroll
        for (int i = 0; i < SH::KL / 4; ++i) {
            const float4 f = src[i];
            v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < SH::KL; ++i) v[i] = 0.0f;
    }
    if constexpr (BITS == 4 && P == 1) {
        // bf16 fragments and the offset term. The sum runs in k order within
        // a lane, then over the four lane groups in a fixed tree: every lane
        // of the row gets the same bits.
        float sum = 0.0f;
#pragma unroll
        for (int kk = 0; kk < SH::SPB; ++kk) {
            uint32_t o[4];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const __bf16 lo = __bf16(v[frag_k<BITS>(0, kk, 2 * d)]);
                const __bf16 hi = __bf16(v[frag_k<BITS>(0, kk, 2 * d + 1)]);
                o[d] = uint32_t(__builtin_bit_cast(uint16_t, lo)) | (uint32_t(__builtin_bit_cast(uint16_t, hi)) << 16);
            }
            const int s = blk * SH::SPB + kk;
            *reinterpret_cast<u32x4*>(XP + (size_t(s) * MT + mt) * 512 + lane * 8) = u32x4{o[0], o[1], o[2], o[3]};
        }
#pragma unroll
        for (int i = 0; i < SH::KL; ++i) sum += float(__bf16(v[i]));
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        if (q == 0) corr[size_t(blk) * (16 * MT) + row] = -136.0f * sum;
        return;
    }
    // Block maximum of the row: the four lanes q share row c.
    float mx = 0.0f;
    bool fin = true;
#pragma unroll
    for (int i = 0; i < SH::KL; ++i) {
        mx = fmaxf(mx, fabsf(v[i]));
        fin = fin && __builtin_isfinite(v[i]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const int bad = __shfl_xor(int(!fin), 16) | __shfl_xor(int(!fin), 32) | int(!fin);
    const int bad2 = bad | __shfl_xor(bad, 16);
    // e with mx * 2^e in [2^14, 2^15): mx = 1.f * 2^(E - 127) for a normal mx
    // with biased exponent E. Clamped to +-126 so that 2^e and 2^-e are normal
    // (blocks whose maximum is below 2^-112 keep smaller pieces).
    int e = 0;
    if (mx > 0.0f && !bad2) {
        int E = int(__builtin_bit_cast(uint32_t, mx) >> 23) & 0xFF;
        if (E == 0) {   // subnormal maximum
            int ee;
            (void)frexpf(mx, &ee);
            E = ee + 126;
        }
        e = min(126, max(-126, 141 - E));
    }
    if (q == 0) ex[size_t(blk) * (16 * MT) + row] = int8_t(e);
    const float pw = __builtin_bit_cast(float, uint32_t(e + 127) << 23);   // 2^e
    const float nan = __builtin_nanf("");
#pragma unroll
    for (int kk = 0; kk < SH::SPB; ++kk) {
        _Float16 h[P][8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float xs = bad2 ? nan : v[frag_k<BITS>(0, kk, t)] * pw;
            const _Float16 h1 = _Float16(xs);
            h[0][t] = h1;
            if constexpr (P == 2) h[1][t] = _Float16(xs - float(h1));
        }
        const int s = blk * SH::SPB + kk;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            u32x4 o;
#pragma unroll
            for (int d = 0; d < 4; ++d)
                o[d] = uint32_t(__builtin_bit_cast(uint16_t, h[p][2 * d])) |
                       (uint32_t(__builtin_bit_cast(uint16_t, h[p][2 * d + 1])) << 16);
            *reinterpret_cast<u32x4*>(XP + ((size_t(s) * MT + mt) * P + p) * 512 + lane * 8) = o;
        }
    }
}

// ---- the GEMM ------------------------------------------------------------------

struct DecArgs {
    const uint8_t* W;      // codes; row stride rowb bytes
    const float* S;        // scales [N, groups]
    const _Float16* XP;    // fragment-major pieces
    const int8_t* ex;      // exponents [blocks][16 MT] (f16 pieces)
    const float* corr;     // offset terms [blocks][16 MT] (bf16 path)
    const float* bias;
    float* Y;
    int M, N, K, groups, gshift, rowb, nchunk, has_bias;
    int mtp;     // row tiles of the prepared pieces and exponents
    int mt0;     // first row tile this launch handles (its MT tiles)
    int spin;    // rounds of every bounded hand-over wait (decode_small_kernel)
};

// The load schedule of a compute wave. Step s (one MFMA step of 32 k)
// issues, in this order: the MT * P activation fragments of step s + D;
// when step s + D starts a block, the block's 4 scale loads (none when the
// scales are in LDS) and MT exponent loads. Then it waits for everything issued at step s - D. The prologue
// issues steps -D .. -1's loads, so the count depends only on s % SPC. The
// weight stream is issued by another wave, whose counter it does not share.
template <int BITS, int MT, int P, int D, bool SL>
struct Schedule {
    using SH = DecShape<BITS>;
    static constexpr bool BF = BITS == 4 && P == 1;
    static constexpr int NA = (SL ? 0 : 4) + MT;   // block loads: 4 scales (unless in LDS), MT exponent or offset-term loads
    static constexpr int issued(int i) { return MT * P + ((i + D) % SH::SPB == 0 ? NA : 0); }
    static constexpr int wait(int i) {     // vmcnt before computing step position i
        int n = 0;
        for (int t = i - D + 1; t <= i; ++t) n += issued(((t % SH::SPC) + SH::SPC) % SH::SPC);
        return n;
    }
};


// 4 MW + 1 waves: compute wave w takes chunks kw, kw + 4, ... (kw = w % 4;
// interval t holds chunks 4t .. 4t + 3) for row tiles MT mh .. MT mh + MT - 1
// (mh = w / 4); wave 4 MW streams the weight chunks into a ring of DEC_SLOTS
// intervals (DEC_SLOTS - 1 intervals ahead). With MW = 2 two compute waves
// share each SIMD and convert the same codes for different rows: one wave's
// conversions and waits run beside the other's MFMAs, and each wave keeps
// half the accumulators, which leaves registers for a deeper activation
// prefetch. One barrier per interval: interval t is in LDS and every compute
// wave is done with interval t - 1, whose slot the producer then refills.
// With SL the producer also moves the workgroup's scales once (after interval
// 0), transposed to [group][64 columns] behind the ring: a compute wave then
// reads a block's 16 columns from LDS (16 consecutive words: no bank
// conflict) instead of gathering them from 16 rows in HBM.
template <int BITS, int MT, int P, int D, int MW, bool SL>
__global__ __launch_bounds__(64 * (DEC_KW * MW + 1), 1) void decode_kernel(DecArgs a) {
    using SH = DecShape<BITS>;
    using SC = Schedule<BITS, MT, P, D, SL>;
    constexpr bool BF = SC::BF;   // reduced-precision int4: bf16 fragments, offset codes
    using XF = std::conditional_t<BF, bf16x8, f16x8>;
    static_assert(D >= 1 && D <= SH::SPB, "prefetch depth: at most one block ahead");
    // Activation ring: XR step slots, a power of two above D dividing SPC, so
    // that the slot of step s0 + i (s0 a chunk start) is i % XR.
    constexpr int XR = D < 2 ? 2 : (D < 4 ? 4 : 8);
    static_assert(SH::SPC % XR == 0, "ring slots per chunk");
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, c = lane & 15;
    const int n0 = blockIdx.x * DEC_COLS;
    const int T = (a.nchunk + 3) / 4;
    // Interval t of this workgroup holds chunks 4 ((t + rot) % T) + 0..3:
    // workgroups start at different K offsets, so the weight rows they read
    // at the same moment are spread over K rather than all at one offset
    // (whole intervals only).
    const int rot = a.nchunk % 4 == 0 ? int(blockIdx.x % unsigned(T)) : 0;
    auto iv = [&](int t) { return (t + rot) % T; };

    if (w == DEC_KW * MW) {
        // ---- producer. Instruction i of a chunk covers rows 8i .. 8i+7;
        // lane l lands at slot l % 8 of row 8i + l / 8 and fetches the
        // piece that belongs there. Rows past N re-read row N - 1; chunks
        // past the end re-read the last chunk into a free slot.
        const int drow = lane >> 3, dslot = lane & 7;
        uint32_t doff[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 8 * i + drow;
            const int piece = dslot ^ (r & 7);
            doff[i] = uint32_t(min(n0 + r, a.N - 1)) * uint32_t(a.rowb) + 16u * uint32_t(piece);
        }
        const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
        auto dma_interval = [&](int t) {
#pragma unroll
            for (int cw = 0; cw < 4; ++cw) {
                const int chunk = min(4 * iv(t < T ? t : T - 1) + cw, a.nchunk - 1);
                const uint32_t lds = lds0 + uint32_t((t % DEC_SLOTS) * 4 + cw) * DEC_CHUNK;
                // M0 carries the LDS destination of a direct-to-LDS load. The
                // compiler reserves M0 but uses it in this kernel for nothing
                // else (no LDS-DMA builtins, no indexed register access).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds + i * 1024),
                                 "v"(doff[i] + uint32_t(chunk) * 128u), "s"(a.W)
                                 : "memory", "m0");
#pragma clang diagnostic pop
            }
        };
        static_assert(DEC_SLOTS == 4, "the waits below count at most two intervals ahead");
        dma_interval(0);
        if constexpr (SL) {
            // Scales: one 4-byte gather per group, lane l = row n0 + l
            // (rows past N re-read row N - 1).
            const uint32_t srow = uint32_t(min(n0 + lane, a.N - 1)) * uint32_t(a.groups) * 4u;
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
            for (int g = 0; g < a.groups; ++g)
                asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds0 + DEC_LDS + g * 256),
                             "v"(srow + 4u * uint32_t(g)), "s"(a.S)
                             : "memory", "m0");
#pragma clang diagnostic pop
        }
        for (int t = 1; t < DEC_SLOTS - 1 && t < T; ++t) dma_interval(t);
        for (int t = 0; t < T; ++t) {
            // Interval t has landed once at most `ahead` newer intervals (32
            // loads each, issued after it) are in flight; no interval past T
            // is ever issued. The counter holds at most 63, so with two ahead
            // this also waits for the first load of interval t + 1. The
            // scales, issued between intervals 0 and 1, have landed at t = 0.
            const int ahead = min(T - 1 - t, DEC_SLOTS - 2);
            if (ahead >= 2)
                asm volatile("s_waitcnt vmcnt(63)" ::: "memory");
            else if (ahead == 1)
                asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (t + DEC_SLOTS - 1 < T) dma_interval(t + DEC_SLOTS - 1);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();   // the ring is quiet: the partials may overwrite it
        __syncthreads();   // partials written
        return;
    }

    // ---- compute wave w: chunks kw + 4t, SPC steps each, row tiles
    // tile0 .. tile0 + MT - 1 of the prepared pieces.
    const int kw = w % DEC_KW, mh = w / DEC_KW;
    const int tile0 = a.mt0 + mh * MT;
    const int cnt = a.nchunk > kw ? (a.nchunk - kw + 3) / 4 : 0;
    const int nsteps = cnt * SH::SPC;

    XF xa[XR][MT][P];
    const uint32_t xlane = uint32_t(lane) * 16u;
    auto load_x = [&](int s, int slot) {   // this wave's step s (clamped)
        const int ss = s < nsteps ? s : nsteps - 1;
        const int gstep = (kw + 4 * iv(ss / SH::SPC)) * SH::SPC + ss % SH::SPC;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int p = 0; p < P; ++p)
                asm volatile("global_load_dwordx4 %0, %1, %2"
                             : "=v"(xa[slot][mt][p])
                             : "v"(((uint32_t(gstep) * a.mtp + tile0 + mt) * P + p) * 1024u + xlane), "s"(a.XP));
    };
    // Block loads: scales of the lane's 4 columns, and for its rows
    // 16 mt + 4 q .. +3 the exponents (f16 pieces: one dword per row tile) or
    // the offset terms (bf16: one 16-byte load per row tile). With D <= SPB
    // at most the next block is in flight, so two slots (block b in slot
    // b & 1; a chunk holds blocks 2j and 2j + 1).
    float bs[2][4];
    uint32_t be[2][BF ? 1 : MT];
    f32x4 bc[2][BF ? MT : 1];
    auto load_blk = [&](int b, int slot) {   // this wave's block b (clamped)
        const int bb = b < 2 * cnt ? b : 2 * cnt - 1;
        const int gblk = 2 * (kw + 4 * iv(bb >> 1)) + (bb & 1);
        if constexpr (!SL) {
            const uint32_t g = uint32_t(gblk) >> a.gshift;
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                const uint32_t n = uint32_t(min(n0 + 16 * ct + c, a.N - 1));
                asm volatile("global_load_dword %0, %1, %2"
                             : "=v"(bs[slot][ct])
                             : "v"((n * a.groups + g) * 4u), "s"(a.S));
            }
        }
        if constexpr (BF) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                asm volatile("global_load_dwordx4 %0, %1, %2"
                             : "=v"(bc[slot][mt])
                             : "v"((uint32_t(gblk) * (16u * a.mtp) + 16u * (tile0 + mt) + 4u * q) * 4u), "s"(a.corr));
        } else {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                asm volatile("global_load_dword %0, %1, %2"
                             : "=v"(be[slot][mt])
                             : "v"(uint32_t(gblk) * (16u * a.mtp) + 16u * (tile0 + mt) + 4u * q), "s"(a.ex));
        }
    };

    f32x4 acc[MT][4], tmp[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) acc[mt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    u32x4 wc[4];   // the lane's 16-byte code piece of the current block, per column tile

    if (cnt > 0) {
#pragma unroll
        for (int t = -D; t < 0; ++t) {
            load_x(t + D, (t + D) % XR);
            if ((t + D) % SH::SPB == 0) load_blk((t + D) / SH::SPB, ((t + D) / SH::SPB) & 1);
        }
    }
    for (int j = 0; j < T; ++j) {
        __syncthreads();   // interval j is in LDS
        if (j >= cnt) continue;
        const uint8_t* cs = smem + ((j % DEC_SLOTS) * 4 + kw) * DEC_CHUNK;
        const int s0 = j * SH::SPC;
#pragma unroll
        for (int i = 0; i < SH::SPC; ++i) {
            const int s = s0 + i;
            load_x(s + D, (i + D) % XR);
            if ((i + D) % SH::SPB == 0) load_blk((s + D) / SH::SPB, ((i + D) / SH::SPB) & 1);
            // Everything issued at step s - D (and before) has landed.
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(SC::wait(i)) : "memory");
            const int slot = i % XR;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int p = 0; p < P; ++p) asm volatile("" : "+v"(xa[slot][mt][p]));

            const int kk = i % SH::SPB, hb = i / SH::SPB;   // step in block, block in chunk
            if constexpr (BF) {
                if (kk == 0) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) asm volatile("" : "+v"(bc[hb][mt]));
                }
            }
            if (kk == 0) {
                // The block's code pieces: row 16 ct + c, piece 4 hb + q.
#pragma unroll
                for (int ct = 0; ct < 4; ++ct) {
                    const int r = 16 * ct + c;
                    const int sl = (4 * hb + q) ^ (r & 7);
                    wc[ct] = *reinterpret_cast<const u32x4*>(cs + r * 128 + sl * 16);
                }
                if constexpr (SL) {
                    const int g = (2 * (kw + 4 * iv(j)) + hb) >> a.gshift;
                    const float* sc = reinterpret_cast<const float*>(smem + DEC_LDS) + g * 64 + c;
#pragma unroll
                    for (int ct = 0; ct < 4; ++ct) bs[hb][ct] = sc[16 * ct];
                }
            }
            // B fragments of this step and the MFMAs.
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                if constexpr (BF) {
                    // A block's partial starts from its offset term: the
                    // offset leaves inside the fp32 accumulation, before the
                    // scale (exact when the activations are small integers).
                    const bf16x8 b = codes_to_bf16_off(wc[ct][kk]);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const f32x4 t0 = kk == 0 ? bc[hb][mt] : tmp[mt][ct];
                        tmp[mt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[slot][mt][0], b, t0, 0, 0, 0);
                    }
                } else {
                    f16x2 h[4];
                    if constexpr (BITS == 4) {
                        codes_to_f16<4>(wc[ct][kk], h);
                    } else {
                        codes_to_f16<8>(wc[ct][2 * kk], h);
                        codes_to_f16<8>(wc[ct][2 * kk + 1], h + 2);
                    }
                    const f16x8 b = {h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        f32x4 t0 = kk == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : tmp[mt][ct];
#pragma unroll
                        for (int p = 0; p < P; ++p)
                            t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[slot][mt][p], b, t0, 0, 0, 0);
                        tmp[mt][ct] = t0;
                    }
                }
            }
            if (kk == SH::SPB - 1) {
                const int bslot = (i / SH::SPB) & 1;
                asm volatile("" : "+v"(bs[bslot][0]), "+v"(bs[bslot][1]), "+v"(bs[bslot][2]), "+v"(bs[bslot][3]));
                if constexpr (BF) {
                    // Block done: acc += partial * scale.
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                acc[mt][ct][r] = __builtin_fmaf(tmp[mt][ct][r], bs[bslot][ct], acc[mt][ct][r]);
                } else {
                    // Block done: acc += (partial * 2^-e) * scale, per row.
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        asm volatile("" : "+v"(be[bslot][mt]));
                        const uint32_t e4 = be[bslot][mt];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            // 2^-e as an fp32 bit pattern (|e| <= 127: a normal power of two).
                            const float inv =
                                __builtin_bit_cast(float, uint32_t(127 - int(int8_t(e4 >> (8 * r)))) << 23);
#pragma unroll
                            for (int ct = 0; ct < 4; ++ct)
                                acc[mt][ct][r] = __builtin_fmaf(tmp[mt][ct][r] * inv, bs[bslot][ct], acc[mt][ct][r]);
                        }
                    }
                }
            }
        }
    }
    // Loads past the end (clamped re-reads) land before their registers are
    // reused.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int sl = 0; sl < XR; ++sl)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int p = 0; p < P; ++p) asm volatile("" : "+v"(xa[sl][mt][p]));
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
        asm volatile("" : "+v"(bs[sl][0]), "+v"(bs[sl][1]), "+v"(bs[sl][2]), "+v"(bs[sl][3]));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if constexpr (BF)
                asm volatile("" : "+v"(bc[sl][mt]));
            else
                asm volatile("" : "+v"(be[sl][mt]));
        }
    }
    // ---- the four K parts' partials, summed in a fixed order. Layout
    // [kw][column][16 MT MW rows + 4 pad]: a lane's four rows of one column
    // are one 16-byte store, and the padded column stride (16 MT MW + 4
    // floats) puts 16 consecutive columns on 16 distinct 16-byte bank groups.
    constexpr int RP = 16 * MT * MW + 4;
    static_assert(DEC_KW * 64 * RP * 4 <= DEC_LDS, "partials fit the ring");
    __syncthreads();   // the producer's last loads have landed
    float* red = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
            *reinterpret_cast<f32x4*>(red + (kw * 64 + 16 * ct + c) * RP + 16 * (mh * MT + mt) + 4 * q) = acc[mt][ct];
    __syncthreads();
    const int rows = min(a.M - 16 * a.mt0, 16 * MT * MW);
    // A thread keeps one column (the stride is a multiple of 64). Its bias is
    // loaded and waited for before the first store: a load used only inside
    // the conditional stores makes the compiler wait for all outstanding
    // memory operations, earlier stores included, before each store.
    const int col = threadIdx.x & 63, n = n0 + col;
    if (n >= a.N || w >= DEC_KW * MW) return;   // the stream wave stores nothing
    float bv = a.has_bias ? a.bias[n] : 0.0f;
    asm volatile("" : "+v"(bv));
    for (int m4 = w; m4 < (rows + 3) / 4; m4 += DEC_KW * MW) {
        f32x4 y = *reinterpret_cast<const f32x4*>(red + (0 * 64 + col) * RP + 4 * m4);
#pragma unroll
        for (int v = 1; v < 4; ++v) y += *reinterpret_cast<const f32x4*>(red + (v * 64 + col) * RP + 4 * m4);
        if (a.has_bias) y += bv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * m4 + r;
            if (m < rows) a.Y[size_t(16 * a.mt0 + m) * a.N + n] = y[r];
        }
    }
}

// ---- M <= 16: one launch, activations converted in the workgroup ----------------
//
// Every workgroup reads X itself (fp32; rows past M re-read row M - 1 and give
// accumulator rows that are never stored) and makes the f16 pieces in
// registers, so there is no prepare launch. Eight compute waves, two per
// SIMD so that one wave's LDS and MFMA latencies hide under the other's VALU
// work: wave w takes half h = w / 4 (k 64h .. 64h + 63 for int4, 32h .. for
// int8) of k-block 4t + w % 4. A compute wave moves its 16-row activation
// half-block global -> LDS with direct-to-LDS loads (whole 256- or 128-byte
// row runs; 16-byte slots XOR-swizzled by row, so the fragment reads are
// conflict-free), two half-blocks ahead, into a private three-slot ring: no
// other wave reads it, so nothing guards it. The stream wave moves the
// workgroup's scales once and the weight blocks per interval (interval t =
// k-blocks 4t .. 4t+3) into a three-interval ring. The loop is unrolled over
// the ring so that every LDS slot offset is an immediate. Each half-block has
// its own power-of-two activation factor.
//
// No workgroup barrier per interval (it would hold both waves of a SIMD in
// the same phase): the stream wave publishes in LDS how many intervals have
// landed (after its own load-counter wait), each compute wave adds one to
// its slot's count when it has read an interval, and the stream wave refills
// a slot only when all eight waves have read it. A wave's LDS operations are
// performed in issue order, so a count raised after a wave's reads is seen
// only after those reads. Every wait is bounded (DS_SPIN rounds of s_sleep,
// unless the test hook dgm_debug_wait_limit sets fewer):
// a fault in this protocol gives wrong results, never a hang.
//
// Reduced-precision int4 (one piece) runs on bf16 instead: x rounded to bf16
// keeps its own exponent (no block maximum, no factor, no rescale), and the
// codes enter as 128 + (code + 8), exact in bf16. The offset is removed inside
// the accumulator: one more MFMA per step multiplies the same activations by
// the constant -136, and the code MFMAs of every column tile accumulate onto
// that. The fp32 partial then only takes the group scale.
//
// A non-finite activation propagates: NaN gives a NaN output row, an infinity
// an infinite or NaN one (two pieces: NaN, as inf - f16(inf) is NaN).
constexpr int DS_CW = 8;                     // compute waves
constexpr int DS_THREADS = 64 * (DS_CW + 1); // + the stream wave
constexpr int DS_XS = 3;                     // activation slots per compute wave
constexpr int DS_WS = 3;                     // weight intervals in the ring
constexpr int DS_XSLOT = 4096;               // one activation half-block: 16 rows x KB / 2 x 4 B
constexpr int DS_WBLK = 4096;                // one weight block: 64 rows x 64 B
constexpr int DS_WINT = 4 * DS_WBLK;         // one interval
constexpr int DS_XOFF = 0;
constexpr int DS_WOFF = DS_XOFF + DS_CW * DS_XS * DS_XSLOT;   // 96 KB
constexpr int DS_SOFF = DS_WOFF + DS_WS * DS_WINT;            // 144 KB
constexpr int DS_SMAX = 16384 - 16;                           // scales of 64 rows: groups <= 63
constexpr int DS_FOFF = DS_SOFF + DS_SMAX;                    // hand-over counters (4 x u32)
constexpr int DS_LDS = DS_FOFF + 16;                          // 160 KB
constexpr int DS_SPIN = 1 << 22;                              // bound of every hand-over wait
static_assert(DS_XS == DS_WS, "one unrolled loop walks both rings");
static_assert(DS_CW * 16 * 64 * 4 <= DS_WOFF, "the partials fit the activation slots");

template <int BITS, int P>
__global__ __launch_bounds__(DS_THREADS, 1) void decode_small_kernel(DecArgs a, const float* __restrict__ X) {
    using SH = DecShape<BITS>;
    constexpr int KH = SH::KB / 2;              // k of a half-block (64 or 32)
    constexpr int SPH = KH / 32;                // MFMA steps per half-block (2 or 1)
    constexpr int KLH = KH / 4;                 // k of a half-block per lane group q (16 or 8)
    constexpr int XROW = KH * 4;                // bytes of one activation row of a half-block
    constexpr int PR = XROW / 16;               // 16-byte pieces per row (16 or 8)
    constexpr int XI = 16 * XROW / 1024;        // DMA instructions per activation half-block (4 or 2)
    constexpr int RPI = 1024 / XROW;            // rows per DMA instruction (4 or 8)
    constexpr int PQ = KLH / 4;                 // pieces per lane group q (4 or 2)
    constexpr int RSH = 16 / PR;                // rows sharing a 256-byte bank sweep (1 or 2)
    constexpr bool BF = BITS == 4 && P == 1;    // reduced-precision int4: bf16 path
    using XF = std::conditional_t<BF, bf16x8, f16x8>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, c = lane & 15;
    const int n0 = blockIdx.x * DEC_COLS;
    const int nblk = a.K / SH::KB;
    const int T = (nblk + 3) / 4;
    const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
    // Slot of activation piece p of row r: conflict-free for 16 consecutive rows.
    auto xslot = [](int p, int r) { return p ^ ((r / RSH) % PR); };
    // Hand-over counters: [0] intervals landed, [1 + s] reads of ring slot s
    // (an LDS pointer, so that polling them is a ds_read).
    typedef __attribute__((address_space(3))) uint32_t lds_u32;
    volatile lds_u32* cnt = (volatile lds_u32*)(reinterpret_cast<uintptr_t>(smem) + DS_FOFF);
    if (threadIdx.x < 4) cnt[threadIdx.x] = 0u;
    __syncthreads();
    auto wait_for = [&](int i, uint32_t want) {
        bool met = false;
#pragma nounroll
        for (int spin = 0; spin < a.spin; ++spin) {
            if (__builtin_amdgcn_readfirstlane(cnt[i]) >= want) {
                met = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        // A wait that gave up is reported (dgm_end returns an error): the
        // flag is set by a vector atomic, one lane's value non-zero.
        if (!met) __hip_atomic_fetch_or(&g_wait_gave_up, uint32_t(lane == 0), __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::: "memory");
    };

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    if (w == DS_CW) {
        // ---- stream wave: weight interval t into slot t % DS_WS, two
        // intervals ahead, and once (after interval 0) the scales of rows
        // n0 .. n0+63, transposed to [group][64 columns]: one 4-byte gather
        // per group. Weight DMA instruction i of a block covers rows
        // 16i .. 16i+15: lane l lands at slot l % 4 of row 16i + l / 4 and
        // fetches the piece that belongs there (slot = piece ^ ((row >> 2) & 3)).
        // M0 carries the LDS destination of a direct-to-LDS load. The
        // compiler reserves M0 but uses it in this kernel for nothing else.
        uint32_t woff[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 16 * i + (lane >> 2);
            const int piece = (lane & 3) ^ ((r >> 2) & 3);
            woff[i] = uint32_t(min(n0 + r, a.N - 1)) * uint32_t(a.rowb) + 16u * uint32_t(piece);
        }
        auto dma_interval = [&](int t) {
#pragma unroll
            for (int cw = 0; cw < 4; ++cw) {
                const uint8_t* src = a.W + size_t(min(4 * t + cw, nblk - 1)) * 64;
                const uint32_t lds = lds0 + DS_WOFF + uint32_t((t % DS_WS) * 4 + cw) * DS_WBLK;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds + i * 1024),
                                 "v"(woff[i]), "s"(src)
                                 : "memory", "m0");
            }
        };
        dma_interval(0);
        const uint32_t srow = uint32_t(min(n0 + lane, a.N - 1)) * uint32_t(a.groups) * 4u;
        for (int g = 0; g < a.groups; ++g)
            asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds0 + DS_SOFF + g * 256),
                         "v"(srow + 4u * uint32_t(g)), "s"(a.S)
                         : "memory", "m0");
        if (T > 1) dma_interval(1);
        for (int t = 0; t < T; ++t) {
            // Interval t (and the scales) have landed; interval t + 1 (16
            // loads) may still be in flight.
            if (t + 1 < T)
                asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            cnt[0] = uint32_t(t + 1);
            if (t + 2 < T) {
                // Interval t + 2 refills the slot of t - 1 once all eight
                // compute waves have read t - 1 (its (t - 1) / 3 + 1-th use).
                if (t >= 1) wait_for(1 + (t - 1) % DS_WS, uint32_t(DS_CW * ((t - 1) / DS_WS + 1)));
                dma_interval(t + 2);
            }
        }
        __syncthreads();   // compute waves past their last block
        __syncthreads();   // partials written
        return;
    }

    // ---- compute wave w: half h of k-blocks 4t + w % 4.
    const int wb = w & 3, h = w >> 2;
    const uint32_t xlds = lds0 + DS_XOFF + uint32_t(w * DS_XS) * DS_XSLOT;
    uint32_t xsrc[XI];   // byte offsets, within the half-block's columns of X, of this lane's DMA pieces
#pragma unroll
    for (int j = 0; j < XI; ++j) {
        const int r = RPI * j + lane / PR, s = lane % PR;
        xsrc[j] = uint32_t(min(r, a.M - 1)) * uint32_t(a.K) * 4u + 16u * uint32_t(xslot(s, r));
    }
    auto dma_x = [&](int t, int slot) {   // activation half-block of interval t into slot
        const float* src = X + size_t(min(4 * t + wb, nblk - 1)) * SH::KB + h * KH;
        const uint32_t lds = xlds + uint32_t(slot) * DS_XSLOT;
#pragma unroll
        for (int j = 0; j < XI; ++j)
            asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds + j * 1024), "v"(xsrc[j]),
                         "s"(src)
                         : "memory", "m0");
    };
#pragma clang diagnostic pop

    // LDS byte offsets of this lane's reads in slot 0 (slots are immediates).
    uint32_t xo[PQ];   // activations: row c, pieces PQ q .. PQ q + PQ - 1 (swizzled)
#pragma unroll
    for (int i = 0; i < PQ; ++i) xo[i] = DS_XOFF + uint32_t(w * DS_XS) * DS_XSLOT + c * XROW + (xslot(PQ * q + i, c) << 4);
    uint32_t wo[4];   // bytes 32 h + 8 q .. + 7 of weight row 16 ct + c (piece 2 h + q / 2, swizzled)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
        const int r = 16 * ct + c;
        wo[ct] = DS_WOFF + wb * DS_WBLK + r * 64 + (((2 * h + (q >> 1)) ^ ((r >> 2) & 3)) << 4) + ((q & 1) << 3);
    }
    // Scales of the lane's output columns 16 ct + 4 q .. + 3 ([group][64]).
    const uint32_t so = DS_SOFF + 16u * uint32_t(q);

    // The MFMA takes the weights as A and the activations as B, so the
    // accumulator element r of lane (q, c) is output column 16 ct + 4 q + r
    // of activation row c: the row's factor is the lane's own.
    f32x4 acc[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Activation pieces of a half-block: row c, k = KLH q .. KLH q + KLH - 1,
    // against the power of two 2^e of the row's half-block maximum (the four
    // lanes q of row c meet through two lane swaps). No branch.
    auto convert_x = [&](int slot, XF (&xa)[SPH][P], float& inv) {
        float v[KLH];
#pragma unroll
        for (int i = 0; i < PQ; ++i) {
            const f32x4 f = *reinterpret_cast<const f32x4*>(smem + xo[i] + slot * DS_XSLOT);
            v[4 * i] = f[0]; v[4 * i + 1] = f[1]; v[4 * i + 2] = f[2]; v[4 * i + 3] = f[3];
        }
        if constexpr (BF) {
#pragma unroll
            for (int kk = 0; kk < SPH; ++kk)
#pragma unroll
                for (int t8 = 0; t8 < 8; ++t8) xa[kk][0][t8] = __bf16(v[frag_k<BITS>(0, kk, t8)]);
            inv = 1.0f;
            return;
        } else {
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < KLH; ++i) mx = fmaxf(mx, fabsf(v[i]));
        {
            const auto r32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mx),
                                                              __builtin_bit_cast(uint32_t, mx), false, false);
            mx = fmaxf(__builtin_bit_cast(float, uint32_t(r32[0])), __builtin_bit_cast(float, uint32_t(r32[1])));
            const auto r16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, mx),
                                                              __builtin_bit_cast(uint32_t, mx), false, false);
            mx = fmaxf(__builtin_bit_cast(float, uint32_t(r16[0])), __builtin_bit_cast(float, uint32_t(r16[1])));
        }
        // e with mx * 2^e in [2^14, 2^15): 141 - E for the biased exponent E
        // of mx (of mx * 2^64, less 64, for a subnormal maximum), clamped to
        // +-126 so that 2^e and 2^-e are normal; 0 for an all-zero half-block.
        const int E0 = int(__builtin_bit_cast(uint32_t, mx) >> 23);
        const int Es = int(__builtin_bit_cast(uint32_t, mx * 0x1p64f) >> 23) - 64;
        int e = min(126, max(-126, 141 - (E0 == 0 ? Es : E0)));
        e = mx > 0.0f ? e : 0;
        const float pw = __builtin_bit_cast(float, uint32_t(e + 127) << 23);
        inv = __builtin_bit_cast(float, uint32_t(127 - e) << 23);
#pragma unroll
        for (int kk = 0; kk < SPH; ++kk)
#pragma unroll
            for (int t8 = 0; t8 < 8; ++t8) {
                const float xv = v[frag_k<BITS>(0, kk, t8)];
                const _Float16 h1 = _Float16(xv * pw);
                xa[kk][0][t8] = h1;
                if constexpr (P == 2) xa[kk][1][t8] = _Float16(__builtin_fmaf(xv, pw, -float(h1)));
            }
        }
    };

    // The half-block's weights (interval slot) against the converted activations.
    auto weights = [&](int t, int slot, const XF (&xa)[SPH][P], float inv) {
        const int gb = 4 * t + wb;
        u32x2 wd[4];
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) wd[ct] = *reinterpret_cast<const u32x2*>(smem + wo[ct] + slot * DS_WINT);
        const uint32_t gs = so + uint32_t(gb >> a.gshift) * 256u;
        float f[4][4];   // 2^-e * scale of column 16 ct + 4 q + r
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const f32x4 sv = *reinterpret_cast<const f32x4*>(smem + gs + 64 * ct);
#pragma unroll
            for (int r = 0; r < 4; ++r) f[ct][r] = BF ? sv[r] : inv * sv[r];
        }
        f32x4 tmp[4];
        if constexpr (BF) {
            // -136 * sum of the activations, then the biased codes on top.
            const __bf16 n136 = __bf16(-136.0f);
            const bf16x8 neg = {n136, n136, n136, n136, n136, n136, n136, n136};
            f32x4 corr = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kk = 0; kk < SPH; ++kk) corr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(neg, xa[kk][0], corr, 0, 0, 0);
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                f32x4 t0 = corr;
#pragma unroll
                for (int kk = 0; kk < SPH; ++kk)
                    t0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(codes_to_bf16_off(wd[ct][kk]), xa[kk][0], t0, 0, 0, 0);
                tmp[ct] = t0;
            }
        } else {
#pragma unroll
        for (int kk = 0; kk < SPH; ++kk) {
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                f16x2 hv[4];
                if constexpr (BITS == 4) {
                    codes_to_f16<4>(wd[ct][kk], hv);
                } else {
                    codes_to_f16<8>(wd[ct][0], hv);
                    codes_to_f16<8>(wd[ct][1], hv + 2);
                }
                const f16x8 b = {hv[0][0], hv[0][1], hv[1][0], hv[1][1], hv[2][0], hv[2][1], hv[3][0], hv[3][1]};
                f32x4 t0 = kk == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : tmp[ct];
#pragma unroll
                for (int p = 0; p < P; ++p) t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, xa[kk][p], t0, 0, 0, 0);
                tmp[ct] = t0;
            }
        }
        }
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[ct][r] = __builtin_fmaf(tmp[ct][r], f[ct][r], acc[ct][r]);
    };

    dma_x(0, 0);
    if (T > 1) dma_x(1, 1);
    for (int t0 = 0; t0 < T; t0 += DS_XS) {
#pragma unroll
        for (int u = 0; u < DS_XS; ++u) {
            const int t = t0 + u;
            if (t >= T) break;
            if (t + 2 < T) dma_x(t + 2, (u + 2) % DS_XS);   // own slot of t - 1, read completely
            if (t + 2 < T)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * XI) : "memory");
            else if (t + 1 < T)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(XI) : "memory");
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            // The activations need no other wave: convert them before the
            // barrier that hands over the weights.
            const bool live = 4 * t + wb < nblk;
            XF xa[SPH][P];
            float inv = 1.0f;
            if (live) convert_x(u, xa, inv);
            wait_for(0, uint32_t(t + 1));   // weight interval t is in LDS
            if (live) weights(t, u, xa, inv);
            // This wave's reads of slot u are issued: count them.
            asm volatile("" ::: "memory");
            if (lane == 0)
                __hip_atomic_fetch_add(const_cast<lds_u32*>(cnt + 1 + u), 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }

    // ---- the eight waves' partials, summed in a fixed order (activation
    // slots reused: every wave is past its last block).
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem + DS_XOFF);   // [8][16][64]
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) *reinterpret_cast<f32x4*>(red + (w * 16 + c) * 64 + 16 * ct + 4 * q) = acc[ct];
    __syncthreads();
    // One column per thread (the stride is a multiple of 64); its bias is
    // waited for before the first store, as in decode_kernel.
    const int col = threadIdx.x & 63, n = n0 + col;
    if (n >= a.N || w >= DS_CW) return;   // the stream wave stores nothing
    float bv = a.has_bias ? a.bias[n] : 0.0f;
    asm volatile("" : "+v"(bv));
    for (int m = w; m < a.M; m += DS_CW) {
        float y = red[m * 64 + col];
#pragma unroll
        for (int v = 1; v < DS_CW; ++v) y += red[(v * 16 + m) * 64 + col];
        if (a.has_bias) y += bv;
        a.Y[size_t(m) * a.N + n] = y;
    }
}

// Rounds of every bounded hand-over wait; the test hook dgm_debug_wait_limit
// lowers it to force a give-up (the kernels still end normally).
std::atomic<int> g_wait_limit{DS_SPIN};

template <int BITS, int P>
int launch_decode_small(dgm_gpu* g, const DecArgs& a0, const float* X) {
    auto kern = decode_small_kernel<BITS, P>;
    DecArgs a = a0;
    a.spin = g_wait_limit.load();
    g->spin_waits = true;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, DS_LDS);
    if (e != hipSuccess)
        return dgm::fail(g, DGM_ERR_HIP, "decode: cannot reserve %d bytes of LDS: %s", DS_LDS, hipGetErrorString(e));
    hipLaunchKernelGGL(kern, dim3(unsigned((a.N + DEC_COLS - 1) / DEC_COLS)), dim3(DS_THREADS), DS_LDS, g->stream, a,
                       X);
    return DGM_OK;
}

// Scales of the workgroup's 64 rows behind the weight ring: at most
// (160 KB - DEC_LDS) / 256 = 128 groups; more keep the per-block gathers.
constexpr int DEC_SL_MAX = (160 * 1024 - DEC_LDS) / 256;

template <int BITS, int MT, int P, int D, int MW, bool SL>
int launch_decode_sl(dgm_gpu* g, const DecArgs& a) {
    auto kern = decode_kernel<BITS, MT, P, D, MW, SL>;
    const int lds = DEC_LDS + (SL ? 256 * a.groups : 0);
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess)
        return dgm::fail(g, DGM_ERR_HIP, "decode: cannot reserve %d bytes of LDS: %s", lds, hipGetErrorString(e));
    hipLaunchKernelGGL(kern, dim3(unsigned((a.N + DEC_COLS - 1) / DEC_COLS)), dim3(64 * (DEC_KW * MW + 1)), lds,
                       g->stream, a);
    return DGM_OK;
}

template <int BITS, int MT, int P, int D, int MW = 1>
int launch_decode(dgm_gpu* g, const DecArgs& a) {
    return a.groups <= DEC_SL_MAX ? launch_decode_sl<BITS, MT, P, D, MW, true>(g, a)
                                  : launch_decode_sl<BITS, MT, P, D, MW, false>(g, a);
}

// The one-launch kernel's domain: M <= 16, the scales of 64 rows in LDS (at
// most 63 groups), 32-bit X offsets.
bool small_ok(int M, int K, int groups) {
    return M <= 16 && groups <= DS_SMAX / 256 && int64_t(M) * K * 4 < (int64_t(1) << 32);
}

// Reduced-precision int4 (bf16 fragments) keeps up to four row tiles in one
// group of compute waves; the other modes take three or four row tiles as two
// groups of two (two compute waves per SIMD), with the prefetch depth each
// fits in its register budget.
template <int BITS, int P>
constexpr bool DEC_ONE_GROUP = BITS == 4 && P == 1;
template <int BITS, int P>
constexpr int DEC_D2 = P == 2 ? 1 : 2;

template <int BITS, int P>
int decode_dispatch(dgm_gpu* g, DecArgs& a, const float* X) {
    using SH = DecShape<BITS>;
    if (small_ok(a.M, a.K, a.groups)) return launch_decode_small<BITS, P>(g, a, X);
    // Row tiles of the prepared pieces: for the two-group kernel three are
    // padded to four (zero rows), which it covers as 2 x 2.
    const int MT = (a.M <= 32 || DEC_ONE_GROUP<BITS, P>) ? (a.M + 15) / 16 : 4;
    const int nblk = a.K / SH::KB;
    const size_t xp_bytes = size_t(nblk) * SH::SPB * MT * P * 1024;
    // Exponents (int8) or, on the bf16 path, offset terms (fp32) per (block, row).
    const size_t ex_bytes = size_t(nblk) * 16 * MT * ((BITS == 4 && P == 1) ? 4 : 1);
    uint8_t* ws = static_cast<uint8_t*>(dgm::workspace(g, xp_bytes + ex_bytes + 256));
    if (!ws) return dgm::ws_error(g);
    _Float16* xp = reinterpret_cast<_Float16*>(ws);
    int8_t* ex = reinterpret_cast<int8_t*>(ws + xp_bytes);
    float* corr = reinterpret_cast<float*>(ws + xp_bytes);
    const unsigned jobs = unsigned(MT * nblk);
    hipLaunchKernelGGL((decode_prep_kernel<BITS, P>), dim3((jobs + 3) / 4), dim3(256), 0, g->stream, X, xp, ex, corr,
                       a.M, a.K, MT);
    a.XP = xp;
    a.ex = ex;
    a.corr = corr;
    a.mtp = MT;
    a.mt0 = 0;
    // Prefetch depth: as many activation steps in flight as the registers
    // allow (at most one block ahead). Every variant must fit its register
    // budget without spilling (256 with one compute wave per SIMD, 168 with
    // two): a spilled register whose hand-waited load is still in flight
    // would be copied before it holds the data. build.py checks this.
    constexpr int SPB = SH::SPB;
    switch (MT) {
        case 1: return launch_decode<BITS, 1, P, SPB>(g, a);
        case 2: return launch_decode<BITS, 2, P, (SPB > 2 ? SPB / 2 : 1)>(g, a);
        default: break;
    }
    if constexpr (DEC_ONE_GROUP<BITS, P>)
        return MT == 3 ? launch_decode<BITS, 3, P, 2>(g, a) : launch_decode<BITS, 4, P, 1>(g, a);
    else
        return launch_decode<BITS, 2, P, DEC_D2<BITS, P>, 2>(g, a);
}

}  // namespace

namespace dgm {

void decode_wait_check(dgm_gpu* g) {
    g->spin_waits = false;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return;
    if (cur != g->device && hipSetDevice(g->device) != hipSuccess) return;
    uint32_t flag = 0;
    if (hipMemcpyFromSymbol(&flag, HIP_SYMBOL(g_wait_gave_up), sizeof(flag)) == hipSuccess && flag != 0) {
        const uint32_t zero = 0;
        (void)hipMemcpyToSymbol(HIP_SYMBOL(g_wait_gave_up), &zero, sizeof(zero));
        fail(g, DGM_ERR_HIP, "a decode kernel gave up a bounded in-workgroup wait: its results are not valid");
    }
    if (cur != g->device) (void)hipSetDevice(cur);
}

// The decode kernel's domain: quantized weights, 1 <= M <= 64, blocks inside
// groups (G a multiple of 128 for int4, 64 for int8), whole chunks (K a
// multiple of 256 / 128), 32-bit byte offsets, aligned buffers.
bool decode_ok(int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p) {
    if (bits != 4 && bits != 8) return false;
    if (p->M < 1 || p->M > 64 || p->K == 0 || p->N == 0) return false;
    const uint32_t kb = bits == 4 ? 128 : 64;
    if (p->qGroup == 0 || p->qGroup % kb != 0 || p->K % kb != 0) return false;
    const uint32_t bpg = p->qGroup / kb;   // blocks per group: a power of two
    if ((bpg & (bpg - 1)) != 0) return false;
    // Whole chunks (two blocks) unless the one-launch kernel takes the shape.
    if (!small_ok(int(p->M), int(p->K), int(p->K / p->qGroup)) && p->K % (2 * kb) != 0) return false;
    const int64_t rowb = bits == 4 ? p->K / 2 : p->K;
    if (int64_t(p->N) * rowb >= (int64_t(1) << 32)) return false;
    if (int64_t(p->N) * (p->K / p->qGroup) * 4 >= (int64_t(1) << 32)) return false;
    const int64_t MT = (p->M + 15) / 16;
    if (int64_t(p->K / kb) * (kb / 32) * MT * 2 * 1024 >= (int64_t(1) << 32)) return false;
    return aligned(W, 16) && aligned(X, 16) && aligned(S, 4);
}

int decode_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X, const float* bias, float* Y,
               const dgm_GemmP* p) {
    DecArgs a{};
    a.W = static_cast<const uint8_t*>(W);
    a.S = scale;
    a.bias = bias;
    a.Y = Y;
    a.M = int(p->M);
    a.N = int(p->N);
    a.K = int(p->K);
    a.groups = int(p->K / p->qGroup);
    a.gshift = __builtin_ctz(p->qGroup / (bits == 4 ? 128u : 64u));
    a.rowb = bits == 4 ? a.K / 2 : a.K;
    a.nchunk = a.rowb / 128;
    a.has_bias = p->hasBias != 0;
    const bool exact = g->math == DGM_MATH_FP32;
    if (bits == 4) return exact ? decode_dispatch<4, 2>(g, a, X) : decode_dispatch<4, 1>(g, a, X);
    return exact ? decode_dispatch<8, 2>(g, a, X) : decode_dispatch<8, 1>(g, a, X);
}

}  // namespace dgm

// Test hook (no counterpart in the reference): bounds every hand-over wait of
// the decode kernels to `spins` rounds; 0 restores the default bound.
extern "C" int dgm_debug_wait_limit(int64_t spins) {
    if (spins < 0 || spins > DS_SPIN) return DGM_ERR_ARG;
    g_wait_limit.store(spins ? int(spins) : DS_SPIN);
    return DGM_OK;
}
