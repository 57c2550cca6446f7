// GEMV-like dequant-fused group-quant forward (gfx950), M <= 4 rows:
//
//   Y[m,n] = sum_g S[n,g] * sum_{k in g} code[n,k] * X[m,k]  (+ bias[n])
//
// in the reference's order: an exact partial of code * x per k-block (a block
// never straddles a group), scaled once, bias last
// (metal/kernels.metal:152-209).
//
// The time of such a call is the HBM stream of W. What limits one launch is
// how many cache lines each CU requests, not how many bytes: a load
// instruction whose 64 lanes cover 8 whole 128-byte lines costs about half
// as much as one that covers 16 half lines (the MFMA operand layout read
// straight from W's rows). So the weights move as runs of whole lines:
//
//  * A workgroup owns 64 W rows (output columns) and all of K. Each of its
//    16 waves owns one 128-byte chunk of those rows (K = 4096 int4: 16
//    chunks) and loads it, direct to LDS, into a slot of its own with eight
//    1 KB loads (8 rows x 128 bytes each; 16-byte slots XOR-swizzled by row,
//    so that the MFMA fragment reads are conflict-free). Every wave issues its
//    whole chunk at once, so the entire matrix is requested in the first
//    microsecond, and a wave only reads what it loaded itself: the main loop
//    has no barrier and no hand-over, it waits on its own load counter,
//    which retires loads in issue order.
//  * The workgroup's scales, 64 rows x (K / G) floats, are one contiguous
//    run of S, loaded as 256-byte runs of 4-byte pieces (so that the last
//    row of S ends a load exactly) and needed only in the epilogue.
#include "common.hpp"
#include "decode_codes.hpp"
#include "pieces.hpp"

#include <type_traits>

namespace {

using namespace dgm_codes;
using namespace dgm_pieces;

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int ST_COLS = 64;                  // W rows (output columns) per workgroup
constexpr int ST_CHUNK = ST_COLS * 128;      // one chunk: 64 rows x 128 bytes
constexpr int ST_LDS_MAX = 160 * 1024 - 512;   // dynamic LDS; the kernel keeps 2^-sigma statically

template <int BITS>
struct StShape {
    static constexpr int KB = BITS == 4 ? 128 : 64;   // k per 64-byte block of a row
};

struct StreamArgs {
    const uint8_t* W;      // codes, row stride rowb bytes
    const float* S;        // scales [N, groups]
    const float* X;        // activations [M, K]
    const float* bias;
    float* Y;
    int M, N, K, groups, gshift, rowb, nchunk, has_bias;
    int ns;                // loads of the scales (256 bytes each)
    uint32_t s_off, x_off; // LDS byte offsets of the scales and of the piece regions
};

// M0 carries the LDS destination of a direct-to-LDS load. The compiler
// reserves M0 but uses it in this kernel for nothing else (no LDS-DMA
// builtins, no indexed register access). Weights are read once per call:
// non-temporal, so that they do not evict X and the scales from L2.
#define ST_DMA(lds, voff, base)                                                                 \
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"(lds), "v"(voff), \
                 "s"(base)                                                                      \
                 : "memory", "m0")

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// ---- GEMV-like calls (M <= 4, P * M <= 16): int8 MFMA ----------------------------
//
// The same weight stream, with the arithmetic of the int8-MFMA skinny kernel
// (gemm_skinny.hip): a code dword becomes B operands by masking (16 * code as
// int8: three bit operations per 8 int4 weights, against nine for the f16
// conversion), and the activations are split exactly into P int8 pieces
// (pieces.hpp) that occupy MFMA rows (virtual row m * P + p, so that the
// accumulator rows 4q .. 4q+3 of a lane hold whole rows' pieces).
//
// With every load issued at once, the memory system serves a CU's requests
// in no useful order: a load issued first may land last. So nothing here
// waits for data another wave needs, and the only data a wave waits for
// before its first weight tile is its own slice of X:
//  * each wave issues its X slice (one 1 KB row run per row), then its share
//    of the workgroup's scales, then its weight chunk (non-temporal, so that
//    the weight stream of one call does not evict X from L2);
//  * each wave splits its own k-range of X into pieces (4 values per lane,
//    one power of two per row over the range, registers -> a private LDS
//    region) and consumes its own weight chunk column tile by column tile as
//    the loads land (two 1 KB loads per tile, waited for by count);
//  * the exact int32 block partials are kept per block and scaled only after
//    the loop, so the scales, published by the epilogue's barrier, are never
//    on the path of a weight tile.
// The epilogue combines in a fixed order: per lane, pieces then blocks with
// their scales (y_w = sum_b s_b * 2^-sigma_w * sum_p 128^-p * part_b,p),
// then the 16 waves by a fixed butterfly; / 16 for int4 codes, bias last.
template <int BITS, int P, int FM, int NW>
__global__ __launch_bounds__(64 * NW, 1) void stream_i8_kernel(StreamArgs a) {
    using SH = StShape<BITS>;
    constexpr int H = BITS == 4 ? 2 : 1;            // MFMAs (64 k each) per block
    constexpr int QB = BITS == 4 ? 32 : 16;         // piece bytes of a block per lane group q
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    static_assert(P * FM <= 16 && FM <= 4, "pieces fill one 16-row tile");
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, c = lane & 15;
    const int n0 = blockIdx.x * ST_COLS;
    const int M = a.M;
    const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
    const bool live = w < a.nchunk;                 // this wave's chunk (host: nchunk <= NW)
    const uint32_t ring = lds0 + uint32_t(w) * ST_CHUNK;
    const int kbeg = 2 * w * SH::KB;                // this wave's k-range [kbeg, kbeg + 2 KB)
    constexpr int RB = 2 * SH::KB;                  // bytes of one piece row (one chunk of k)
    uint8_t* preg = smem + a.x_off + size_t(w) * P * FM * RB;

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    // ---- small loads: this wave's X slice as inline asm (a load the
    // compiler can see would make it wait for every load in flight, the
    // direct-to-LDS ones included, before the first use of its result), then
    // the scales (shared; wave i % NW issues load i).
    const int e0 = lane * 4;                        // this lane's 4 values of the range
    const bool in = live && e0 < RB;
    f32x4 xq[FM];
#pragma unroll
    for (int m = 0; m < FM; ++m) {
        const uint32_t xo = (in && m < M) ? (uint32_t(m) * uint32_t(a.K) + uint32_t(kbeg + e0)) * 4u : 0u;
        asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(xq[m]) : "v"(xo), "s"(a.X) : "memory");
    }
    int nsw = 0;   // scale loads of this wave
    {
        const uint32_t sbase = uint32_t(n0) * uint32_t(a.groups) * 4u;
        const uint32_t send = uint32_t(a.N) * uint32_t(a.groups) * 4u;
        for (int i = w; i < a.ns; i += NW, ++nsw) {
            const uint32_t src = sbase + uint32_t(i) * 256u + 4u * uint32_t(lane);
            asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds0 + a.s_off + uint32_t(i) * 256u),
                         "v"(src < send ? src : send - 4u), "s"(a.S)
                         : "memory", "m0");
        }
    }
    // ---- this wave's weight chunk. Load i covers rows 8i .. 8i+7 (column
    // tile ct is loads 2ct, 2ct + 1); lane l lands at slot l % 8 of row
    // 8i + l / 8 and fetches the piece that belongs there (piece = slot ^
    // (row & 7)). Rows past N re-read row N - 1.
    if (live) {
        const uint32_t co = uint32_t(w) * 128u;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 8 * i + (lane >> 3);
            const int piece = (lane & 7) ^ (r & 7);
            const uint32_t off = uint32_t(min(n0 + r, a.N - 1)) * uint32_t(a.rowb) + 16u * uint32_t(piece) + co;
            ST_DMA(ring + i * 1024, off, a.W);
        }
    }
#pragma clang diagnostic pop
    // X has landed once at most the scale and weight loads are in flight
    // (host: at most 4 scale loads per wave).
    {
        const int younger = nsw + (live ? 8 : 0);
        switch (younger) {
            case 12: wait_vm<12>(); break;
            case 11: wait_vm<11>(); break;
            case 10: wait_vm<10>(); break;
            case 9: wait_vm<9>(); break;
            case 8: wait_vm<8>(); break;
            case 4: wait_vm<4>(); break;
            case 3: wait_vm<3>(); break;
            case 2: wait_vm<2>(); break;
            case 1: wait_vm<1>(); break;
            default: wait_vm<0>(); break;
        }
    }

    // ---- pieces of this wave's k-range, one power of two per row.
    float inv[FM];   // 2^-sigma per row
#pragma unroll
    for (int m = 0; m < FM; ++m) {
        asm volatile("" : "+v"(xq[m]));   // not before the wait above
        inv[m] = 1.0f;
        if (m >= M) continue;
        const float4 xv = make_float4(xq[m][0], xq[m][1], xq[m][2], xq[m][3]);
        const float mx = wave_max(in ? absmax4(0.0f, xv) : 0.0f);
        const int sigma = row_sigma(mx);
        inv[m] = (mx <= 3.4e38f) ? ldexpf(1.0f, -sigma) : __builtin_nanf("");
        if (in) {
            int cp[4][4];
            split_pieces(xv.x, sigma, cp[0]);
            split_pieces(xv.y, sigma, cp[1]);
            split_pieces(xv.z, sigma, cp[2]);
            split_pieces(xv.w, sigma, cp[3]);
#pragma unroll
            for (int pp = 0; pp < P; ++pp) {
                uint8_t* row = preg + size_t(m * P + pp) * RB;
                const uint32_t b0 = uint32_t(cp[0][pp]) & 0xFFu, b1 = uint32_t(cp[1][pp]) & 0xFFu;
                const uint32_t b2 = uint32_t(cp[2][pp]) & 0xFFu, b3 = uint32_t(cp[3][pp]) & 0xFFu;
                if constexpr (BITS == 4) {
                    // k = e0 .. e0+3 (e0 % 4 == 0): even k at byte (k & ~31) + (k & 31) / 2,
                    // odd k 16 bytes further (piece_off).
                    const int off = piece_off<4>(e0);
                    *reinterpret_cast<uint16_t*>(row + off) = uint16_t(b0 | (b2 << 8));
                    *reinterpret_cast<uint16_t*>(row + off + 16) = uint16_t(b1 | (b3 << 8));
                } else {
                    *reinterpret_cast<uint32_t*>(row + e0) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
                }
            }
        }
    }
    // The wave reads back only its own piece writes: LDS operations of one
    // wave complete in order, so a compiler fence is all that is needed.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    f32x4 pf[2][4];   // exact block partials of the chunk's two blocks, per column tile
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) pf[hb][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (live) {
        const int v = c < P * M ? c : 0;             // virtual row of this lane's A fragments
        const uint8_t* arow = preg + size_t(v) * RB + q * QB;
        i32x4 af[2][H];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int h = 0; h < H; ++h) af[hb][h] = *reinterpret_cast<const i32x4*>(arow + hb * SH::KB + 16 * h);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            // Loads 2ct, 2ct + 1 of the chunk have landed.
            if (ct == 0) wait_vm<6>();
            else if (ct == 1) wait_vm<4>();
            else if (ct == 2) wait_vm<2>();
            else wait_vm<0>();
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                const int r = 16 * ct + c;
                const u32x4 wc = *reinterpret_cast<const u32x4*>(
                    smem + uint32_t(w) * ST_CHUNK + r * 128 + (((4 * hb + q) ^ (r & 7)) << 4));
                i32x4 part;
                if constexpr (BITS == 4) {
                    i32x4 be, bo;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        be[d] = int((wc[d] << 4) & 0xF0F0F0F0u);   // even k: 16 * code
                        bo[d] = int(wc[d] & 0xF0F0F0F0u);          // odd k: 16 * code
                    }
                    part = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[hb][0], be, i32x4{0, 0, 0, 0}, 0, 0, 0);
                    part = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[hb][1], bo, part, 0, 0, 0);
                } else {
                    part = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[hb][0], __builtin_bit_cast(i32x4, wc),
                                                                 i32x4{0, 0, 0, 0}, 0, 0, 0);
                }
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) pf[hb][ct][rr] = float(part[rr]);
            }
        }
    } else {
        wait_vm<0>();
    }

    // ---- epilogue, one barrier. A lane's accumulator rows 4q .. 4q+3 hold
    // whole rows' pieces (virtual row m * P + p), so each wave folds them in
    // registers, B_hb = 2^-sigma_m * sum_p 128^-p * part_hb,p (exact powers
    // of two), and stores B [hb][row][64 columns] over its own ring slot (its
    // last read of it precedes these writes in issue order), columns rotated
    // by 4 w. Then lane l of wave w' takes column 4 w' + l / 16 of source
    // wave l % 16 (16 slots 8 KB apart, on 16 banks thanks to the rotation):
    // y_w = s0 B_0 + s1 B_1 with the blocks' scales, and the 16 waves are
    // summed by a fixed butterfly. Waves past the last chunk contribute zero.
    static_assert(NW == 16, "one source wave per lane of a 16-lane group");
    constexpr int RPL = 4 / P;                      // rows per lane
    {
        float* mine = reinterpret_cast<float*>(smem + uint32_t(w) * ST_CHUNK);
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const int m = RPL * q + i;
            if (m < M) {
                const float sc = inv[m < FM ? m : 0];
#pragma unroll
                for (int hb = 0; hb < 2; ++hb)
#pragma unroll
                    for (int ct = 0; ct < 4; ++ct) {
                        const f32x4 t = pf[hb][ct];
                        float u;
                        if constexpr (P == 4)
                            u = t[0] + (t[1] + (t[2] + t[3] * 0.0078125f) * 0.0078125f) * 0.0078125f;
                        else
                            u = t[2 * i] + t[2 * i + 1] * 0.0078125f;
                        mine[(hb * FM + m) * ST_COLS + ((16 * ct + c + 4 * w) & 63)] = u * sc;
                    }
            }
        }
    }
    __syncthreads();
    const float kshift = BITS == 4 ? 0.0625f : 1.0f;   // int4 codes entered as 16 * code
    const float* ss = reinterpret_cast<const float*>(smem + a.s_off);
    const int src = lane & 15, col = 4 * w + (lane >> 4), n = n0 + col;
    const bool slive = src < a.nchunk;
    const float s0 = slive ? ss[col * a.groups + ((2 * src) >> a.gshift)] : 0.0f;
    const float s1 = slive ? ss[col * a.groups + ((2 * src + 1) >> a.gshift)] : 0.0f;
    const float* b0 = reinterpret_cast<const float*>(smem + uint32_t(src) * ST_CHUNK) + ((col + 4 * src) & 63);
    const float* b1 = b0 + FM * ST_COLS;
    for (int m = 0; m < M; ++m) {
        float y = slive ? __builtin_fmaf(b1[m * ST_COLS], s1, b0[m * ST_COLS] * s0) : 0.0f;
        y += __shfl_xor(y, 8, 16);
        y += __shfl_xor(y, 4, 16);
        y += __shfl_xor(y, 2, 16);
        y += __shfl_xor(y, 1, 16);
        if (src == 0 && n < a.N) {
            y *= kshift;
            if (a.has_bias) y += a.bias[n];
            a.Y[size_t(m) * a.N + n] = y;
        }
    }
}

// LDS layout of a call: one 8 KB chunk slot per wave, the scales, the waves'
// piece regions (P * FM rows of one chunk's k each). lds == 0 when the call
// does not fit (more chunks than waves, more than 4 scale loads per wave, or
// too many pieces).
constexpr int ST_WAVES = 16;

struct StPlan {
    int pieces, fm;
    uint32_t s_off, x_off, lds;
};

StPlan st_plan(int bits, bool exact, int M, int groups, int nchunk) {
    StPlan p{};
    const int kb = bits == 4 ? 128 : 64;
    p.pieces = exact ? 4 : 2;
    p.fm = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
    if (M > 4 || p.pieces * p.fm > 16 || nchunk > ST_WAVES || groups > 4 * ST_WAVES) return StPlan{};
    p.s_off = uint32_t(ST_WAVES) * ST_CHUNK;
    p.x_off = (p.s_off + uint32_t(groups) * 256u + 15u) & ~15u;
    p.lds = p.x_off + uint32_t(ST_WAVES * p.pieces * p.fm * 2 * kb);
    if (p.lds > uint32_t(ST_LDS_MAX)) return StPlan{};
    return p;
}

template <int BITS, int P>
int launch_p(dgm_gpu* g, const StreamArgs& a, const StPlan& pl) {
    auto kern = pl.fm == 1 ? stream_i8_kernel<BITS, P, 1, ST_WAVES>
                           : (pl.fm == 2 ? stream_i8_kernel<BITS, P, 2, ST_WAVES> : stream_i8_kernel<BITS, P, 4, ST_WAVES>);
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       int(pl.lds));
    if (e != hipSuccess)
        return dgm::fail(g, DGM_ERR_HIP, "stream: cannot reserve %u bytes of LDS: %s", pl.lds, hipGetErrorString(e));
    hipLaunchKernelGGL(kern, dim3(unsigned((a.N + ST_COLS - 1) / ST_COLS)), dim3(64 * ST_WAVES), pl.lds, g->stream, a);
    return DGM_OK;
}

}  // namespace

namespace dgm {

// The streaming kernel's domain: quantized weights, 1 <= M <= 4, whole
// 128-byte chunks (int4: K % 256 == 0; int8: K % 128 == 0), at most 16
// chunks per row (K <= 4096 int4, 2048 int8), blocks inside groups, at most
// 64 groups (4 scale loads per wave), the pieces in LDS (the fp32 mode: M = 1
// at K = 4096; the reduced mode: M <= 2), 16-byte aligned codes and X,
// 32-bit byte offsets.
bool stream_ok(dgm_gpu* g, int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p) {
    if (bits != 4 && bits != 8) return false;
    if (p->M < 1 || p->M > 4 || p->K == 0 || p->N == 0) return false;
    const uint32_t kb = bits == 4 ? 128 : 64;
    if (p->qGroup == 0 || p->qGroup % kb != 0 || p->K % (2 * kb) != 0) return false;
    const uint32_t bpg = p->qGroup / kb;
    if ((bpg & (bpg - 1)) != 0) return false;
    const int64_t rowb = bits == 4 ? p->K / 2 : p->K;
    const int64_t groups = p->K / p->qGroup;
    if (int64_t(p->N) * rowb >= (int64_t(1) << 32)) return false;
    if (int64_t(p->N) * groups * 4 >= (int64_t(1) << 32)) return false;
    if (st_plan(bits, g->math == DGM_MATH_FP32, int(p->M), int(groups), int(rowb / 128)).lds == 0) return false;
    return aligned(W, 16) && aligned(X, 16) && aligned(S, 4);
}

int stream_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X, const float* bias, float* Y,
               const dgm_GemmP* p) {
    StreamArgs a{};
    a.W = static_cast<const uint8_t*>(W);
    a.S = scale;
    a.X = X;
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
    a.ns = a.groups;
    const bool exact = g->math == DGM_MATH_FP32;
    const StPlan pl = st_plan(bits, exact, a.M, a.groups, a.nchunk);
    if (pl.lds == 0) return fail(g, DGM_ERR_UNSUPPORTED, "stream: the call does not fit LDS");
    a.s_off = pl.s_off;
    a.x_off = pl.x_off;
    if (bits == 4) return exact ? launch_p<4, 4>(g, a, pl) : launch_p<4, 2>(g, a, pl);
    return exact ? launch_p<8, 4>(g, a, pl) : launch_p<8, 2>(g, a, pl);
}

}  // namespace dgm
