// K-sliced decode-shaped forward (gfx950), 2 to 16 rows:
//
//   Y[m,n] = sum_g S[n,g] * sum_{k in g} code[n,k] * X[m,k]  (+ bias[n])
//
// with the arithmetic of the streaming kernel (gemm_stream.hip): exact int8
// pieces of X against 16 * code on int8 MFMA, an exact int32 partial per
// k-block scaled once, bias last (metal/kernels.metal:152-209).
//
// A decode-shaped call is an HBM stream of W, and what one CU can move per
// microsecond is the limit. A workgroup that owns output columns over all of
// K must also receive all M x K activations, which at M = 16 is twice its
// share of the weights. So K is split instead:
//
//  * A workgroup owns 448 W rows (output columns) and one slice of K (two
//    128-byte chunks of each row: 512 k of int4, 256 k of int8), so it
//    receives only its slice of X. For K = 4096, N = 14336 int4 that is 32
//    column groups x 8 slices = 256 workgroups, one per CU.
//  * Each of its 14 waves owns 32 of the rows: it loads their two chunks
//    direct to LDS (eight 1 KB loads of whole 128-byte lines, 16-byte slots
//    XOR-swizzled by row, non-temporal) and their scales, and only ever reads
//    what it loaded itself, waiting on its own load counter.
//  * The slice of X is shared: wave w splits rows w and w + 14 into exact
//    int8 pieces (one power of two per row and slice) in LDS; a barrier
//    publishes them. The workgroup's X and scale loads land before any of
//    its weight loads is issued (a barrier between them): a CU serves its
//    requests in no useful order, and X queued behind 140 KB of weights
//    would hold every wave's first MFMA until the weights had landed.
//  * Per k-block the int32 MFMA partial is exact; its pieces are folded and
//    scaled by the block's group scale in fp32; the slice's partial row is
//    written to a [slice][M][N] fp32 buffer.
//  * slab_sum_kernel adds the slices in order (slice 0 first) and the bias.
//
// The partial sums are the price: 8 slices x M x N x 4 bytes written and read
// again, plus a second launch. Measured on c4 (K = 4096, N = 14336 int4,
// graph replay of rotated weight copies) against the one-launch kernel
// (gemm_decode.hip): fp32 mode M = 2..4 11.4 us vs 11.8-16.7, M = 8 12.6 vs
// 15.6, M = 16 15.9 vs 16.1; reduced mode M = 3..8 11.5-12.0 vs 11.8-12.1,
// M = 16 14.3 vs 12.9. The library routes the fp32 mode up to 16 rows and
// the reduced mode up to 8 rows here.
#include "common.hpp"
#include "pieces.hpp"

namespace {

using namespace dgm_pieces;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int SB_WAVES = 14;
constexpr int SB_CTW = 2;                          // column tiles (16 W rows) per wave
constexpr int SB_ROWS = 16 * SB_CTW;               // W rows per wave
constexpr int SB_COLS = SB_WAVES * SB_ROWS;        // W rows (output columns) per workgroup
constexpr int SB_NCH = 2;                          // 128-byte chunks of a W row per slice
constexpr int SB_WBYTES = SB_ROWS * SB_NCH * 128;  // one wave's weights: 8 KB
constexpr int SB_NB = 2 * SB_NCH;                  // k-blocks (64 bytes of a row) per slice
constexpr int SB_S_OFF = SB_WAVES * SB_WBYTES;     // scales [wave][32 rows][4 blocks]
constexpr int SB_SIG_OFF = SB_S_OFF + SB_WAVES * SB_ROWS * SB_NB * 4;   // 2^-sigma per row
constexpr int SB_X_OFF = SB_SIG_OFF + 16 * 4;      // piece rows
constexpr int SB_MAX_M = 16;

// Bytes of one piece row (one k per byte) of a slice, padded by 16 so that
// the 16 rows of a fragment read start on distinct bank groups.
template <int BITS>
constexpr int sb_xrow() { return (BITS == 4 ? 512 : 256) + 16; }

template <int BITS, int RT>
constexpr int sb_lds() { return SB_X_OFF + 16 * RT * sb_xrow<BITS>(); }

struct SlabArgs {
    const uint8_t* W;      // codes, row stride rowb bytes
    const float* S;        // scales [N, groups]
    const float* X;        // activations [M, K]
    float* part;           // partial sums [slices][M][N]
    int M, N, K, groups, gshift, rowb;
};

#define SB_DMA16(lds, voff, base)                                                               \
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"(lds), "v"(voff), \
                 "s"(base)                                                                      \
                 : "memory", "m0")

template <int N>
__device__ __forceinline__ void sb_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int BITS, int P, int RT>
__global__ __launch_bounds__(64 * SB_WAVES, 1) void slab_kernel(SlabArgs a) {
    constexpr int KS = BITS == 4 ? 512 : 256;       // k of a slice
    constexpr int KB = BITS == 4 ? 128 : 64;        // k of a block
    constexpr int H = BITS == 4 ? 2 : 1;            // MFMAs (64 k each) per block
    constexpr int QB = BITS == 4 ? 32 : 16;         // piece bytes of a block per lane group q
    constexpr int XROW = sb_xrow<BITS>();
    constexpr int RPL = 4 / P;                      // rows per lane in an accumulator tile
    constexpr int XV = KS / 256;                    // 16-byte X loads per lane and row (4 values each)
    static_assert(16 * RT <= P * SB_MAX_M + 15 && RT >= 1, "row tiles");
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, c = lane & 15;
    const int n0 = blockIdx.x * SB_COLS + w * SB_ROWS;   // this wave's first W row
    const int sl = blockIdx.y;                      // the slice: k = KS sl .. KS sl + KS - 1
    const int M = a.M;
    const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    // ---- X rows w and w + 14 of the slice (inline asm, so that the compiler
    // does not wait for the direct-to-LDS loads before using them).
    f32x4 xr[2][XV];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int m = w + SB_WAVES * i;
#pragma unroll
        for (int v = 0; v < XV; ++v) {
            const uint32_t xo =
                m < M ? (uint32_t(m) * uint32_t(a.K) + uint32_t(sl * KS + 256 * v + 4 * lane)) * 4u : 0u;
            asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(xr[i][v]) : "v"(xo), "s"(a.X) : "memory");
        }
    }
    // ---- the scales of this wave's rows and the slice's blocks: lane l of
    // load t takes row 16 t + l / 4, block l % 4 (rows past N re-read row
    // N - 1).
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int r = min(n0 + 16 * t + (lane >> 2), a.N - 1);
        const uint32_t g = uint32_t(sl * SB_NB + (lane & 3)) >> a.gshift;
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(
                         lds0 + uint32_t(SB_S_OFF + (w * SB_ROWS + 16 * t) * SB_NB * 4)),
                     "v"((uint32_t(r) * uint32_t(a.groups) + g) * 4u), "s"(a.S)
                     : "memory", "m0");
    }
    // Every wave's X and scales have landed before any weight load is issued.
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    // ---- this wave's weights: chunk ch, load i covers rows 8i .. 8i+7;
    // lane l lands at slot l % 8 of row 8i + l / 8 and fetches the piece that
    // belongs there (piece = slot ^ (row & 7)).
    const uint32_t wslot = lds0 + uint32_t(w * SB_WBYTES);
#pragma unroll
    for (int ch = 0; ch < SB_NCH; ++ch)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 8 * i + (lane >> 3);
            const int piece = (lane & 7) ^ (r & 7);
            const uint32_t off = uint32_t(min(n0 + r, a.N - 1)) * uint32_t(a.rowb) +
                                 uint32_t((sl * SB_NCH + ch) * 128 + 16 * piece);
            SB_DMA16(wslot + uint32_t(ch * 4096 + i * 1024), off, a.W);
        }
#pragma clang diagnostic pop

    // ---- pieces of rows w, w + 14: one power of two per row over the slice.
    float* sig = reinterpret_cast<float*>(smem + SB_SIG_OFF);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int v = 0; v < XV; ++v) asm volatile("" : "+v"(xr[i][v]));
        const int m = w + SB_WAVES * i;
        if (m >= M) continue;
        float mx = 0.0f;
#pragma unroll
        for (int v = 0; v < XV; ++v) mx = absmax4(mx, make_float4(xr[i][v][0], xr[i][v][1], xr[i][v][2], xr[i][v][3]));
        mx = wave_max(mx);
        const int sigma = row_sigma(mx);
        if (lane == 0) sig[m] = (mx <= 3.4e38f) ? ldexpf(1.0f, -sigma) : __builtin_nanf("");
#pragma unroll
        for (int v = 0; v < XV; ++v) {
            const int e0 = 256 * v + 4 * lane;   // k within the slice
            int cp[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) split_pieces(xr[i][v][j], sigma, cp[j]);
#pragma unroll
            for (int pp = 0; pp < P; ++pp) {
                uint8_t* row = smem + SB_X_OFF + size_t(m * P + pp) * XROW;
                const uint32_t b0 = uint32_t(cp[0][pp]) & 0xFFu, b1 = uint32_t(cp[1][pp]) & 0xFFu;
                const uint32_t b2 = uint32_t(cp[2][pp]) & 0xFFu, b3 = uint32_t(cp[3][pp]) & 0xFFu;
                if constexpr (BITS == 4) {
                    const int off = piece_off<4>(e0);
                    *reinterpret_cast<uint16_t*>(row + off) = uint16_t(b0 | (b2 << 8));
                    *reinterpret_cast<uint16_t*>(row + off + 16) = uint16_t(b1 | (b3 << 8));
                } else {
                    *reinterpret_cast<uint32_t*>(row + e0) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
                }
            }
        }
    }
    // Every wave's pieces and powers of two are in LDS (the direct-to-LDS
    // loads stay in flight: a wave reads only its own, after its own wait).
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // ---- the slice: per block, the A fragments of every row tile, then each
    // column tile's codes as B operands (16 * code as int8).
    float acc[RT][SB_CTW][RPL];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < SB_CTW; ++ct)
#pragma unroll
            for (int i = 0; i < RPL; ++i) acc[rt][ct][i] = 0.0f;
    const float* sc = reinterpret_cast<const float*>(smem + SB_S_OFF) + (w * SB_ROWS + c) * SB_NB;
    const uint8_t* wl = smem + w * SB_WBYTES;
#pragma unroll
    for (int ch = 0; ch < SB_NCH; ++ch) {
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const int blk = 2 * ch + hb;
            // One block's fragments and one column tile's partials live at
            // a time (the register budget of four waves per SIMD).
            __builtin_amdgcn_sched_barrier(0);
            i32x4 af[RT][H];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int h = 0; h < H; ++h)
                    af[rt][h] = *reinterpret_cast<const i32x4*>(smem + SB_X_OFF + (16 * rt + c) * XROW + blk * KB +
                                                                q * QB + 16 * h);
#pragma unroll
            for (int ct = 0; ct < SB_CTW; ++ct) {
                __builtin_amdgcn_sched_barrier(0);
                if (hb == 0) {
                    // Weight loads 4 ch + 2 ct, 4 ch + 2 ct + 1 of this wave have landed.
                    if (ch == 0 && ct == 0) sb_wait<6>();
                    else if (ch == 0) sb_wait<4>();
                    else if (ct == 0) sb_wait<2>();
                    else sb_wait<0>();
                }
                const int r = 16 * ct + c;
                const u32x4 wc = *reinterpret_cast<const u32x4*>(wl + ch * 4096 + r * 128 + (((4 * hb + q) ^ (r & 7)) << 4));
                const float s = sc[16 * ct * SB_NB + blk];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    i32x4 part;
                    if constexpr (BITS == 4) {
                        i32x4 be, bo;
#pragma unroll
                        for (int d = 0; d < 4; ++d) {
                            be[d] = int((wc[d] << 4) & 0xF0F0F0F0u);   // even k: 16 * code
                            bo[d] = int(wc[d] & 0xF0F0F0F0u);          // odd k: 16 * code
                        }
                        part = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[rt][0], be, i32x4{0, 0, 0, 0}, 0, 0, 0);
                        part = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[rt][1], bo, part, 0, 0, 0);
                    } else {
                        part = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[rt][0], __builtin_bit_cast(i32x4, wc),
                                                                     i32x4{0, 0, 0, 0}, 0, 0, 0);
                    }
                    // Accumulator rows 4q .. 4q+3 of the tile are virtual rows
                    // m * P + p: fold the pieces, then scale.
                    if constexpr (P == 4) {
                        const float u = float(part[0]) +
                                        (float(part[1]) + (float(part[2]) + float(part[3]) * 0.0078125f) * 0.0078125f) *
                                            0.0078125f;
                        acc[rt][ct][0] = __builtin_fmaf(u, s, acc[rt][ct][0]);
                    } else {
                        const float u0 = float(part[0]) + float(part[1]) * 0.0078125f;
                        const float u1 = float(part[2]) + float(part[3]) * 0.0078125f;
                        acc[rt][ct][0] = __builtin_fmaf(u0, s, acc[rt][ct][0]);
                        acc[rt][ct][1] = __builtin_fmaf(u1, s, acc[rt][ct][1]);
                    }
                    // Folded here, not deferred (the partials would stay live).
#pragma unroll
                    for (int i = 0; i < RPL; ++i) asm volatile("" : "+v"(acc[rt][ct][i]));
                }
            }
        }
    }

    // ---- the slice's partial rows: 2^-sigma of the row and 1/16 for int4
    // codes (exact powers of two).
    const float kshift = BITS == 4 ? 0.0625f : 1.0f;
#pragma unroll
    for (int ct = 0; ct < SB_CTW; ++ct) {
        const int n = n0 + 16 * ct + c;
        if (n >= a.N) continue;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int i = 0; i < RPL; ++i) {
                const int m = (16 * rt + 4 * q) / P + i;
                if (m < M)   // read once, by the sum kernel: non-temporal
                    __builtin_nontemporal_store(acc[rt][ct][i] * (sig[m] * kshift),
                                                a.part + (size_t(sl) * M + m) * a.N + n);
            }
    }
}

// Y[m, n] = part[0][m][n] + part[1][m][n] + ... (in slice order) + bias[n].
// Four outputs per thread when N % 4 == 0; every load of a group of eight
// slices is issued before the first add.
template <int V>
__global__ __launch_bounds__(256) void slab_sum_kernel(const float* __restrict__ part, const float* __restrict__ bias,
                                                       float* __restrict__ Y, int slices, int M, int N) {
    typedef float fv __attribute__((ext_vector_type(V)));
    const int64_t total = int64_t(M) * N;
    const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * V;
    if (i >= total) return;
    fv y;
    for (int s0 = 0; s0 < slices; s0 += 8) {
        fv v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            v[j] = s0 + j < slices ? *reinterpret_cast<const fv*>(part + int64_t(s0 + j) * total + i) : fv(0.0f);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (s0 + j < slices) y = s0 + j == 0 ? v[j] : y + v[j];
    }
    if (bias) {
        const int n = int(i % N);
#pragma unroll
        for (int e = 0; e < V; ++e) y[e] += bias[n + e];
    }
    *reinterpret_cast<fv*>(Y + i) = y;
}

template <int BITS, int P, int RT>
int launch_slab(dgm_gpu* g, const SlabArgs& a, int slices) {
    auto kern = slab_kernel<BITS, P, RT>;
    constexpr int lds = sb_lds<BITS, RT>();
    static_assert(lds <= 160 * 1024, "slab LDS");
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       lds);
    if (e != hipSuccess)
        return dgm::fail(g, DGM_ERR_HIP, "slab: cannot reserve %d bytes of LDS: %s", lds, hipGetErrorString(e));
    hipLaunchKernelGGL(kern, dim3(unsigned((a.N + SB_COLS - 1) / SB_COLS), unsigned(slices)), dim3(64 * SB_WAVES), lds,
                       g->stream, a);
    return DGM_OK;
}

template <int BITS, int P>
int launch_slab_rt(dgm_gpu* g, const SlabArgs& a, int slices) {
    switch ((a.M * P + 15) / 16) {
        case 1: return launch_slab<BITS, P, 1>(g, a, slices);
        case 2: return launch_slab<BITS, P, 2>(g, a, slices);
        case 3: if constexpr (P == 4) return launch_slab<BITS, P, 3>(g, a, slices); else break;
        case 4: if constexpr (P == 4) return launch_slab<BITS, P, 4>(g, a, slices); else break;
        default: break;
    }
    return dgm::fail(g, DGM_ERR_UNSUPPORTED, "slab: M = %d", a.M);
}

int64_t slab_slices(int bits, int64_t K) { return (bits == 4 ? K / 2 : K) / (SB_NCH * 128); }

}  // namespace

namespace dgm {

// The K-sliced kernel's domain: quantized weights, M <= 16 in the fp32 mode
// and M <= 8 in the reduced mode (measured crossovers), whole slices of
// two 128-byte chunks per row (int4: K % 512 == 0; int8: K % 256 == 0),
// blocks inside groups, at least two slices and 64 workgroups, the partial
// sums within the static scratch size (so that dgm_gemmNT and
// dgm_gemmNT_noalloc route every shape alike), 16-byte aligned codes and X,
// 32-bit byte offsets.
bool slab_ok(dgm_gpu* g, int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p) {
    if (bits != 4 && bits != 8) return false;
    const uint32_t max_m = g->math == DGM_MATH_FP32 ? SB_MAX_M : 8;
    if (p->M < 1 || p->M > max_m || p->K == 0 || p->N == 0) return false;
    const int64_t kb = bits == 4 ? 128 : 64;
    if (p->qGroup == 0 || p->qGroup % kb != 0 || p->K % (2 * SB_NCH * kb) != 0) return false;
    const uint32_t bpg = p->qGroup / uint32_t(kb);
    if ((bpg & (bpg - 1)) != 0) return false;
    const int64_t slices = slab_slices(bits, p->K);
    const int64_t cgroups = (int64_t(p->N) + SB_COLS - 1) / SB_COLS;
    if (slices < 2 || slices * cgroups < 64 || slices > 65535) return false;
    if (slices * p->M * int64_t(p->N) * 4 > int64_t(kScratchBytes)) return false;
    const int64_t rowb = bits == 4 ? p->K / 2 : p->K;
    if (int64_t(p->N) * rowb >= (int64_t(1) << 32)) return false;
    if (int64_t(p->N) * (p->K / p->qGroup) * 4 >= (int64_t(1) << 32)) return false;
    if (int64_t(p->M) * p->K * 4 >= (int64_t(1) << 32)) return false;
    return aligned(W, 16) && aligned(X, 16) && aligned(S, 4);
}

int slab_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X, const float* bias, float* Y,
             const dgm_GemmP* p) {
    const int slices = int(slab_slices(bits, p->K));
    const size_t pbytes = size_t(slices) * p->M * p->N * 4;
    float* part = static_cast<float*>(workspace(g, pbytes));
    if (!part) return ws_error(g);
    SlabArgs a{};
    a.W = static_cast<const uint8_t*>(W);
    a.S = scale;
    a.X = X;
    a.part = part;
    a.M = int(p->M);
    a.N = int(p->N);
    a.K = int(p->K);
    a.groups = int(p->K / p->qGroup);
    a.gshift = __builtin_ctz(p->qGroup / (bits == 4 ? 128u : 64u));
    a.rowb = bits == 4 ? a.K / 2 : a.K;
    const bool exact = g->math == DGM_MATH_FP32;
    int rc;
    if (bits == 4) rc = exact ? launch_slab_rt<4, 4>(g, a, slices) : launch_slab_rt<4, 2>(g, a, slices);
    else rc = exact ? launch_slab_rt<8, 4>(g, a, slices) : launch_slab_rt<8, 2>(g, a, slices);
    if (rc) return rc;
    const int64_t total = int64_t(a.M) * a.N;
    const float* b = p->hasBias ? bias : nullptr;
    if (a.N % 4 == 0 && aligned(Y, 16))
        hipLaunchKernelGGL(slab_sum_kernel<4>, dim3(unsigned((total / 4 + 255) / 256)), dim3(256), 0, g->stream, part,
                           b, Y, slices, a.M, a.N);
    else
        hipLaunchKernelGGL(slab_sum_kernel<1>, dim3(unsigned((total + 255) / 256)), dim3(256), 0, g->stream, part, b,
                           Y, slices, a.M, a.N);
    return DGM_OK;
}

}  // namespace dgm
