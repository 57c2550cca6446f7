// Skinny (M <= 64) dequant-fused group-quant forward on int8 MFMA (gfx950).
//
//   Y[m,n] = sum_g S[n,g] * sum_{k in g} code[n,k] * X[m,k]  (+ bias[n])
//
// This is the order of the reference's quantized kernels: an exact per-group
// partial of code * x, scaled once per group, bias last
// (metal/kernels.metal:152-209).
//
// Decode-shaped GEMMs stream the packed weights from HBM exactly once; the
// design keeps the per-weight VALU work near 0.4 instructions so that the
// stream, not the ALUs, sets the time:
//
//  * Weight codes feed v_mfma_i32_16x16x64_i8 directly. An int4 byte holds two
//    signed nibbles; masking the high nibble in place (b & 0xF0) or shifting
//    the low one up ((b << 4) & 0xF0) gives 16 * code as a signed int8 with no
//    sign-extension work, so one 16-byte load of 32 nibbles becomes the B
//    operands of two MFMAs (even k, odd k) with three bit ops per 8 weights.
//    int8 codes are used as they are.
//  * X is split exactly into int8 pieces against a power-of-two scale 2^-sigma
//    (per row, or per wave k-range in the one-launch variant) chosen so that
//    max|x| * 2^sigma lies in [32, 64):
//        u = x * 2^sigma = c1 + c2 / 128 + c3 / 128^2 + c4 / 128^3 + r,
//    each c in [-64, 64]. The MFMA products and the int32 group sums are exact;
//    the representation error is what limits accuracy: 2^-20 of the range
//    maximum with three pieces, 2^-27 with four. Relative to the output, the
//    error is that fraction of max|x| times sum|w|, so an activation outlier
//    (1e2 - 1e4 x the row's other values) costs three pieces up to ~3e-5 of
//    max|y|: the fp32 mode therefore takes four pieces in the one-launch
//    variant (M <= 4, where they fit one 16-row tile). Calls the library routes
//    here in the fp32 mode are those M <= 3 (four pieces) and the shapes outside
//    the f16 decode kernels' domain (gemm_decode.hip; three pieces). Two pieces
//    (2^-13 of the range maximum) form the reduced-precision mode (bar 1e-2).
//  * Pieces occupy MFMA rows: virtual row v = p * M + m, so M = 1 with three
//    pieces uses 3 of 16 rows of a single tile; the wasted rows cost MFMA
//    cycles only, which this HBM-bound shape has to spare.
//  * The exact int32 group partial is converted and scaled once per k-block
//    (a k-block never straddles a group: the host requires G % 128 == 0 for
//    int4 and G % 64 == 0 for int8).
//
// Work split: a workgroup owns `strips` 16-column strips of W and all of K;
// its waves take contiguous k-block ranges, so every byte of W and of the X
// pieces enters the workgroup once. Loads for the next chunk of k-blocks are
// issued before the MFMAs of the current one. Wave partials are reduced in
// LDS in a fixed order (deterministic results), then the pieces are combined:
//        y = 2^-sigma * (a0 + a1 / 128 + a2 / 128^2) [/ 16 for int4] + bias.
//
// X pieces come either from LDS, computed by every workgroup for the few rows
// of a GEMV-like call (FUSED), or from a workspace written by a one-pass
// prepare kernel (larger M) in fragment-major order: each (k-block, tile, MFMA
// half) is the 64 lanes' 16-byte A fragments as one contiguous 1 KB. Above 64
// virtual rows the tiled kernel (further down) takes over.
#include "common.hpp"
#include "pieces.hpp"

namespace {

using namespace dgm_pieces;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// k values per k-block: one 16-byte load per lane, 4 lanes per row => 64 bytes.
template <int BITS>
struct KBlock {
    static constexpr int K = BITS == 4 ? 128 : 64;
    static constexpr int H = BITS == 4 ? 2 : 1;   // MFMAs (x64 k) per k-block
};

struct SkinnyArgs {
    const uint8_t* W;     // codes; row stride K/2 (int4) or K (int8) bytes
    const float* S;       // scales [N, groups]
    const float* X;       // [M, K] fp32 (FUSED prepare)
    const int8_t* XP;     // pieces [P*M, K] in fragment order (prepared)
    const float* XS;      // 2^-sigma per row (prepared)
    const float* bias;
    float* Y;
    int M, N, K, G, groups;
    int has_bias;
    int gshift;           // log2(k-blocks per group): group of k-block kb = kb >> gshift
    int strips;           // 16-column strips per workgroup (<= template S)
    size_t wave_lds;      // bytes of LDS per wave (pieces, then partial tiles)
    int total_strips;
};

// ---- main kernel ------------------------------------------------------------
// WAVES waves split K into contiguous k-block ranges. A wave holds the codes
// and scales of KBW k-blocks x S strips in registers and issues all of them at
// once, so a workgroup's whole share of W is in flight from the first cycles
// (one round covers K = WAVES * KBW k-blocks; larger K takes more rounds).
// X-piece fragments follow one k-block ahead, from LDS when FUSED, else from
// the prepared workspace.
//
// FUSED (GEMV-like calls): each wave splits only its own k-range of the M rows
// into pieces, against its own power-of-two scale, into a wave-private LDS
// region, so no workgroup barrier precedes the main loop. Each wave then
// stores its partial tiles into its own slot and the epilogue sums the slots
// in wave order, each scaled by that wave's 2^-sigma.
template <int BITS, int P, int T, int S, int KBW, int WAVES, int FM, bool SV>
__global__ __launch_bounds__(64 * WAVES) void skinny_kernel(SkinnyArgs a) {
    static_assert(KBW % 4 == 0, "k-blocks per round must be a multiple of 4");
    constexpr bool FUSED = FM > 0;
    constexpr int KBK = KBlock<BITS>::K;
    constexpr int H = KBlock<BITS>::H;
    constexpr int NT = 64 * WAVES;
    constexpr int XR = FUSED ? WAVES : 1;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float xs_sh[XR][64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l16 = lane & 15;
    const int q = lane >> 4;
    const int M = a.M, N = a.N, K = a.K;
    const int PM = P * M;
    const int strip0 = blockIdx.x * a.strips;
    const int nstrip = min(a.strips, a.total_strips - strip0);
    const int nkb = K / KBK;
    const int per = (nkb + WAVES - 1) / WAVES;
    const int kb_begin = min(nkb, wave * per);
    const int kb_end = min(nkb, kb_begin + per);
    // Loads are never predicated: a masked load that merges zeros into its
    // destination makes the compiler drain every outstanding load first, and
    // at a branch join the wait counts assume the worst path. So addresses are
    // clamped instead: k-blocks past the range re-read the wave's last one
    // (a cache hit, never computed), columns >= N read row 0 (never stored),
    // piece rows >= P*M read row 0 (never combined).
    const int kb_last = kb_end > kb_begin ? kb_end - 1 : 0;
    const size_t wrow = BITS == 4 ? size_t(K) / 2 : size_t(K);
    // Per-wave LDS region: FUSED pieces (P*M rows of per*KBK bytes), then, once
    // the wave is done with them, its partial tiles.
    const int prow = per * KBK;
    const size_t wreg = a.wave_lds;
    uint8_t* myreg = smem + size_t(wave) * wreg;

    const uint8_t* wlane[S];
    const float* slane[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int n = (strip0 + s) * 16 + l16;
        const int nn = (s < nstrip && n < N) ? n : 0;
        wlane[s] = a.W + size_t(nn) * wrow + q * 16;
        slane[s] = a.S + size_t(nn) * a.groups;
    }

    // Scales first, then codes: loads retire in issue order, so k-block c can
    // be computed as soon as its own codes arrive.
    i32x4 wr[KBW][S];
    float sc[KBW][S];
    auto fetch_w = [&](int kb0) {
        if constexpr (SV) {
            // One group per k-block and 4-aligned ranges: the scales of four
            // consecutive k-blocks are one 16-byte load.
#pragma unroll
            for (int c = 0; c < KBW; c += 4) {
                const int kb = kb0 + c < kb_end ? kb0 + c : (kb_last & ~3);
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const float4 v = *reinterpret_cast<const float4*>(slane[s] + kb);
                    sc[c][s] = v.x; sc[c + 1][s] = v.y; sc[c + 2][s] = v.z; sc[c + 3][s] = v.w;
                }
            }
        } else {
#pragma unroll
            for (int c = 0; c < KBW; ++c) {
                const int kb = kb0 + c < kb_end ? kb0 + c : kb_last;
#pragma unroll
                for (int s = 0; s < S; ++s) sc[c][s] = slane[s][kb >> a.gshift];
            }
        }
        __builtin_amdgcn_sched_barrier(0);   // scales stay ahead of the codes
#pragma unroll
        for (int c = 0; c < KBW; ++c) {
            const int kb = kb0 + c < kb_end ? kb0 + c : kb_last;
#pragma unroll
            for (int s = 0; s < S; ++s) wr[c][s] = *reinterpret_cast<const i32x4*>(wlane[s] + size_t(kb) * 64);
        }
    };

    const int8_t* alane[T];
    if constexpr (FUSED) {
        // The wave's x values go into registers before the weight loads, so
        // waiting for them never waits for W (vmcnt retires in issue order).
        const int e0 = lane * 16;                      // element offset in the range
        const int R = (kb_end - kb_begin) * KBK;       // host: per * KBK <= 1024
        const bool in = e0 < R;
        float xv[FM][16];
#pragma unroll
        for (int m = 0; m < FM; ++m) {
            const float* xr = a.X + (in && m < M ? size_t(m) * K + size_t(kb_begin) * KBK + e0 : 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = *reinterpret_cast<const float4*>(xr + 4 * i);
                xv[m][4 * i] = v.x; xv[m][4 * i + 1] = v.y; xv[m][4 * i + 2] = v.z; xv[m][4 * i + 3] = v.w;
            }
        }
        // Keep the machine scheduler from hoisting the weight loads above X.
        __builtin_amdgcn_sched_barrier(0);
        fetch_w(kb_begin);
        int8_t* lx = reinterpret_cast<int8_t*>(myreg);
#pragma unroll
        for (int m = 0; m < FM; ++m) {
            if (m >= M) break;
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                mx = absmax4(mx, make_float4(xv[m][4 * i], xv[m][4 * i + 1], xv[m][4 * i + 2], xv[m][4 * i + 3]));
            mx = wave_max(in ? mx : 0.0f);
            const int sigma = row_sigma(mx);
            if (lane == 0) xs_sh[wave][m] = (mx <= 3.4e38f) ? ldexpf(1.0f, -sigma) : __builtin_nanf("");
            if (in) {
                int8_t* base[P];
#pragma unroll
                for (int p = 0; p < P; ++p) base[p] = lx + size_t(p * M + m) * prow;
                store_pieces16<BITS, P>(base, e0, xv[m], sigma);
            }
        }
        // The wave reads back only its own LDS writes: LDS operations of one
        // wave complete in order, so a compiler fence is all that is needed.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int v = t * 16 + l16;
            alane[t] = lx + size_t(v < PM ? v : 0) * prow - size_t(kb_begin) * KBK +
                       (BITS == 4 ? q * 32 : q * 16);
        }
    } else {
        fetch_w(kb_begin);
        // Prepared pieces are fragment-major (tiled_prepare_kernel with TP = T):
        // fragment (kb, t, h) is 1 KB, lane-contiguous.
#pragma unroll
        for (int t = 0; t < T; ++t) alane[t] = a.XP + size_t(t * H) * 1024 + lane * 16;
    }

    i32x4 af[2][T][H];
    auto fetch_a = [&](int st, int kb) {
        kb = kb < kb_end ? kb : kb_last;
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int h = 0; h < H; ++h) {
                if constexpr (FUSED)
                    af[st][t][h] = *reinterpret_cast<const i32x4*>(alane[t] + size_t(kb) * KBK + h * 16);
                else
                    af[st][t][h] = *reinterpret_cast<const i32x4*>(alane[t] + (size_t(kb) * T * H + h) * 1024);
            }
    };

    f32x4 acc[S][T];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[s][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // One k-block: all MFMAs first, then the epilogue, so the int32 -> fp32
    // scaling of one strip overlaps the MFMAs of the next.
    auto compute = [&](int c, int st) {
        i32x4 bw[S][H];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if constexpr (BITS == 4) {
                const i32x4 w = wr[c][s];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    bw[s][0][j] = int((uint32_t(w[j]) << 4) & 0xF0F0F0F0u);   // even k: 16*code
                    bw[s][1][j] = int(uint32_t(w[j]) & 0xF0F0F0F0u);          // odd k: 16*code
                }
            } else {
                bw[s][0] = wr[c][s];
            }
        }
        i32x4 part[S][T];
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int t = 0; t < T; ++t)
                part[s][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[st][t][0], bw[s][0], i32x4{0, 0, 0, 0}, 0, 0, 0);
        if constexpr (H == 2) {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int t = 0; t < T; ++t)
                    part[s][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[st][t][1], bw[s][1], part[s][t], 0, 0, 0);
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const float sv = sc[c][s];
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[s][t][r] += float(part[s][t][r]) * sv;
        }
    };

    fetch_a(0, kb_begin);
    for (int r0 = kb_begin; r0 < kb_end; r0 += KBW) {
        if (r0 != kb_begin) fetch_w(r0);
#pragma unroll
        for (int c = 0; c < KBW; c += 2) {
            fetch_a(1, r0 + c + 1);
            if (r0 + c < kb_end) compute(c, 0);
            fetch_a(0, r0 + c + 2);
            if (r0 + c + 1 < kb_end) compute(c + 1, 1);
        }
    }

    // -- each wave stores its partial tiles in its own slot; the epilogue sums
    // the slots in wave order (deterministic) and combines the pieces.
    if constexpr (!FUSED) {
        if (threadIdx.x < M) xs_sh[0][threadIdx.x] = a.XS[threadIdx.x];
    }
    float* slot = reinterpret_cast<float*>(myreg);
    if constexpr (FUSED) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");   // pieces reads done
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) slot[(s * T + t) * 256 + (4 * q + r) * 16 + l16] = acc[s][t][r];
    __syncthreads();

    const int ncols = nstrip * 16;
    const float kshift = BITS == 4 ? 0.0625f : 1.0f;   // int4 codes entered as 16 * code
    for (int idx = threadIdx.x; idx < M * ncols; idx += NT) {
        const int m = idx / ncols;
        const int c = idx - m * ncols;
        const int s = c >> 4, col = c & 15;
        const int n = strip0 * 16 + c;
        if (n >= N) continue;
        float y = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float* sl = reinterpret_cast<const float*>(smem + size_t(w) * wreg);
            float u = 0.0f;
#pragma unroll
            for (int p = P - 1; p >= 0; --p) {
                const int v = p * M + m;
                u = sl[(s * T + (v >> 4)) * 256 + (v & 15) * 16 + col] + u * 0.0078125f;
            }
            y += FUSED ? u * xs_sh[FUSED ? w : 0][m] : u;
        }
        if constexpr (!FUSED) y *= xs_sh[0][m];
        y *= kshift;
        if (a.has_bias) y += a.bias[n];
        a.Y[size_t(m) * N + n] = y;
    }
}

template <int BITS, int P, int T, int S, int KBW, int WAVES, int FM, bool SV>
int launch_kernel(dgm_gpu* g, const SkinnyArgs& a0, hipStream_t st) {
    SkinnyArgs a = a0;
    a.total_strips = (a.N + 15) / 16;
    // Aim for one workgroup per CU, at most S strips each.
    int strips = (a.total_strips + g->num_cus - 1) / g->num_cus;
    strips = strips < 1 ? 1 : (strips > S ? S : strips);
    a.strips = strips;
    const unsigned grid = unsigned((a.total_strips + strips - 1) / strips);
    const int per = (a.K / KBlock<BITS>::K + WAVES - 1) / WAVES;
    const size_t slot = size_t(S) * T * 256 * sizeof(float);
    const size_t pieces = FM > 0 ? size_t(P) * a.M * per * KBlock<BITS>::K : 0;
    a.wave_lds = ((slot > pieces ? slot : pieces) + 15) & ~size_t(15);
    const size_t lds = size_t(WAVES) * a.wave_lds;
    auto kern = skinny_kernel<BITS, P, T, S, KBW, WAVES, FM, SV>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess)
            return dgm::fail(g, DGM_ERR_HIP, "skinny: cannot reserve %zu bytes of LDS: %s", lds,
                             hipGetErrorString(e));
    }
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * WAVES), lds, st, a);
    return DGM_OK;
}

// Vector scale loads need one group per k-block, 4-aligned wave ranges and
// 16-byte aligned scale rows.
template <int BITS, int P, int T, int S, int KBW, int WAVES, int FM>
int launch_skinny(dgm_gpu* g, const SkinnyArgs& a, hipStream_t st) {
    const int nkb = a.K / KBlock<BITS>::K;
    const int per = (nkb + WAVES - 1) / WAVES;
    const bool sv = a.gshift == 0 && nkb % 4 == 0 && per % 4 == 0 && a.groups % 4 == 0 &&
                    dgm::aligned(a.S, 16);
    if (sv) return launch_kernel<BITS, P, T, S, KBW, WAVES, FM, true>(g, a, st);
    return launch_kernel<BITS, P, T, S, KBW, WAVES, FM, false>(g, a, st);
}

// ---- tiled decode kernel (virtual rows 17 .. 192, i.e. 8 <= M <= 64) ----------
// For more than a handful of rows the per-workgroup share of X pieces, not W,
// sets the time: the k-split kernel above makes every workgroup read all
// P*M*K bytes of pieces with 16-row fragment loads. Here:
//  * the prepare pass writes the pieces fragment-major: for each k-block, tile
//    and MFMA half, the 64 lanes' 16-byte A fragments are one contiguous 1 KB,
//    so staging is whole-line traffic;
//  * a workgroup owns 64 columns of W (4 strips) over all of K, and its 4 waves
//    split the virtual-row tiles (TW each), so a wave holds only TW x 4 tiles of
//    accumulators;
//  * per chunk of KC k-blocks, the A fragments and the 64 W rows go global ->
//    LDS with direct loads (double-buffered, one barrier per chunk); the W rows
//    land with 16-byte slots XOR-swizzled by row so fragment reads are free of
//    bank conflicts; the scales of the 64 rows are staged once.
// Each k-block: int32 MFMA partials over the k-block, then one fp32 scaling per
// group as in the k-split kernel (the reference's order).

// Prepare: one workgroup per row m of X; fragment-major pieces, zero rows up to
// 16 * TP.
template <int BITS, int P>
__global__ __launch_bounds__(256) void tiled_prepare_kernel(const float* __restrict__ X, int8_t* __restrict__ XP,
                                                            float* __restrict__ XS, int M, int K, int TP) {
    constexpr int KBK = KBlock<BITS>::K, H = KBlock<BITS>::H;
    __shared__ float red[4];
    const int m = blockIdx.x;
    const float* xr = X + size_t(m) * K;
    float mx = 0.0f;
    for (int k = threadIdx.x * 4; k < K; k += 256 * 4) mx = absmax4(mx, *reinterpret_cast<const float4*>(xr + k));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = nmax(nmax(red[0], red[1]), nmax(red[2], red[3]));
    const int sigma = row_sigma(mx);
    if (threadIdx.x == 0) XS[m] = (mx <= 3.4e38f) ? ldexpf(1.0f, -sigma) : __builtin_nanf("");
    for (int k0 = threadIdx.x * 16; k0 < K; k0 += 256 * 16) {
        float x[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(xr + k0 + 4 * i);
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
        int c[16][4];
#pragma unroll
        for (int i = 0; i < 16; ++i) split_pieces(x[i], sigma, c[i]);
        const int kb = k0 / KBK, kk = k0 - kb * KBK;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int v = p * M + m, t = v >> 4, l16 = v & 15;
            if constexpr (BITS == 4) {
                const int q = kk >> 5, half = (kk >> 4) & 1;
                uint32_t e0 = 0, e1 = 0, o0 = 0, o1 = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    e0 |= (uint32_t(c[2 * i][p]) & 0xFFu) << (8 * i);
                    e1 |= (uint32_t(c[8 + 2 * i][p]) & 0xFFu) << (8 * i);
                    o0 |= (uint32_t(c[2 * i + 1][p]) & 0xFFu) << (8 * i);
                    o1 |= (uint32_t(c[8 + 2 * i + 1][p]) & 0xFFu) << (8 * i);
                }
                int8_t* f = XP + size_t((kb * TP + t) * H) * 1024 + (q * 16 + l16) * 16 + half * 8;
                *reinterpret_cast<uint2*>(f) = make_uint2(e0, e1);
                *reinterpret_cast<uint2*>(f + 1024) = make_uint2(o0, o1);
            } else {
                const int q = kk >> 4;
                uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
                for (int i = 0; i < 16; ++i) w[i >> 2] |= (uint32_t(c[i][p]) & 0xFFu) << (8 * (i & 3));
                *reinterpret_cast<uint4*>(XP + size_t(kb * TP + t) * 1024 + (q * 16 + l16) * 16) =
                    make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
    }
    // Padding rows (P*M .. 16*TP - 1) are zero so their products vanish.
    const int nkb = K / KBK;
    for (int v = P * M + m; v < 16 * TP; v += M) {
        const int t = v >> 4, l16 = v & 15;
        for (int e = threadIdx.x; e < nkb * H * 4; e += 256) {
            const int q = e & 3, h = (e >> 2) % H, kb = (e >> 2) / H;
            *reinterpret_cast<uint4*>(XP + size_t((kb * TP + t) * H + h) * 1024 + (q * 16 + l16) * 16) =
                make_uint4(0u, 0u, 0u, 0u);
        }
    }
}

struct TiledArgs {
    const uint8_t* W;
    const float* S;
    const int8_t* XP;
    const float* XS;
    const float* bias;
    float* Y;
    int M, N, K, groups, gshift, has_bias;
};

typedef __attribute__((address_space(1))) const void global_cvoid;
typedef __attribute__((address_space(3))) void lds_void;

template <int BITS, int TW>
struct TiledShape {
    static constexpr int KBK = KBlock<BITS>::K, H = KBlock<BITS>::H;
    static constexpr int TP = 4 * TW;
    static constexpr int KC = TW == 1 ? 4 : 2;               // k-blocks per chunk
    static constexpr int ABYTES = TP * H * KC * 1024;       // A fragments of a chunk
    static constexpr int SPR = KC * 4;                      // 16-byte slots of a W row per chunk
    static constexpr int WBYTES = 64 * SPR * 16;            // 64 W rows
    static constexpr int BUF = ABYTES + WBYTES;
};

template <int BITS, int P, int TW>
__global__ __launch_bounds__(256) void tiled_kernel(TiledArgs a) {
    using SH = TiledShape<BITS, TW>;
    constexpr int KBK = SH::KBK, H = SH::H, TP = SH::TP, KC = SH::KC, SPR = SH::SPR;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, q = lane >> 4;
    const int K = a.K, N = a.N, M = a.M, groups = a.groups;
    const int n0 = blockIdx.x * 64;
    const int nch = K / (KBK * KC);
    const size_t wrow = BITS == 4 ? size_t(K) / 2 : size_t(K);
    float* scl = reinterpret_cast<float*>(smem);                       // [64][groups]
    const int sbytes = (64 * groups * 4 + 15) & ~15;
    uint8_t* bufs = smem + sbytes;

    // -- scales of the 64 rows, once (16-byte units; groups % 4 == 0).
    {
        const int upr = groups >> 2, units = 64 * upr;
        for (int u0 = wave * 64; u0 < units; u0 += 256) {
            const int u = u0 + lane;
            const int row = u / upr, c = u - row * upr;
            const float* src = a.S + size_t(min(n0 + row, N - 1)) * groups + 4 * c;
            __builtin_amdgcn_global_load_lds((global_cvoid*)src, (lds_void*)(smem + u0 * 16), 16, 0, 0);
        }
    }
    // -- one chunk: A fragments (contiguous in XP) and 64 W rows x KC k-blocks.
    auto issue = [&](int ch, int b) {
        uint8_t* dst = bufs + b * SH::BUF;
        const int8_t* asrc = a.XP + size_t(ch) * SH::ABYTES;
        for (int i = wave; i < SH::ABYTES / 1024; i += 4)
            __builtin_amdgcn_global_load_lds((global_cvoid*)(asrc + i * 1024 + lane * 16), (lds_void*)(dst + i * 1024),
                                             16, 0, 0);
        uint8_t* wdst = dst + SH::ABYTES;
        constexpr int RPI = 64 / SPR;   // W rows per instruction
        for (int i = wave; i < SH::WBYTES / 1024; i += 4) {
            const int row = i * RPI + lane / SPR, slot = lane % SPR;
            const uint8_t* src = a.W + size_t(min(n0 + row, N - 1)) * wrow + size_t(ch) * KC * 64 +
                                 ((slot ^ (row & (SPR - 1))) << 4);
            __builtin_amdgcn_global_load_lds((global_cvoid*)src, (lds_void*)(wdst + i * 1024), 16, 0, 0);
        }
    };

    f32x4 acc[4][TW];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < TW; ++t) acc[s][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int ch, int b) {
        const uint8_t* src = bufs + b * SH::BUF;
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) {
            i32x4 af[TW][H];
#pragma unroll
            for (int t = 0; t < TW; ++t)
#pragma unroll
                for (int h = 0; h < H; ++h)
                    af[t][h] = *reinterpret_cast<const i32x4*>(src + ((kk * TP + wave * TW + t) * H + h) * 1024 + lane * 16);
            const int g = (ch * KC + kk) >> a.gshift;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int row = 16 * s + l16;
                const i32x4 w = *reinterpret_cast<const i32x4*>(src + SH::ABYTES + row * (SPR * 16) +
                                                                (((kk * 4 + q) ^ (row & (SPR - 1))) << 4));
                i32x4 bw[H];
                if constexpr (BITS == 4) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        bw[0][j] = int((uint32_t(w[j]) << 4) & 0xF0F0F0F0u);   // even k: 16*code
                        bw[H - 1][j] = int(uint32_t(w[j]) & 0xF0F0F0F0u);      // odd k: 16*code
                    }
                } else {
                    bw[0] = w;
                }
                const float sv = scl[row * groups + g];
#pragma unroll
                for (int t = 0; t < TW; ++t) {
                    i32x4 part = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[t][0], bw[0], i32x4{0, 0, 0, 0}, 0, 0, 0);
                    if constexpr (H == 2) part = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[t][1], bw[1], part, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[s][t][r] += float(part[r]) * sv;
                }
            }
        }
    };

    issue(0, 0);
    for (int ch = 0; ch < nch; ch += 2) {
        __syncthreads();   // chunk ch (and the scales) landed; buffer 1 is free
        issue(min(ch + 1, nch - 1), 1);
        compute(ch, 0);
        if (ch + 1 >= nch) break;
        __syncthreads();
        issue(min(ch + 2, nch - 1), 0);
        compute(ch + 1, 1);
    }

    // -- combine the pieces of each row: y = 2^-sigma (a0 + a1/128 + a2/128^2) [/16] + bias.
    __syncthreads();   // also drains the last (redundant) chunk load
    float* tile = reinterpret_cast<float*>(bufs);   // [16 * TP][64]
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) tile[(16 * (wave * TW + t) + 4 * q + r) * 64 + 16 * s + l16] = acc[s][t][r];
    __syncthreads();
    const float kshift = BITS == 4 ? 0.0625f : 1.0f;
    for (int idx = threadIdx.x; idx < M * 64; idx += 256) {
        const int m = idx >> 6, c = idx & 63;
        const int n = n0 + c;
        if (n >= N) continue;
        float u = 0.0f;
#pragma unroll
        for (int p = P - 1; p >= 0; --p) u = tile[(p * M + m) * 64 + c] + u * 0.0078125f;
        float y = u * a.XS[m];
        y *= kshift;
        if (a.has_bias) y += a.bias[n];
        a.Y[size_t(m) * N + n] = y;
    }
}

inline int K_of(const SkinnyArgs& s) { return s.K; }

template <int BITS, int P, int TW>
int launch_tiled(dgm_gpu* g, const SkinnyArgs& s, hipStream_t st) {
    using SH = TiledShape<BITS, TW>;
    const int TP = SH::TP;
    const size_t xp_bytes = size_t(K_of(s)) / SH::KBK * TP * SH::H * 1024;
    uint8_t* ws = static_cast<uint8_t*>(dgm::workspace(g, xp_bytes + 64 * sizeof(float) + 256));
    if (!ws) return dgm::ws_error(g);
    int8_t* xp = reinterpret_cast<int8_t*>(ws);
    float* xs = reinterpret_cast<float*>(ws + ((xp_bytes + 255) & ~size_t(255)));
    hipLaunchKernelGGL((tiled_prepare_kernel<BITS, P>), dim3(s.M), dim3(256), 0, st, s.X, xp, xs, s.M, s.K, TP);
    TiledArgs a{};
    a.W = s.W; a.S = s.S; a.XP = xp; a.XS = xs; a.bias = s.bias; a.Y = s.Y;
    a.M = s.M; a.N = s.N; a.K = s.K; a.groups = s.groups; a.gshift = s.gshift; a.has_bias = s.has_bias;
    const size_t sbytes = (size_t(64) * s.groups * 4 + 15) & ~size_t(15);
    const size_t lds = sbytes + 2 * size_t(SH::BUF);
    auto kern = tiled_kernel<BITS, P, TW>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess)
            return dgm::fail(g, DGM_ERR_HIP, "skinny: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(e));
    }
    hipLaunchKernelGGL(kern, dim3(unsigned((s.N + 63) / 64)), dim3(256), lds, st, a);
    return DGM_OK;
}

// The tiled kernel's conditions: whole chunks of k-blocks, scale rows in
// 16-byte units that fit LDS next to two buffers, and the combine tile
// (16 * TP x 64 floats) inside the two buffers.
template <int BITS, int TW>
bool tiled_fits(const SkinnyArgs& s) {
    using SH = TiledShape<BITS, TW>;
    if (s.K % (SH::KBK * SH::KC) != 0) return false;
    if (s.groups % 4 != 0 || !dgm::aligned(s.S, 16)) return false;
    const size_t lds = ((size_t(64) * s.groups * 4 + 15) & ~size_t(15)) + 2 * size_t(SH::BUF);
    return lds <= 160 * 1024 && size_t(16) * SH::TP * 64 * 4 <= 2 * size_t(SH::BUF);
}

// GEMV-like calls prepare X inside every workgroup (no second launch): at
// most 4 rows (the kernel's row registers), P * M virtual rows in one 16-row
// tile, and a wave's k-range (a quarter of K) at most 64 lanes x 16 elements.
bool fused_fits(int bits, int M, int K, int P) {
    const int kbk = bits == 4 ? 128 : 64;
    return M <= 4 && P * M <= 16 && ((K / kbk + 3) / 4) * kbk <= 1024;
}

template <int BITS, int P>
int launch_fused(dgm_gpu* g, SkinnyArgs& a, hipStream_t st) {
    if (a.M == 1) return launch_skinny<BITS, P, 1, 2, 8, 4, 1>(g, a, st);
    return launch_skinny<BITS, P, 1, 2, 8, 4, 4>(g, a, st);
}

template <int BITS, int P>
int dispatch_pieces(dgm_gpu* g, SkinnyArgs& a, hipStream_t st) {
    const int M = a.M;
    const int rows = P * M;
    if (fused_fits(BITS, M, a.K, P)) return launch_fused<BITS, P>(g, a, st);
    // Beyond 4 tiles of virtual rows the accumulators of the k-split kernel
    // crowd the register file; the tiled kernel splits the rows over waves.
    if (rows > 64 && rows <= 192) {
        if (rows <= 128 && tiled_fits<BITS, 2>(a)) return launch_tiled<BITS, P, 2>(g, a, st);
        if (tiled_fits<BITS, 3>(a)) return launch_tiled<BITS, P, 3>(g, a, st);
    }
    // Every workgroup reads all of the pieces (P*M*K bytes), so many strips per
    // workgroup; registers then bound waves x k-blocks per round. The pieces
    // are prepared fragment-major for the chosen tile count.
    const int T = (rows + 15) / 16;
    const int TT = T <= 4 ? T : (T <= 8 ? 8 : 12);
    const size_t xp_bytes = size_t(a.K / KBlock<BITS>::K) * TT * KBlock<BITS>::H * 1024;
    uint8_t* ws = static_cast<uint8_t*>(dgm::workspace(g, xp_bytes + 64 * sizeof(float) + 256));
    if (!ws) return dgm::ws_error(g);
    int8_t* xp = reinterpret_cast<int8_t*>(ws);
    float* xs = reinterpret_cast<float*>(ws + ((xp_bytes + 255) & ~size_t(255)));
    hipLaunchKernelGGL((tiled_prepare_kernel<BITS, P>), dim3(M), dim3(256), 0, st, a.X, xp, xs, M, a.K, TT);
    a.XP = xp;
    a.XS = xs;
    if (T <= 1) return launch_skinny<BITS, P, 1, 4, 4, 8, 0>(g, a, st);
    if (T <= 2) return launch_skinny<BITS, P, 2, 4, 4, 8, 0>(g, a, st);
    if (T <= 3) return launch_skinny<BITS, P, 3, 4, 8, 4, 0>(g, a, st);
    if (T <= 4) return launch_skinny<BITS, P, 4, 4, 8, 4, 0>(g, a, st);
    if (T <= 8) return launch_skinny<BITS, P, 8, 4, 4, 4, 0>(g, a, st);
    return launch_skinny<BITS, P, 12, 2, 8, 4, 0>(g, a, st);
}

}  // namespace

namespace dgm {

// True when the skinny kernel handles this forward: quantized weights, M <= 64,
// k-blocks inside groups, 16-byte aligned rows and buffers.
bool skinny_ok(int bits, const void* W, const float* X, const dgm_GemmP* p) {
    if (bits != 4 && bits != 8) return false;
    if (p->M < 1 || p->M > 64 || p->K == 0) return false;
    const int kbk = bits == 4 ? 128 : 64;
    if (p->qGroup == 0 || (p->qGroup % kbk) != 0 || (p->K % kbk) != 0) return false;
    const uint32_t kpg = p->qGroup / kbk;   // k-blocks per group: a power of two
    if ((kpg & (kpg - 1)) != 0) return false;
    if (int64_t(p->N) * (bits == 4 ? p->K / 2 : p->K) > (int64_t(1) << 40)) return false;
    return aligned(W, 16) && aligned(X, 16);
}

int skinny_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X,
               const float* bias, float* Y, const dgm_GemmP* p) {
    SkinnyArgs a{};
    a.W = static_cast<const uint8_t*>(W);
    a.S = scale;
    a.X = X;
    a.bias = bias;
    a.Y = Y;
    a.M = int(p->M);
    a.N = int(p->N);
    a.K = int(p->K);
    a.G = int(p->qGroup);
    a.groups = int(p->K / p->qGroup);
    a.has_bias = p->hasBias != 0;
    a.gshift = __builtin_ctz(p->qGroup / (bits == 4 ? 128u : 64u));
    const bool exact = g->math == DGM_MATH_FP32;
    hipStream_t st = g->stream;
    // The fp32 mode takes four pieces where they fit one tile (M <= 4): the
    // pieces then hold 2^-27 of the maximum of each wave's k-range, so an
    // outlier costs its neighbours nothing measurable. Elsewhere three.
    if (exact && fused_fits(bits, a.M, a.K, 4))
        return bits == 4 ? launch_fused<4, 4>(g, a, st) : launch_fused<8, 4>(g, a, st);
    if (bits == 4) return exact ? dispatch_pieces<4, 3>(g, a, st) : dispatch_pieces<4, 2>(g, a, st);
    return exact ? dispatch_pieces<8, 3>(g, a, st) : dispatch_pieces<8, 2>(g, a, st);
}

// The GEMV-like shapes (M <= 3) where the skinny kernel's one-launch path
// applies in the current math mode (four pieces in the fp32 mode, two in the
// reduced one). From M = 4 on, the f16 decode kernel is as fast (c4 shape).
bool skinny_fused_ok(dgm_gpu* g, int bits, const void* W, const float* X, const dgm_GemmP* p) {
    if (p->M > 3 || !skinny_ok(bits, W, X, p)) return false;
    return fused_fits(bits, int(p->M), int(p->K), g->math == DGM_MATH_FP32 ? 4 : 2);
}

}  // namespace dgm
