// Large-M dequant-fused group-quant forward on bf16 MFMA (gfx950):
//
//   Y[m,n] = sum_k bf16(X[m,k]) * bf16(deq(W)[n,k])  (+ bias[n]),  fp32 accumulate
//
// deq(W)[n,k] = code * S[n, k/G] rounded once to fp32 (the reference's
// dequant, src/Check.swift:433-458), then rounded to bf16 (nearest even).
// This is the reduced-precision path (max relative error <= 1e-2); the
// fp32-accurate forward for the same shapes is gemm_f32_kernel.
//
// Design (prefill shapes, MFMA-bound):
//  * X is converted to bf16 once by a pre-pass (it is re-read by every tile
//    column, so converting it inside the GEMM would repeat the work N/256
//    times).
//  * A workgroup computes a 256 x 256 tile of Y with twelve waves in two
//    roles. Eight MFMA waves each own a 64 x 128 block = 4 x 8
//    v_mfma_f32_16x16x32_bf16 tiles (128 fp32 accumulators) and only read LDS
//    and issue MFMAs. Four producer waves load the X tile (global -> LDS with
//    global_load_lds_dwordx4, no VGPR staging) and the weight codes, and
//    dequantize the codes into the bf16 weight tile in LDS, one weight row
//    per lane. Each SIMD holds two MFMA waves and one producer, so the
//    dequantization's VALU work runs beside the MFMAs. K advances 64 per step.
//  * A wave instruction of the X load fills 1 KB of LDS in lane order, so rows
//    are unpadded (128 B) and the 16-byte chunks of row r sit at slot
//    c ^ (r & 7): each lane fetches the global chunk that belongs in its slot.
//    Fragment reads (16 rows, one chunk) then hit 8 distinct slots per 8-lane
//    group, free of bank conflicts: a probe of ds_read_b128 on gfx950 takes 23
//    cycles per wave instruction with this map, as with contiguous lanes, and
//    32 when rows 8-15 are further XOR-ed by 1. The weight tile uses the same
//    swizzle (its one-row-per-lane stores cost the same either way).
//  * Stages: three for X, two for the weights (160 KB of LDS). During step k
//    the MFMA waves read stage k; the producers store the weights of step k+1
//    (codes loaded during step k-1) and then issue the loads of step k+2, and
//    enter the step's barrier once everything but those loads has landed, so
//    every load has a whole step to arrive. One barrier per step.
//  * Dequant: int4 bytes are flipped to offset binary and masked into the
//    high nibble, so each byte is 16*(code+8) as an unsigned value and
//    converts with one v_cvt_f32_ubyte; fma(f, s/16, -8s) then yields
//    code*s with a single rounding (the exact product minus an exact offset),
//    i.e. the reference's fp32 dequant bit for bit, followed by one
//    v_cvt_pk_bf16_f32 per pair. int8 codes use (code+128) and fma(f, s, -128s).
//  * Tile order is XCD-aware: workgroups are dealt round-robin to the 8 XCDs,
//    so the logical tile index is remapped to give each XCD a contiguous range,
//    walked in groups of 4 tile rows; the ~32 tiles an XCD runs at once then
//    share A and B rows in its L2.
#include "common.hpp"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int RS = BK * 2;        // LDS row stride in bytes (chunks swizzled, no pad)
constexpr int TILE = BM * RS;     // one operand tile (BM == BN)
constexpr int GROUP_M = 4;        // tile rows per group of the XCD-local order

struct Bf16Args {
    const uint16_t* Xb;   // X as bf16 [M, K]
    const uint8_t* W;     // codes [N, K/2] (int4) or [N, K] (int8)
    const float* S;       // scales [N, groups]
    const float* bias;
    float* Y;
    int M, N, K, G, groups, has_bias;
    int tiles_m, tiles_n;
};

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    const bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// X fp32 -> bf16 (nearest even). A block converts 1024 chunks of 8 floats:
// thread t takes chunks t, t + 256, t + 512, t + 768 (consecutive threads on
// consecutive 32-byte chunks), issuing all eight 16-byte loads before the
// first conversion. X is read once here, so its loads bypass the caches'
// retention (non-temporal); the bf16 copy is stored normally, to be re-read
// by the GEMM.
constexpr int CVT_CHUNKS = 4;
__global__ __launch_bounds__(256) void x_to_bf16_kernel(const float* __restrict__ X, uint16_t* __restrict__ Xb,
                                                        int64_t n8) {
    const int64_t base = int64_t(blockIdx.x) * (256 * CVT_CHUNKS) + threadIdx.x;
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4 v[2 * CVT_CHUNKS];
#pragma unroll
    for (int c = 0; c < CVT_CHUNKS; ++c) {
        const int64_t i = min(base + 256 * c, n8 - 1);
        const f32x4* p = reinterpret_cast<const f32x4*>(X) + 2 * i;
        v[2 * c] = __builtin_nontemporal_load(p);
        v[2 * c + 1] = __builtin_nontemporal_load(p + 1);
    }
#pragma unroll
    for (int c = 0; c < CVT_CHUNKS; ++c) {
        const int64_t i = base + 256 * c;
        if (i < n8)
            reinterpret_cast<uint4*>(Xb)[i] =
                make_uint4(pack_bf16(v[2 * c][0], v[2 * c][1]), pack_bf16(v[2 * c][2], v[2 * c][3]),
                           pack_bf16(v[2 * c + 1][0], v[2 * c + 1][1]), pack_bf16(v[2 * c + 1][2], v[2 * c + 1][3]));
    }
}

typedef __attribute__((address_space(1))) const void global_cvoid;
typedef __attribute__((address_space(3))) void lds_void;

// Byte offset of 16-byte chunk c of row r in a swizzled operand tile.
__device__ __forceinline__ int swz(int r, int c) { return r * RS + ((c ^ (r & 7)) << 4); }

// ---- the kernel ------------------------------------------------------------------
// Twelve waves: waves 0-7 only read LDS and issue MFMAs (a 64 x 128 block
// each); waves 8-11 are producers: they issue the X tile's direct-to-LDS loads
// and load, dequantize and store the weight tile of the next step while the
// MFMA waves work on the current one. Waves are dealt to the SIMDs round
// robin, so each SIMD holds two MFMA waves and one producer and the
// dequantization's VALU work overlaps MFMA issue instead of following it.
// LDS: three X stages (the X tile of step k+2 is loaded during step k) and two
// weight stages, 5 x 32 KB.
constexpr int NTW = 768;
constexpr int LDS_WS = 5 * TILE;

template <int BITS>
__global__ __launch_bounds__(NTW) void gemm_bf16_kernel(Bf16Args a) {
    constexpr int CB = BITS == 4 ? 2 : 4;   // 16-byte code loads per producer lane per 64-k step
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int l16 = lane & 15, q = lane >> 4;
    const int M = a.M, N = a.N, K = a.K;

    const int total = a.tiles_m * a.tiles_n;
    int L = blockIdx.x;
    if (total % 8 == 0) L = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    const int group = L / (GROUP_M * a.tiles_n);
    const int first_m = group * GROUP_M;
    const int gm = min(GROUP_M, a.tiles_m - first_m);
    const int within = L - group * GROUP_M * a.tiles_n;
    const int m0 = (first_m + within % gm) * BM;
    const int n0 = (within / gm) * BN;
    const int nk = K / BK;

    if (wave >= 8) {
        // ---- producer p: X rows 64p .. 64p+63 (8 per instruction), W row 64p + lane.
        // Every global load is inline asm and waited for by count: step ks
        // issues X of step ks + 2 (8 direct-to-LDS loads) and then the codes
        // and scales of step ks + 3 (NW loads) into the code buffer it has
        // just dequantized, so codes have two steps to arrive and X stays
        // two steps ahead. (With compiler-visible direct-to-LDS loads the
        // compiler waits for all of them before any LDS store.)
        constexpr int NW = CB + 2;
        const int p = __builtin_amdgcn_readfirstlane(wave - 8);
        const int arl = lane >> 3, aslot = lane & 7;
        uint32_t aoff[8];   // byte offsets into Xb
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = p * 64 + j * 8 + arl;
            aoff[j] = (uint32_t(min(m0 + r, M - 1)) * uint32_t(K) + ((aslot ^ (r & 7)) * 8)) * 2u;
        }
        const int brow = p * 64 + lane;
        const int bn = min(n0 + brow, N - 1);
        const uint32_t boff = uint32_t(bn) * uint32_t(BITS == 4 ? K / 2 : K);
        const uint32_t soff = uint32_t(bn) * uint32_t(a.groups) * 4u;
        const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
        auto xdma = [&](int ks, int st) {
            const uint32_t lds = lds0 + uint32_t(st * TILE + p * 64 * RS);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds + j * 8 * RS),
                             "v"(aoff[j] + uint32_t(ks * BK * 2)), "s"(a.Xb)
                             : "memory", "m0");
        };
#pragma clang diagnostic pop
        auto wload = [&](u32x4 (&c)[CB], float (&s)[2], int ks) {
            const uint32_t k0 = uint32_t(ks * BK);
#pragma unroll
            for (int j = 0; j < CB; ++j)
                asm volatile("global_load_dwordx4 %0, %1, %2"
                             : "=v"(c[j])
                             : "v"(boff + (BITS == 4 ? k0 / 2 : k0) + 16u * j), "s"(a.W));
            asm volatile("global_load_dword %0, %1, %2" : "=v"(s[0]) : "v"(soff + (k0 / a.G) * 4u), "s"(a.S));
            asm volatile("global_load_dword %0, %1, %2" : "=v"(s[1]) : "v"(soff + ((k0 + 32) / a.G) * 4u), "s"(a.S));
        };
        // The loaded registers become visible to the compiler only here,
        // after the wait that covers them.
        auto pin = [](u32x4 (&c)[CB], float (&s)[2]) {
#pragma unroll
            for (int j = 0; j < CB; ++j) asm volatile("" : "+v"(c[j]));
            asm volatile("" : "+v"(s[0]), "+v"(s[1]));
        };
        // k half h (32 k) of the step: chunks 4h .. 4h+3 of the row.
        auto dequant_store = [&](const u32x4 (&c)[CB], const float (&sc)[2], int st) {
            uint8_t* Bs = smem + (3 + st) * TILE;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float s = sc[h];
                if constexpr (BITS == 4) {
                    const float s16 = s * 0.0625f, off = -8.0f * s;
                    const uint32_t w4[4] = {c[h][0], c[h][1], c[h][2], c[h][3]};
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t x = w4[d] ^ 0x88888888u;
                        uint32_t lo = (x << 4) & 0xF0F0F0F0u;
                        uint32_t hi = x & 0xF0F0F0F0u;
                        asm("" : "+v"(lo));
                        asm("" : "+v"(hi));
                        const float fe[4] = {float(lo & 0xFFu), float((lo >> 8) & 0xFFu), float((lo >> 16) & 0xFFu),
                                             float(lo >> 24)};
                        const float fo[4] = {float(hi & 0xFFu), float((hi >> 8) & 0xFFu), float((hi >> 16) & 0xFFu),
                                             float(hi >> 24)};
                        uint32_t o[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            o[i] = pack_bf16(__builtin_fmaf(fe[i], s16, off), __builtin_fmaf(fo[i], s16, off));
                        *reinterpret_cast<uint4*>(Bs + swz(brow, h * 4 + d)) = make_uint4(o[0], o[1], o[2], o[3]);
                    }
                } else {
                    const float off = -128.0f * s;
                    const uint32_t w8[8] = {c[2 * h][0], c[2 * h][1], c[2 * h][2], c[2 * h][3],
                                            c[2 * h + 1][0], c[2 * h + 1][1], c[2 * h + 1][2], c[2 * h + 1][3]};
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        uint32_t o[4];
#pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            const uint32_t x = w8[2 * d + e] ^ 0x80808080u;
                            const float f0 = float(x & 0xFFu), f1 = float((x >> 8) & 0xFFu);
                            const float f2 = float((x >> 16) & 0xFFu), f3 = float(x >> 24);
                            o[2 * e] = pack_bf16(__builtin_fmaf(f0, s, off), __builtin_fmaf(f1, s, off));
                            o[2 * e + 1] = pack_bf16(__builtin_fmaf(f2, s, off), __builtin_fmaf(f3, s, off));
                        }
                        *reinterpret_cast<uint4*>(Bs + swz(brow, h * 4 + d)) = make_uint4(o[0], o[1], o[2], o[3]);
                    }
                }
            }
        };
        u32x4 c0[CB], c1[CB];
        float s0[2], s1[2];
        auto clampk = [&](int ks) { return ks < nk ? ks : nk - 1; };
        // X stage i at i * TILE, weight stage i at (3 + i) * TILE.
        wload(c0, s0, 0);
        xdma(0, 0);
        wload(c1, s1, clampk(1));
        xdma(clampk(1), 1);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(16 + NW) : "memory");   // codes of step 0
        pin(c0, s0);
        dequant_store(c0, s0, 0);
        wload(c0, s0, clampk(2));
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(8 + 2 * NW) : "memory");   // X of step 0
        // Step ks: codes of step ks + 1 are in (cc, cs), issued two steps ago;
        // X of step ks + 1 landed by the barrier.
        auto step = [&](int ks, u32x4 (&cc)[CB], float (&cs)[2]) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(8 + NW) : "memory");
            pin(cc, cs);
            dequant_store(cc, cs, (ks + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            xdma(clampk(ks + 2), (ks + 2) % 3);
            wload(cc, cs, clampk(ks + 3));
            __builtin_amdgcn_sched_barrier(0);
            // Barrier once X of step ks + 1 has landed (the newer loads stay in
            // flight) and every weight store of this wave is done.
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(8 + 2 * NW) : "memory");
        };
        int ks = 0;
        for (; ks + 1 < nk; ks += 2) {
            step(ks, c1, s1);
            step(ks + 1, c0, s0);
        }
        if (ks < nk) step(ks, c1, s1);
        // The last steps' clamped loads (re-reads of the last step, never
        // consumed) land before the wave ends: no direct-to-LDS write may
        // outlive the workgroup's LDS.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        pin(c0, s0);
        pin(c1, s1);
        return;
    }

    // ---- MFMA waves
    const int wm = wave >> 1, wn = wave & 1;
    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int cw0 = ((0 * 4 + q) ^ (l16 & 7)) << 4, cw1 = ((1 * 4 + q) ^ (l16 & 7)) << 4;
    auto compute = [&](int xs, int ws) {
        const uint8_t* As = smem + xs * TILE + (wm * 64 + l16) * RS;
        const uint8_t* Bs = smem + (3 + ws) * TILE + (wn * 128 + l16) * RS;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int cw = kk ? cw1 : cw0;
            bf16x8 af[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const bf16x8*>(As + i * 16 * RS + cw);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const bf16x8 bfj = *reinterpret_cast<const bf16x8*>(Bs + j * 16 * RS + cw);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfj, acc[i][j], 0, 0, 0);
            }
        }
    };
    __syncthreads();
    for (int ks = 0; ks < nk; ++ks) {
        compute(ks % 3, ks & 1);
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int col = n0 + wn * 128 + j * 16 + l16;
        const float bv = (a.has_bias && col < N) ? a.bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm * 64 + i * 16 + 4 * q + r;
                if (row < M && col < N) __builtin_nontemporal_store(acc[i][j][r] + bv, a.Y + size_t(row) * N + col);
            }
    }
}

}  // namespace

namespace dgm {

// The bf16 path takes quantized forwards with M > 64 in the reduced-precision
// mode: K a multiple of 128, every 32-k half inside one group, aligned operands.
bool bf16_ok(int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p) {
    if (bits != 4 && bits != 8) return false;
    if (p->M <= 64 || p->K == 0 || (p->K % (2 * BK)) != 0) return false;
    if (p->qGroup == 0 || (p->qGroup % 32) != 0) return false;   // a thread's 32 k share a group
    if (int64_t(p->M) * p->K >= (int64_t(1) << 32)) return false;   // 32-bit element offsets
    (void)S;
    return aligned(W, 16) && aligned(X, 16);
}

int bf16_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X, const float* bias,
             float* Y, const dgm_GemmP* p) {
    const int64_t mk = int64_t(p->M) * p->K;
    uint16_t* xb = static_cast<uint16_t*>(workspace(g, size_t(mk) * 2));
    if (!xb) return ws_error(g);
    hipStream_t st = g->stream;
    const int64_t n8 = mk / 8;
    hipLaunchKernelGGL(x_to_bf16_kernel, dim3(unsigned((n8 + 256 * CVT_CHUNKS - 1) / (256 * CVT_CHUNKS))), dim3(256), 0,
                       st, X, xb, n8);

    Bf16Args a{};
    a.Xb = xb;
    a.W = static_cast<const uint8_t*>(W);
    a.S = scale;
    a.bias = bias;
    a.Y = Y;
    a.M = int(p->M);
    a.N = int(p->N);
    a.K = int(p->K);
    a.G = int(p->qGroup);
    a.groups = int(p->K / p->qGroup);
    a.has_bias = p->hasBias != 0;
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    const unsigned grid = unsigned(a.tiles_m) * unsigned(a.tiles_n);
    auto kern = bits == 4 ? gemm_bf16_kernel<4> : gemm_bf16_kernel<8>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, LDS_WS);
    if (e != hipSuccess)
        return fail(g, DGM_ERR_HIP, "bf16 gemm: cannot reserve %d bytes of LDS: %s", LDS_WS, hipGetErrorString(e));
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NTW), LDS_WS, st, a);
    return DGM_OK;
}

}  // namespace dgm
