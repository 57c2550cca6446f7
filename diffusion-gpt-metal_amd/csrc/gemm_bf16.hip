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
//    column, so converting it inside the GEMM would repeat the work N/128
//    times).
//  * A workgroup computes a 512 x 128 tile of Y with twelve waves in two
//    roles. Eight MFMA waves each own a 128 x 64 block = 8 x 4
//    v_mfma_f32_16x16x32_bf16 tiles (128 fp32 accumulators) and only read LDS
//    and issue MFMAs. Four producer waves load the X tile (global -> LDS with
//    global_load_lds_dwordx4, no VGPR staging) and the weight codes, and
//    dequantize the codes into the bf16 weight tile in LDS, half a weight row
//    (32 k) per lane. Each SIMD holds two MFMA waves and one producer, so the
//    dequantization's VALU work runs beside the MFMAs. K advances 64 per step.
//    The tall tile halves the weights dequantized per step against the
//    256 x 256 tile with the same MFMA work (the producers' dequantization
//    sets the step time): int8 gains ~5%, int4 is unchanged.
//  * A wave instruction of the X load fills 1 KB of LDS in lane order, so rows
//    are unpadded (128 B) and the 16-byte chunks of row r sit at slot
//    c ^ (r & 7): each lane fetches the global chunk that belongs in its slot.
//    Fragment reads (16 rows, one chunk) then hit 8 distinct slots per 8-lane
//    group, free of bank conflicts: a probe of ds_read_b128 on gfx950 takes 23
//    cycles per wave instruction with this map, as with contiguous lanes, and
//    32 when rows 8-15 are further XOR-ed by 1. The weight tile uses the same
//    swizzle (its one-row-per-lane stores cost the same either way).
//  * Stages: two for X, two for the weights (160 KB of LDS). During step k
//    the MFMA waves read stage k; the producers first issue X of step k+1,
//    then store the weights of step k+1 (codes loaded two steps earlier),
//    then issue the codes of step k+3, and enter the step's barrier once X of
//    step k+1 has landed. All producer loads are inline asm with counted
//    waits. One barrier per step.
//  * Dequant: int4 bytes are flipped to offset binary and masked into the
//    high nibble, so each byte is 16*(code+8) as an unsigned value and
//    converts with one v_cvt_f32_ubyte; fma(f, s/16, -8s) then yields
//    code*s with a single rounding (the exact product minus an exact offset),
//    i.e. the reference's fp32 dequant bit for bit, followed by one
//    v_cvt_pk_bf16_f32 per pair. int8 codes use (code+128) and fma(f, s, -128s).
//  * Tile order is XCD-aware: workgroups are dealt round-robin to the 8 XCDs,
//    so the logical tile index is remapped to give each XCD a contiguous range,
//    walked in groups of tile rows (1 for int4, 4 for int8); the ~32 tiles an
//    XCD runs at once then share X and weight rows in its L2.
#include "common.hpp"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 512, BN = 128, BK = 64;
constexpr int RS = BK * 2;        // LDS row stride in bytes (chunks swizzled, no pad)
// Tile rows per group of the XCD-local order. int4: one (the ~32 tiles an XCD
// runs at once share one 64 KB X slice per step and read 4 KB of codes each;
// +1.7% against groups of 4); int8 codes are twice the bytes and groups of 4
// rows, which share each weight slice four ways, are ~1% faster.
template <int BITS>
constexpr int GROUP_M = BITS == 4 ? 1 : 4;

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
// Twelve waves: waves 0-7 only read LDS and issue MFMAs (a 128 x 64 block
// each); waves 8-11 are producers: they issue the X tile's direct-to-LDS loads
// and load, dequantize and store the weight tile of the next step while the
// MFMA waves work on the current one. Waves are dealt to the SIMDs round
// robin, so each SIMD holds two MFMA waves and one producer and the
// dequantization's VALU work overlaps MFMA issue instead of following it.
// The tile is 512 rows of X by 128 weight rows: per 64-k step the producers
// dequantize 128 x 64 weights (each W element is dequantized once per 512
// rows of Y) and move 512 x 64 of X. LDS: two X stages (the X tile of step
// k+1 is loaded at the start of step k) and two weight stages, 2 x 64 + 2 x 16
// KB.
constexpr int NTW = 768;
constexpr int TILE_X = BM * RS;
constexpr int TILE_W = BN * RS;
constexpr int LDS_WS = 2 * TILE_X + 2 * TILE_W;

template <int BITS>
__global__ __launch_bounds__(NTW) void gemm_bf16_kernel(Bf16Args a) {
    constexpr int CB = BITS == 4 ? 1 : 2;   // 16-byte code loads per producer lane per 64-k step (32 k)
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int l16 = lane & 15, q = lane >> 4;
    const int M = a.M, N = a.N, K = a.K;

    const int total = a.tiles_m * a.tiles_n;
    int L = blockIdx.x;
    if (total % 8 == 0) L = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    constexpr int GM = GROUP_M<BITS>;
    const int group = L / (GM * a.tiles_n);
    const int first_m = group * GM;
    const int gm = min(GM, a.tiles_m - first_m);
    const int within = L - group * GM * a.tiles_n;
    const int m0 = (first_m + within % gm) * BM;
    const int n0 = (within / gm) * BN;
    const int nk = K / BK;

    if (wave >= 8) {
        // ---- producer p: X rows 128p .. 128p+127 (8 per instruction); W row
        // 32p + lane % 32, k half lane / 32 (32 k, one group).
        // Every global load is inline asm and waited for by count: step ks
        // issues X of step ks + 1 (16 direct-to-LDS loads) first and, after
        // the weight stores, the codes and scale of step ks + 3 (NW loads)
        // into the code buffer it has just dequantized, so codes have two
        // steps to arrive. (With compiler-visible direct-to-LDS loads the
        // compiler waits for all of them before any LDS store.)
        constexpr int NW = CB + 1;
        const int p = __builtin_amdgcn_readfirstlane(wave - 8);
        const int arl = lane >> 3, aslot = lane & 7;
        uint32_t aoff[16];   // byte offsets into Xb
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int r = p * 128 + j * 8 + arl;
            aoff[j] = (uint32_t(min(m0 + r, M - 1)) * uint32_t(K) + ((aslot ^ (r & 7)) * 8)) * 2u;
        }
        const int brow = p * 32 + (lane & 31), hh = lane >> 5;
        const int bn = min(n0 + brow, N - 1);
        const uint32_t boff = uint32_t(bn) * uint32_t(BITS == 4 ? K / 2 : K) + uint32_t(hh) * (BITS == 4 ? 16u : 32u);
        const uint32_t soff = uint32_t(bn) * uint32_t(a.groups) * 4u;
        const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
        auto xdma = [&](int ks, int st) {
            const uint32_t lds = lds0 + uint32_t(st * TILE_X + p * 128 * RS);
#pragma unroll
            for (int j = 0; j < 16; ++j)
                asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds + j * 8 * RS),
                             "v"(aoff[j] + uint32_t(ks * BK * 2)), "s"(a.Xb)
                             : "memory", "m0");
        };
#pragma clang diagnostic pop
        auto wload = [&](u32x4 (&c)[CB], float& s, int ks) {
            const uint32_t k0 = uint32_t(ks * BK);
#pragma unroll
            for (int j = 0; j < CB; ++j)
                asm volatile("global_load_dwordx4 %0, %1, %2"
                             : "=v"(c[j])
                             : "v"(boff + (BITS == 4 ? k0 / 2 : k0) + 16u * j), "s"(a.W));
            asm volatile("global_load_dword %0, %1, %2"
                         : "=v"(s)
                         : "v"(soff + ((k0 + 32u * hh) / a.G) * 4u), "s"(a.S));
        };
        // The loaded registers become visible to the compiler only here,
        // after the wait that covers them.
        auto pin = [](u32x4 (&c)[CB], float& s) {
#pragma unroll
            for (int j = 0; j < CB; ++j) asm volatile("" : "+v"(c[j]));
            asm volatile("" : "+v"(s));
        };
        // The lane's 32 k: chunks 4 hh .. 4 hh + 3 of its weight row.
        auto dequant_store = [&](const u32x4 (&c)[CB], float s, int st) {
            uint8_t* Bs = smem + 2 * TILE_X + st * TILE_W;
            if constexpr (BITS == 4) {
                const float s16 = s * 0.0625f, off = -8.0f * s;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t x = c[0][d] ^ 0x88888888u;
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
                    *reinterpret_cast<u32x4*>(Bs + swz(brow, hh * 4 + d)) = u32x4{o[0], o[1], o[2], o[3]};
                }
            } else {
                const float off = -128.0f * s;
                const uint32_t w8[8] = {c[0][0], c[0][1], c[0][2], c[0][3], c[1][0], c[1][1], c[1][2], c[1][3]};
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
                    *reinterpret_cast<u32x4*>(Bs + swz(brow, hh * 4 + d)) = u32x4{o[0], o[1], o[2], o[3]};
                }
            }
        };
        u32x4 c0[CB], c1[CB];
        float s0, s1;
        auto clampk = [&](int ks) { return ks < nk ? ks : nk - 1; };
        // X stage i at i * TILE_X, weight stage i at 2 * TILE_X + i * TILE_W.
        wload(c0, s0, 0);
        wload(c1, s1, clampk(1));
        xdma(0, 0);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(16 + NW) : "memory");   // codes of step 0
        pin(c0, s0);
        dequant_store(c0, s0, 0);
        wload(c0, s0, clampk(2));
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(NW) : "memory");   // X of step 0
        // Step ks: codes of step ks + 1 are in (cc, cs), issued two steps ago.
        auto step = [&](int ks, u32x4 (&cc)[CB], float& cs) {
            xdma(clampk(ks + 1), (ks + 1) & 1);   // stage of step ks - 1, free since the last barrier
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(32 + NW) : "memory");
            pin(cc, cs);
            dequant_store(cc, cs, (ks + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            wload(cc, cs, clampk(ks + 3));
            __builtin_amdgcn_sched_barrier(0);
            // Barrier once X of step ks + 1 has landed (the codes stay in
            // flight) and every weight store of this wave is done.
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(NW) : "memory");
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

    // ---- MFMA waves: rows wm*128 .. +127, columns wn*64 .. +63.
    const int wm = wave >> 1, wn = wave & 1;
    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int cw0 = ((0 * 4 + q) ^ (l16 & 7)) << 4, cw1 = ((1 * 4 + q) ^ (l16 & 7)) << 4;
    auto compute = [&](int xs, int ws) {
        const uint8_t* As = smem + xs * TILE_X + (wm * 128 + l16) * RS;
        const uint8_t* Bs = smem + 2 * TILE_X + ws * TILE_W + (wn * 64 + l16) * RS;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int cw = kk ? cw1 : cw0;
            bf16x8 bf[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) bf[j] = *reinterpret_cast<const bf16x8*>(Bs + j * 16 * RS + cw);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const bf16x8 afi = *reinterpret_cast<const bf16x8*>(As + i * 16 * RS + cw);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afi, bf[j], acc[i][j], 0, 0, 0);
            }
        }
    };
    __syncthreads();
    for (int ks = 0; ks < nk; ++ks) {
        compute(ks & 1, ks & 1);
        __syncthreads();
    }

    // Epilogue. The bias is added to the accumulators before any store, so
    // no store depends on a load: a bias load that only some paths issue
    // makes the compiler wait for every outstanding memory operation
    // (vmcnt(0)) before each dependent store, i.e. for all earlier stores,
    // which serializes the 128 stores of a wave on the write latency.
    if (a.has_bias) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float bv = a.bias[min(n0 + wn * 64 + j * 16 + l16, N - 1)];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i][j] += bv;
        }
    }
    float* yb = a.Y + size_t(m0 + wm * 128 + 4 * q) * N + (n0 + wn * 64 + l16);
    if (m0 + BM <= M && n0 + BN <= N) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    yb[size_t(i * 16 + r) * N + j * 16] = acc[i][j][r];
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int row = m0 + wm * 128 + i * 16 + 4 * q + r, col = n0 + wn * 64 + j * 16 + l16;
                    if (row < M && col < N) yb[size_t(i * 16 + r) * N + j * 16] = acc[i][j][r];
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
    // The kernel addresses X (bf16), the codes and the scales with 32-bit byte offsets.
    if (int64_t(p->M) * p->K * 2 >= (int64_t(1) << 32)) return false;
    if (int64_t(p->N) * p->K * bits / 8 >= (int64_t(1) << 32)) return false;
    if (int64_t(p->N) * (p->K / p->qGroup) * 4 >= (int64_t(1) << 32)) return false;
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
