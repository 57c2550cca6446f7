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
//  * A workgroup of 8 waves computes a 256 x 256 tile of Y; each wave owns a
//    64 x 128 block = 4 x 8 v_mfma_f32_16x16x32_bf16 tiles (128 fp32
//    accumulators), so two waves share each SIMD and one wave's MFMAs overlap
//    the other's dequantization, LDS and memory instructions. K advances 64
//    per step.
//  * The X tile goes global -> LDS with global_load_lds_dwordx4 (no VGPR
//    staging). A wave instruction
//    fills 1 KB of LDS in lane order, so rows are unpadded (128 B) and the
//    16-byte chunks of row r sit at slot c ^ (r & 7): each lane fetches the
//    global chunk that belongs in its slot. Fragment reads (16 rows, one
//    chunk) then hit 8 distinct slots per 8-lane group, free of bank
//    conflicts. The weight tile uses the same swizzle.
//  * Each weight row is dequantized once per workgroup, by two threads (32 k
//    each), into the bf16 weight tile in LDS.
//  * Two stages: the loads of step k+1 are issued before the MFMAs of step k;
//    the weight codes of step k+1 are dequantized and stored to the other
//    stage after the MFMAs; one barrier per step. The loop is unrolled by two
//    so every stage index is a compile-time constant.
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

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int RS = BK * 2;        // LDS row stride in bytes (chunks swizzled, no pad)
constexpr int TILE = BM * RS;     // one operand tile (BM == BN)
constexpr int STAGE = 2 * TILE;
constexpr size_t LDS_BYTES = 2 * STAGE;
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

// X fp32 -> bf16 (nearest even), 8 elements per thread.
__global__ __launch_bounds__(256) void x_to_bf16_kernel(const float* __restrict__ X, uint16_t* __restrict__ Xb,
                                                        int64_t n8) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n8) return;
    const float4 a = reinterpret_cast<const float4*>(X)[2 * i];
    const float4 b = reinterpret_cast<const float4*>(X)[2 * i + 1];
    reinterpret_cast<uint4*>(Xb)[i] =
        make_uint4(pack_bf16(a.x, a.y), pack_bf16(a.z, a.w), pack_bf16(b.x, b.y), pack_bf16(b.z, b.w));
}

typedef __attribute__((address_space(1))) const void global_cvoid;
typedef __attribute__((address_space(3))) void lds_void;

// Byte offset of 16-byte chunk c of row r in a swizzled operand tile.
__device__ __forceinline__ int swz(int r, int c) { return r * RS + ((c ^ (r & 7)) << 4); }

// ---- eight-wave variant --------------------------------------------------------
// Same tile, stages, swizzle and dequantization as gemm_bf16_kernel, with 8
// waves of 64 x 128 (128 accumulators each), so two waves share each SIMD and
// one wave's MFMAs overlap the other's dequantization, LDS and memory work.
// X rows: wave w loads 32 rows; weight rows: two threads per row, 32 k each.
constexpr int NT8 = 512;

template <int BITS>
__global__ __launch_bounds__(NT8) void gemm_bf16_w8_kernel(Bf16Args a) {
    constexpr int WB = BITS == 4 ? 1 : 2;   // 16-byte code loads per thread per step (32 k)
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int l16 = lane & 15, q = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;   // rows wm*64, cols wn*128
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

    // -- X tile: wave w loads rows w*32 .. w*32+31, 8 rows per instruction.
    const int arl = lane >> 3, aslot = lane & 7;
    uint32_t aoff[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int r = wave * 32 + p * 8 + arl;
        aoff[p] = uint32_t(min(m0 + r, M - 1)) * uint32_t(K) + ((aslot ^ (r & 7)) * 8);
    }
    // -- weight tile: thread t -> row t/2, k half (t & 1) of the 64-k step.
    const int brow = t >> 1, bh = t & 1;
    const int bn = min(n0 + brow, N - 1);
    const uint8_t* bptr = a.W + size_t(bn) * (BITS == 4 ? K / 2 : K);
    const float* sptr = a.S + size_t(bn) * a.groups;

    uint4 breg[WB];
    float sreg;
    auto gload = [&](int ks, int st) {
        const int k0 = ks * BK;
        uint8_t* As = smem + st * STAGE + wave * 32 * RS;
#pragma unroll
        for (int p = 0; p < 4; ++p)
            __builtin_amdgcn_global_load_lds((global_cvoid*)(a.Xb + aoff[p] + k0),
                                             (lds_void*)(As + p * 8 * RS), 16, 0, 0);
        const int kh = k0 + 32 * bh;
#pragma unroll
        for (int j = 0; j < WB; ++j)
            breg[j] = *reinterpret_cast<const uint4*>(bptr + (BITS == 4 ? kh / 2 : kh) + 16 * j);
        sreg = sptr[kh / a.G];
    };

    auto dequant_store = [&](int st) {
        uint8_t* Bs = smem + st * STAGE + TILE;
        const float s = sreg;
        if constexpr (BITS == 4) {
            const float s16 = s * 0.0625f, off = -8.0f * s;
            const uint32_t w4[4] = {breg[0].x, breg[0].y, breg[0].z, breg[0].w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {   // 8 nibbles = k 8d..8d+7 of the half
                const uint32_t x = w4[d] ^ 0x88888888u;
                uint32_t lo = (x << 4) & 0xF0F0F0F0u;
                uint32_t hi = x & 0xF0F0F0F0u;
                // Opaque to the optimizer (no instruction): keeps each byte
                // extraction below a single v_cvt_f32_ubyte{0..3} instead of a
                // shift and mask folded into every byte.
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
                *reinterpret_cast<uint4*>(Bs + swz(brow, bh * 4 + d)) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        } else {
            const float off = -128.0f * s;
            const uint32_t w8[8] = {breg[0].x, breg[0].y, breg[0].z, breg[0].w,
                                    breg[1].x, breg[1].y, breg[1].z, breg[1].w};
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
                *reinterpret_cast<uint4*>(Bs + swz(brow, bh * 4 + d)) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
    };

    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int cw0 = ((0 * 4 + q) ^ (l16 & 7)) << 4, cw1 = ((1 * 4 + q) ^ (l16 & 7)) << 4;
    auto compute = [&](int st) {
        const uint8_t* As = smem + st * STAGE + (wm * 64 + l16) * RS;
        const uint8_t* Bs = smem + st * STAGE + TILE + (wn * 128 + l16) * RS;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int cw = kk ? cw1 : cw0;
            bf16x8 bf[8], af[2];
#pragma unroll
            for (int j = 0; j < 8; ++j) bf[j] = *reinterpret_cast<const bf16x8*>(Bs + j * 16 * RS + cw);
            af[0] = *reinterpret_cast<const bf16x8*>(As + cw);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (i + 1 < 4) af[(i + 1) & 1] = *reinterpret_cast<const bf16x8*>(As + (i + 1) * 16 * RS + cw);
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i & 1], bf[j], acc[i][j], 0, 0, 0);
            }
        }
    };

    const int nk = K / BK;   // even (host)
    gload(0, 0);
    dequant_store(0);
    __syncthreads();
    for (int ks = 0; ks < nk; ks += 2) {
        gload(ks + 1, 1);
        __builtin_amdgcn_sched_barrier(0);
        compute(0);
        __builtin_amdgcn_sched_barrier(0);
        dequant_store(1);
        __syncthreads();
        gload(ks + 2 < nk ? ks + 2 : ks + 1, 0);
        __builtin_amdgcn_sched_barrier(0);
        compute(1);
        __builtin_amdgcn_sched_barrier(0);
        dequant_store(0);
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
                if (row < M && col < N) a.Y[size_t(row) * N + col] = acc[i][j][r] + bv;
            }
    }
}

}  // namespace

namespace dgm {

// The bf16 path takes quantized forwards with M > 64 in the reduced-precision
// mode: K a multiple of 128, every 32-k half inside one group, aligned operands.
bool bf16_ok(int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p) {
    if (bits != 4 && bits != 8) return false;
    if (p->M <= 64 || p->K == 0 || (p->K % (2 * BK)) != 0) return false;   // even step count
    if (p->qGroup == 0 || (p->qGroup % 32) != 0) return false;   // a thread's 32 k share a group
    if (int64_t(p->M) * p->K >= (int64_t(1) << 32)) return false;   // 32-bit element offsets
    (void)S;
    return aligned(W, 16) && aligned(X, 16);
}

int bf16_fwd(dgm_gpu* g, int bits, const void* W, const float* scale, const float* X, const float* bias,
             float* Y, const dgm_GemmP* p) {
    const int64_t mk = int64_t(p->M) * p->K;
    uint16_t* xb = static_cast<uint16_t*>(workspace(g, size_t(mk) * 2));
    if (!xb) return DGM_ERR_HIP;
    hipStream_t st = g->stream;
    const int64_t n8 = mk / 8;
    hipLaunchKernelGGL(x_to_bf16_kernel, dim3(unsigned((n8 + 255) / 256)), dim3(256), 0, st, X, xb, n8);

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
    // Eight waves (two per SIMD): one wave's MFMAs overlap the other's
    // dequantization and LDS traffic (~10% over the four-wave kernel at c5,
    // identical results).
    auto kern = bits == 4 ? gemm_bf16_w8_kernel<4> : gemm_bf16_w8_kernel<8>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(LDS_BYTES));
    if (e != hipSuccess)
        return fail(g, DGM_ERR_HIP, "bf16 gemm: cannot reserve %zu bytes of LDS: %s", LDS_BYTES,
                    hipGetErrorString(e));
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NT8), LDS_BYTES, st, a);
    return DGM_OK;
}

}  // namespace dgm
