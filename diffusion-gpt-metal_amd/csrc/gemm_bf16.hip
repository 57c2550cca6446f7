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
//    128 x 64 block = 8 x 4 v_mfma_f32_16x16x32_bf16 tiles (128 fp32
//    accumulators, so two waves fit per SIMD with their staging registers).
//    K advances 64 per step.
//  * Both operand tiles live in LDS as bf16 rows of 64 k with a 16-byte pad
//    (row stride 144 B), which spreads the 16 rows read by one ds_read_b128
//    over distinct banks. Two stages: the global loads of step k+1 are issued
//    before the MFMAs of step k; the weight tile of step k+1 is dequantized
//    in registers and stored to the other stage afterwards; one barrier per
//    step.
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
constexpr int NT = 512;
constexpr int RS = BK * 2 + 16;   // LDS row stride in bytes
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

template <int BITS>
__global__ __launch_bounds__(NT) void gemm_bf16_kernel(Bf16Args a) {
    constexpr int WB = BITS == 4 ? 1 : 2;   // 16-byte code loads per thread per step
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int l16 = lane & 15, q = lane >> 4;
    const int wm = wave >> 2, wn = wave & 3;   // wave block: rows wm*128, cols wn*64
    const int M = a.M, N = a.N, K = a.K;

    // -- tile of this workgroup (XCD-aware order).
    const int total = a.tiles_m * a.tiles_n;
    int L = blockIdx.x;
    if (total % 8 == 0) L = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    const int group = L / (GROUP_M * a.tiles_n);
    const int first_m = group * GROUP_M;
    const int gm = min(GROUP_M, a.tiles_m - first_m);
    const int within = L - group * GROUP_M * a.tiles_n;
    const int m0 = (first_m + within % gm) * BM;
    const int n0 = (within / gm) * BN;

    // -- per-thread global addresses. A: 4 passes of 64 rows x 8 16-byte
    // chunks (128 contiguous bytes per row per step). B: two threads per
    // weight row, one 32-k half (one scale) each. Rows past the matrix are
    // clamped (never stored).
    const int arow = t >> 3, achunk = t & 7;
    uint32_t aoff[4];   // element offsets (the host bounds M*K below 2^32)
#pragma unroll
    for (int p = 0; p < 4; ++p) aoff[p] = uint32_t(min(m0 + p * 64 + arow, M - 1)) * uint32_t(K) + achunk * 8;
    const int brow_i = t >> 1, bh = t & 1;
    const int bn = min(n0 + brow_i, N - 1);
    const uint8_t* bptr = a.W + size_t(bn) * (BITS == 4 ? K / 2 : K) + bh * (BITS == 4 ? 16 : 32);
    const float* sptr = a.S + size_t(bn) * a.groups;

    uint4 areg[4];
    uint4 breg[WB];
    float sreg;
    auto gload = [&](int ks) {
        const int k0 = ks * BK;
#pragma unroll
        for (int j = 0; j < WB; ++j)
            breg[j] = *reinterpret_cast<const uint4*>(bptr + (BITS == 4 ? k0 / 2 : k0) + 16 * j);
        sreg = sptr[(k0 + 32 * bh) / a.G];
#pragma unroll
        for (int p = 0; p < 4; ++p) areg[p] = *reinterpret_cast<const uint4*>(a.Xb + aoff[p] + k0);
    };

    auto lstore = [&](int st) {
        uint8_t* As = smem + st * STAGE;
        uint8_t* Bs = As + TILE;
#pragma unroll
        for (int p = 0; p < 4; ++p)
            *reinterpret_cast<uint4*>(As + (p * 64 + arow) * RS + achunk * 16) = areg[p];
        uint8_t* bdst = Bs + brow_i * RS + bh * 64;   // this thread's 32 k
        const float s = sreg;
        if constexpr (BITS == 4) {
            const float s16 = s * 0.0625f, off = -8.0f * s;
            const uint32_t w4[4] = {breg[0].x, breg[0].y, breg[0].z, breg[0].w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {   // 8 nibbles = k 8d..8d+7 of the half
                const uint32_t x = w4[d] ^ 0x88888888u;            // offset binary
                const uint32_t lo = (x << 4) & 0xF0F0F0F0u;        // even k: 16*(code+8)
                const uint32_t hi = x & 0xF0F0F0F0u;               // odd k
                uint32_t o[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float fe = float((lo >> (8 * i)) & 0xFFu);
                    const float fo = float((hi >> (8 * i)) & 0xFFu);
                    o[i] = pack_bf16(__builtin_fmaf(fe, s16, off), __builtin_fmaf(fo, s16, off));
                }
                *reinterpret_cast<uint4*>(bdst + 16 * d) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        } else {
            const float off = -128.0f * s;
            const uint32_t w8[8] = {breg[0].x, breg[0].y, breg[0].z, breg[0].w,
                                    breg[1].x, breg[1].y, breg[1].z, breg[1].w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {   // 8 codes = k 8d..8d+7 of the half
                uint32_t o[4];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint32_t x = w8[2 * d + e] ^ 0x80808080u;   // code + 128
                    const float f0 = float(x & 0xFFu), f1 = float((x >> 8) & 0xFFu);
                    const float f2 = float((x >> 16) & 0xFFu), f3 = float(x >> 24);
                    o[2 * e] = pack_bf16(__builtin_fmaf(f0, s, off), __builtin_fmaf(f1, s, off));
                    o[2 * e + 1] = pack_bf16(__builtin_fmaf(f2, s, off), __builtin_fmaf(f3, s, off));
                }
                *reinterpret_cast<uint4*>(bdst + 16 * d) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
    };

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int st) {
        const uint8_t* As = smem + st * STAGE + (wm * 128 + l16) * RS + q * 16;
        const uint8_t* Bs = smem + st * STAGE + TILE + (wn * 64 + l16) * RS + q * 16;
        // B fragments stay in registers for the sub-step; A fragments stream
        // through a two-deep ping-pong (the next one loads under the 4 MFMAs
        // of the current one).
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            bf16x8 bf[4], af[2];
#pragma unroll
            for (int j = 0; j < 4; ++j) bf[j] = *reinterpret_cast<const bf16x8*>(Bs + j * 16 * RS + kk * 64);
            af[0] = *reinterpret_cast<const bf16x8*>(As + kk * 64);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (i + 1 < 8) af[(i + 1) & 1] = *reinterpret_cast<const bf16x8*>(As + (i + 1) * 16 * RS + kk * 64);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i & 1], bf[j], acc[i][j], 0, 0, 0);
            }
        }
    };

    const int nk = K / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int ks = 0; ks < nk; ++ks) {
        // The next step's loads are unconditional (the last step re-reads its
        // own tile): a conditional load would make its consumers wait for all
        // loads in flight.
        gload(ks + 1 < nk ? ks + 1 : ks);
        // Phases stay apart: mixing the dequant of step k+1 into the MFMAs of
        // step k raises register pressure until it spills; the two waves on
        // each SIMD overlap one's MFMAs with the other's dequant instead.
        __builtin_amdgcn_sched_barrier(0);
        compute(ks & 1);
        __builtin_amdgcn_sched_barrier(0);
        lstore((ks + 1) & 1);
        __syncthreads();
    }

    // D layout of 16x16 f32: lane holds rows 4*(lane/16) + r, column lane%16.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = n0 + wn * 64 + j * 16 + l16;
        const float bv = (a.has_bias && col < N) ? a.bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm * 128 + i * 16 + 4 * q + r;
                if (row < M && col < N) a.Y[size_t(row) * N + col] = acc[i][j][r] + bv;
            }
    }
}

}  // namespace

namespace dgm {

// The bf16 path takes quantized forwards with M > 64 in the reduced-precision
// mode: K a multiple of 64, every 32-k half inside one group, aligned operands.
bool bf16_ok(int bits, const void* W, const float* X, const float* S, const dgm_GemmP* p) {
    if (bits != 4 && bits != 8) return false;
    if (p->M <= 64 || p->K == 0 || (p->K % BK) != 0) return false;
    if (p->qGroup == 0 || (p->qGroup % 32) != 0) return false;
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
    auto kern = bits == 4 ? gemm_bf16_kernel<4> : gemm_bf16_kernel<8>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(LDS_BYTES));
    if (e != hipSuccess)
        return fail(g, DGM_ERR_HIP, "bf16 gemm: cannot reserve %zu bytes of LDS: %s", LDS_BYTES,
                    hipGetErrorString(e));
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NT), LDS_BYTES, st, a);
    return DGM_OK;
}

}  // namespace dgm
