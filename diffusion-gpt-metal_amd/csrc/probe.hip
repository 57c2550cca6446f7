// Measurement probes (no counterpart in the reference).
//
// Achievable HBM read rate of one launch, for the bench's roofline: a
// read-only stream of `bytes` from `src`, split into contiguous shares over
// the workgroups, with no arithmetic beyond folding the data into one word
// per workgroup (stored, so that no load is dead).
//  * mode 0: 16-byte non-temporal loads into registers, eight per thread in
//    flight (the pattern of a kernel that computes on registers);
//  * mode 1: 16-byte direct-to-LDS loads, each wave streaming its share
//    through a ring of its own (the pattern of the decode kernels' weights).
#include "common.hpp"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int PR_THREADS = 256;
constexpr int PR_UNROLL = 8;
constexpr int PR_RING = 8;   // 1 KB slots per wave (mode 1)

__global__ __launch_bounds__(PR_THREADS) void probe_reg_kernel(const u32x4* __restrict__ src, uint64_t n16,
                                                               uint32_t* __restrict__ sink) {
    const uint64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const uint64_t b = uint64_t(blockIdx.x) * per;
    const uint64_t e = b + per < n16 ? b + per : n16;
    uint32_t acc = 0;
    for (uint64_t i = b + threadIdx.x; i < e; i += PR_THREADS * PR_UNROLL) {
        u32x4 v[PR_UNROLL];
#pragma unroll
        for (int u = 0; u < PR_UNROLL; ++u) {
            const uint64_t j = i + uint64_t(u) * PR_THREADS;
            v[u] = __builtin_nontemporal_load(src + (j < e ? j : i));
        }
#pragma unroll
        for (int u = 0; u < PR_UNROLL; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    // One word per workgroup: the fold of thread 0's share.
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

__global__ __launch_bounds__(PR_THREADS) void probe_lds_kernel(const uint8_t* __restrict__ src, uint64_t nbytes,
                                                               uint32_t* __restrict__ sink) {
    __shared__ __align__(16) uint8_t ring[PR_THREADS / 64][PR_RING * 1024];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t per = ((nbytes / 1024 + gridDim.x - 1) / gridDim.x) * 1024;
    const uint64_t b = uint64_t(blockIdx.x) * per;
    const uint64_t e = b + per < nbytes ? b + per : nbytes;
    int slot = 0;
    for (uint64_t off = b + uint64_t(wave) * 1024; off < e; off += (PR_THREADS / 64) * 1024) {
        // Every load writes slot `slot` of this wave's ring; the hardware
        // keeps at most 63 of them in flight per wave.
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + off + uint64_t(lane) * 16),
                                         (__attribute__((address_space(3))) void*)(&ring[wave][slot * 1024]), 16, 0, 0);
        slot = slot + 1 == PR_RING ? 0 : slot + 1;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t acc = 0;
        for (int w = 0; w < PR_THREADS / 64; ++w) acc ^= *reinterpret_cast<const uint32_t*>(&ring[w][0]);
        sink[blockIdx.x] = acc;
    }
}

// ---- wave-reduction VALU GEMV (int4), the design the MFMA decode kernels are
// measured against. A wave owns GV_ROWS W rows; lane l takes the 16-byte code
// chunks l, l + 64, ... (32 k each) of every row, dequantizes them once
// (code * scale in fp32, the reference's dequant) and multiplies them into
// M running sums per row with fp32 FMAs; the 64 lanes' sums are then added by
// a butterfly. X is read from LDS when it fits (M x K x 4 <= 64 KB), else
// from global memory (L1/L2).
constexpr int GV_ROWS = 4;
constexpr int GV_XLDS_MAX = 64 * 1024;

template <int M, bool XLDS>
__global__ __launch_bounds__(256) void gemv_valu_kernel(const uint8_t* __restrict__ W, const float* __restrict__ S,
                                                        const float* __restrict__ X, float* __restrict__ Y, int N,
                                                        int K, int G) {
    extern __shared__ __align__(16) uint8_t xsm[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * 4 + wave) * GV_ROWS;
    const int rowb = K / 2, nch = K / 32, groups = K / G;
    const u32x4* xv = reinterpret_cast<const u32x4*>(X);
    if constexpr (XLDS) {
        for (int i = threadIdx.x; i < M * K / 4; i += 256) reinterpret_cast<u32x4*>(xsm)[i] = xv[i];
        __syncthreads();
        xv = reinterpret_cast<const u32x4*>(xsm);
    }
    float acc[GV_ROWS][M];
#pragma unroll
    for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
    for (int j = lane; j < nch; j += 64) {
        const int k0 = 32 * j;
        u32x4 c[GV_ROWS];
        float s[GV_ROWS];
#pragma unroll
        for (int r = 0; r < GV_ROWS; ++r) {
            const int n = min(n0 + r, N - 1);
            c[r] = *reinterpret_cast<const u32x4*>(W + size_t(n) * rowb + 16 * j);
            s[r] = S[size_t(n) * groups + k0 / G];
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            float wd[GV_ROWS][8];   // k0 + 8d .. +7, dequantized
#pragma unroll
            for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    wd[r][e] = float(int(c[r][d] << (28 - 4 * e)) >> 28) * s[r];   // signed nibble e
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const f32x4 x0 = __builtin_bit_cast(f32x4, xv[(m * K + k0 + 8 * d) / 4]);
                const f32x4 x1 = __builtin_bit_cast(f32x4, xv[(m * K + k0 + 8 * d) / 4 + 1]);
                const float xf[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[r][m] = __builtin_fmaf(wd[r][e], xf[e], acc[r][m]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float v = acc[r][m];
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0 && n0 + r < N) Y[size_t(m) * N + n0 + r] = v;
        }
}

template <int M>
void launch_gemv(dgm_gpu* g, const uint8_t* W, const float* S, const float* X, float* Y, int N, int K, int G) {
    const unsigned grid = unsigned((N + 4 * GV_ROWS - 1) / (4 * GV_ROWS));
    if (int64_t(M) * K * 4 <= GV_XLDS_MAX)
        hipLaunchKernelGGL((gemv_valu_kernel<M, true>), dim3(grid), dim3(256), size_t(M) * K * 4, g->stream, W, S, X, Y,
                           N, K, G);
    else
        hipLaunchKernelGGL((gemv_valu_kernel<M, false>), dim3(grid), dim3(256), 0, g->stream, W, S, X, Y, N, K, G);
}

}  // namespace

extern "C" int dgm_probe_gemv_valu(dgm_gpu* g, const uint8_t* Wq, const float* scale, const float* X, float* Y,
                                   int64_t M, int64_t N, int64_t K, int64_t qGroup) {
    int rc = dgm::enter(g, "probe_gemv_valu");
    if (rc) return rc;
    if (!Wq || !scale || !X || !Y || N <= 0 || K <= 0 || K % 32 != 0 || qGroup <= 0 || qGroup % 32 != 0 ||
        K % qGroup != 0 || N * (K / 2) >= (int64_t(1) << 31) || !dgm::aligned(Wq, 16) || !dgm::aligned(X, 16))
        return dgm::fail(g, DGM_ERR_ARG, "probe_gemv_valu: bad arguments");
    const int n = int(N), k = int(K), gq = int(qGroup);
    switch (M) {
        case 1: launch_gemv<1>(g, Wq, scale, X, Y, n, k, gq); break;
        case 16: launch_gemv<16>(g, Wq, scale, X, Y, n, k, gq); break;
        default: return dgm::fail(g, DGM_ERR_UNSUPPORTED, "probe_gemv_valu: M must be 1 or 16");
    }
    return dgm::check_launch(g, "probe_gemv_valu");
}

extern "C" int dgm_probe_read(dgm_gpu* g, const void* src, int64_t bytes, int64_t mode, int64_t workgroups,
                              uint32_t* sink) {
    int rc = dgm::enter(g, "probe_read");
    if (rc) return rc;
    if (!src || !sink || bytes <= 0 || bytes % 1024 != 0 || (mode != 0 && mode != 1) || workgroups < 0 ||
        workgroups > (int64_t(1) << 20) || !dgm::aligned(src, 16))
        return dgm::fail(g, DGM_ERR_ARG, "probe_read: bad arguments");
    const unsigned grid = unsigned(workgroups ? workgroups : g->num_cus);
    if (mode == 0)
        hipLaunchKernelGGL(probe_reg_kernel, dim3(grid), dim3(PR_THREADS), 0, g->stream,
                           static_cast<const u32x4*>(src), uint64_t(bytes) / 16, sink);
    else
        hipLaunchKernelGGL(probe_lds_kernel, dim3(grid), dim3(PR_THREADS), 0, g->stream,
                           static_cast<const uint8_t*>(src), uint64_t(bytes), sink);
    return dgm::check_launch(g, "probe_read");
}
