// Achievable HBM read rate of one launch, for the bench's roofline: a
// read-only stream of `bytes` from `src`, split into contiguous shares over
// the workgroups, with no arithmetic beyond folding the data into one word
// per workgroup (stored, so that no load is dead).
//  * mode 0: 16-byte non-temporal loads into registers, eight per thread in
//    flight (the pattern of a kernel that computes on registers);
//  * mode 1: 16-byte direct-to-LDS loads, each wave streaming its share
//    through a ring of its own (the pattern of the decode kernels' weights).
// No counterpart in the reference.
#include "common.hpp"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

}  // namespace

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
