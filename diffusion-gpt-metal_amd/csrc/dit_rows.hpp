// Row helpers shared by the DiT block's fused kernels (dit.hip, dit_loop.hip):
// RMSNorm pieces with 16 lanes per row (4 rows per wave), and the SwiGLU
// logistic. Every operation rounds separately (fp contraction off), as the
// standalone kernels of metal/kernels.metal do.
#pragma once

#include <hip/hip_runtime.h>

namespace dgm_rows {

__device__ __forceinline__ float sum16(float v) {
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off, 16);
    return v;
}

// rstd of one row held by 16 lanes, J float4 chunks per lane:
// 1 / sqrt(mean(x^2) + eps) (rmsnorm_fwd, metal/kernels.metal:807-825).
template <int J>
__device__ __forceinline__ float rstd16(const float4 (&v)[J], int cols, float eps) {
#pragma clang fp contract(off)
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        ss += v[j].x * v[j].x;
        ss += v[j].y * v[j].y;
        ss += v[j].z * v[j].z;
        ss += v[j].w * v[j].w;
    }
    ss = sum16(ss);
    const float mean = ss / float(cols);
    return 1.0f / sqrtf(mean + eps);
}

// (x * rstd) * w, each product rounded.
__device__ __forceinline__ float4 norm4(float4 v, float rs, float4 w) {
#pragma clang fp contract(off)
    return make_float4((v.x * rs) * w.x, (v.y * rs) * w.y, (v.z * rs) * w.z, (v.w * rs) * w.w);
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// The logistic of swiglu_fwd (metal/kernels.metal:911-930), sign-split.
__device__ __forceinline__ float silu_sigmoid(float z) {
#pragma clang fp contract(off)
    if (z >= 0.0f) {
        const float e = expf(-z);
        return 1.0f / (1.0f + e);
    }
    const float e = expf(z);
    return e / (1.0f + e);
}

// Cross-lane sums and maxima on DPP and permlane swaps (no LDS round trips).
// Every lane of the reduced group gets the same bits: each step adds a value
// and its partner's, and addition is commutative.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]: lane ^ 1
    v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]: lane ^ 2
    v += dpp_f<0x141>(v);   // row_half_mirror: the other quad of the 8
    v += dpp_f<0x140>(v);   // row_mirror: the other 8 of the 16
    return v;
}

__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return v;
}

__device__ __forceinline__ float wave64_sum(float v) {
    v = row16_sum(v);
    const auto r16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                      false, false);   // rows 0 <-> 1, 2 <-> 3
    v = __builtin_bit_cast(float, uint32_t(r16[0])) + __builtin_bit_cast(float, uint32_t(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                      false, false);   // lanes 0-31 <-> 32-63
    return __builtin_bit_cast(float, uint32_t(r32[0])) + __builtin_bit_cast(float, uint32_t(r32[1]));
}

}  // namespace dgm_rows
