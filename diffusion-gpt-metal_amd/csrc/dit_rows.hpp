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

}  // namespace dgm_rows
