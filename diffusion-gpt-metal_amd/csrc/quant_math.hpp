// Scalar quantization arithmetic shared by the quantizer and the fused
// optimizer step (metal/kernels.metal:62-67, 86-96; src/Check.swift:399-431).
#pragma once

#include <hip/hip_runtime.h>

namespace dgm {

// code = clamp(rint(w / s), -lim, lim). rintf rounds half to even and the
// divide is IEEE correctly rounded (the library is built with
// -fhip-fp32-correctly-rounded-divide-sqrt, no fast math).
__device__ __forceinline__ int quant_code(float w, float s, int lim) {
    float r = rintf(w / s);
    int q = r > 2147483520.0f ? lim : (r < -2147483520.0f ? -lim : static_cast<int>(r));
    q = q > lim ? lim : q;
    q = q < -lim ? -lim : q;
    return q;
}

// s = max(maxAbs / qmax, 1e-8f), Swift's max(x, y) = y >= x ? y : x.
__device__ __forceinline__ float group_scale(float maxAbs, float qmax) {
    float d = maxAbs / qmax;
    return 1e-8f >= d ? 1e-8f : d;
}

}  // namespace dgm
