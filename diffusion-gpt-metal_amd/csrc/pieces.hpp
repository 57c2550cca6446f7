// Exact int8 pieces of fp32 activations, shared by the int8-MFMA forwards
// (gemm_skinny.hip, gemm_stream.hip): a row's values against a power of two
// 2^-sigma with max|x| * 2^sigma in [32, 64) are split as
//     u = x * 2^sigma = c0 + c1 / 128 + c2 / 128^2 + c3 / 128^3 + r,
// each c in [-64, 64], |r| <= 2^-22, and stored in the byte order the int4
// nibble unpack produces the B operand in.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace dgm_pieces {

// Byte offset of element k inside a piece row. int4: each 32-k chunk is stored
// as [16 even-k bytes][16 odd-k bytes]: masking a code dword keeps the even
// or the odd nibbles (16 * code as int8), so the B operands of an int4 block
// are its even k and its odd k.
template <int BITS>
__device__ __forceinline__ int piece_off(int k) {
    if constexpr (BITS == 4) return (k & ~31) + ((k & 1) << 4) + ((k & 31) >> 1);
    else return k;
}

// max that keeps a NaN (a non-finite row must not be silently dropped).
__device__ __forceinline__ float nmax(float a, float b) { return (b > a || b != b) ? b : a; }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = nmax(v, __shfl_xor(v, off, 64));
    return v;
}

// max |x| over 4 values; x - x is NaN for inf and NaN, so a non-finite value
// turns the maximum into NaN.
__device__ __forceinline__ float absmax4(float m, float4 v) {
    const float bad = (v.x - v.x) + (v.y - v.y) + (v.z - v.z) + (v.w - v.w);
    return nmax(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))) + bad);
}

// Exponent sigma with max|x| * 2^sigma in [32, 64); 0 for an all-zero row.
__device__ __forceinline__ int row_sigma(float maxabs) {
    if (!(maxabs > 0.0f)) return 0;
    int e;
    (void)frexpf(maxabs, &e);   // maxabs = f * 2^e, f in [0.5, 1)
    return 6 - e;
}

// u = x * 2^sigma = c0 + c1 / 128 + c2 / 128^2 + c3 / 128^3 + r, |r| <= 2^-22:
// every step (the difference and the scaling by 128) is exact in fp32.
__device__ __forceinline__ void split_pieces(float x, int sigma, int (&c)[4]) {
    float t = ldexpf(x, sigma);   // exact scaling
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = rintf(t);
        c[i] = int(a);
        t = (t - a) * 128.0f;
    }
}

// Writes the P pieces of 16 consecutive elements x[k0 .. k0+15] of one row to
// piece rows base[p] (byte pointers, row-local offsets).
template <int BITS, int P>
__device__ __forceinline__ void store_pieces16(int8_t* const (&base)[P], int k0, const float (&x)[16],
                                               int sigma) {
    int c[16][4];
#pragma unroll
    for (int i = 0; i < 16; ++i) split_pieces(x[i], sigma, c[i]);
#pragma unroll
    for (int p = 0; p < P; ++p) {
        if constexpr (BITS == 4) {
            // even k -> bytes [h*8, h*8+8) of the chunk, odd k -> 16 + same.
            uint32_t e0 = 0, e1 = 0, o0 = 0, o1 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                e0 |= (uint32_t(c[2 * i][p]) & 0xFFu) << (8 * i);
                e1 |= (uint32_t(c[8 + 2 * i][p]) & 0xFFu) << (8 * i);
                o0 |= (uint32_t(c[2 * i + 1][p]) & 0xFFu) << (8 * i);
                o1 |= (uint32_t(c[8 + 2 * i + 1][p]) & 0xFFu) << (8 * i);
            }
            const int off = piece_off<4>(k0);   // k0 % 16 == 0: even slot of k0
            *reinterpret_cast<uint2*>(base[p] + off) = make_uint2(e0, e1);
            *reinterpret_cast<uint2*>(base[p] + off + 16) = make_uint2(o0, o1);
        } else {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 16; ++i) w[i >> 2] |= (uint32_t(c[i][p]) & 0xFFu) << (8 * (i & 3));
            *reinterpret_cast<uint4*>(base[p] + k0) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

}  // namespace dgm_pieces
