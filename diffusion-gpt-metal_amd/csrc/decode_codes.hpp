// Code-dword conversions shared by the decode-shaped forwards
// (gemm_decode.hip, gemm_stream.hip): int4 / int8 weight codes into the
// 16-bit MFMA operands, and the order in which they produce k values.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace dgm_codes {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// k offset inside a block of fragment element t (0..7) of lane group q at
// block step kk: the order in which the weight conversion below produces
// f16 values from a code dword.
template <int BITS>
__host__ __device__ constexpr int frag_k(int q, int kk, int t) {
    if (BITS == 4) {
        const int pi[8] = {0, 4, 1, 5, 2, 6, 3, 7};
        return 32 * q + 8 * kk + pi[t];
    } else {
        const int pi[8] = {0, 2, 1, 3, 4, 6, 5, 7};
        return 16 * q + 8 * kk + pi[t];
    }
}

// (d & m & ~f) | (~d & m & f) | (~m & c): the bits of d under the mask m,
// flipped where f is set, the constant c elsewhere. One v_bitop3 with f and c
// packed into one operand (they never overlap): truth table 0x6A over
// (d, m, fc) (table bit (d << 2) | (m << 1) | fc). The builtin, not inline
// asm, so that the compiler sees the result register: an MFMA that reads a
// VALU result needs wait states the compiler inserts only for what it sees.
__device__ __forceinline__ uint32_t pick_flip(uint32_t d, uint32_t m, uint32_t fc) {
    return __builtin_amdgcn_bitop3_b32(d, m, fc, 0x6A);
}

// One code dword (int4: 8 nibbles; int8: 4 bytes) -> f16 pairs in frag_k
// order. Each two's-complement code is flipped to offset binary (sign bit
// inverted) and placed under the exponent of 1024.0 (0x6400) in the same
// operation; one packed f16 FMA removes the offset.
template <int BITS>
__device__ __forceinline__ void codes_to_f16(uint32_t dw, f16x2* out) {
    const uint32_t y = dw >> 8;
    if constexpr (BITS == 4) {
        const uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u;
        const uint32_t flo = 0x64086408u, fhi = 0x64806480u;   // 0x6400 | offset-binary flip
        const f16x2 s1 = {_Float16(1.0f), _Float16(1.0f)}, s16 = {_Float16(0.0625f), _Float16(0.0625f)};
        const f16x2 o1 = {_Float16(-1032.0f), _Float16(-1032.0f)}, o16 = {_Float16(-72.0f), _Float16(-72.0f)};
        out[0] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, pick_flip(dw, mlo, flo)), s1, o1);   // k 0, 4
        out[1] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, pick_flip(dw, mhi, fhi)), s16, o16); // k 1, 5
        out[2] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, pick_flip(y, mlo, flo)), s1, o1);    // k 2, 6
        out[3] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, pick_flip(y, mhi, fhi)), s16, o16);  // k 3, 7
    } else {
        const uint32_t mlo = 0x00FF00FFu, flo = 0x64806480u;
        const f16x2 s1 = {_Float16(1.0f), _Float16(1.0f)}, o1 = {_Float16(-1152.0f), _Float16(-1152.0f)};
        out[0] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, pick_flip(dw, mlo, flo)), s1, o1);   // k 0, 2
        out[1] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, pick_flip(y, mlo, flo)), s1, o1);    // k 1, 3
    }
}

// One int4 code dword (8 nibbles) -> bf16 pairs 128 + (code + 8), in frag_k
// order: bf16 keeps 7 mantissa bits, so each nibble goes to bits 0-3 of its
// half (three shifts) and is flipped to offset binary under the exponent of
// 128.0 (0x4300) by one v_bitop3. The offset 136 = 128 + 8 is removed in the
// accumulator (see the reduced-precision path of decode_small_kernel).
__device__ __forceinline__ bf16x8 codes_to_bf16_off(uint32_t dw) {
    const uint32_t m = 0x000F000Fu, fc = 0x43084308u;
    const u32x4 o = {pick_flip(dw, m, fc), pick_flip(dw >> 4, m, fc), pick_flip(dw >> 8, m, fc),
                     pick_flip(dw >> 12, m, fc)};   // k 0,4 | 1,5 | 2,6 | 3,7
    return __builtin_bit_cast(bf16x8, o);
}

}  // namespace dgm_codes
