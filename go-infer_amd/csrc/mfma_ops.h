// Matrix-core helpers shared by the decode and matmul kernels: operand
// types, the 16x16x32 f16 product, and exact conversions of quantised codes
// (int8 and Q4_0 nibbles) into fp16 operands.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gi {
namespace mfma_ops {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Maximum of x and its value in lane l ^ 16 (l ^ 32): one permlane swap
// (a VALU instruction, with no trip through LDS) hands each lane the other
// row's (half's) value in one of its two results.
__device__ __forceinline__ float max_xor16(float x)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    // (elements copied out before the bit cast: hipcc's __builtin_bit_cast
    // of a vector element reads element 0 whatever the index)
    const uint32_t r0 = r[0], r1 = r[1];
    return fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}
__device__ __forceinline__ float max_xor32(float x)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}

// -1.0f in a register the optimiser cannot see through, so that x - hi
// (hi a half) is selected as one mixed-precision multiply-add reading the
// half in place, not as a conversion and a subtraction.
__device__ __forceinline__ float opaque_neg1()
{
    float v;
    asm volatile("" : "=s"(v) : "0"(-1.0f));
    return v;
}

// x0, x1 (already scaled into fp16 range) as packed hi + lo halves: hi = x
// cut to 11 significant bits by the round-toward-zero conversion, lo = x - hi
// (one mixed-precision multiply-add reading hi in place, exact in float32)
// rounded to nearest, so hi + lo is x to 2^-23 relative.  neg1 is -1
// (opaque_neg1).
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t &hi, uint32_t &lo, float neg1)
{
    const h2 h = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(x0, x1));
    hi = __builtin_bit_cast(uint32_t, h);
    const h2 l = {(_Float16)fmaf((float)h[0], neg1, x0), (_Float16)fmaf((float)h[1], neg1, x1)};
    lo = __builtin_bit_cast(uint32_t, l);
}

// Eight int8 codes -> eight exact fp16 values: (x ^ 0x80) is x + 128 as an
// unsigned byte, 0x64 above it makes the half 1024 + x + 128, and the bias
// 1152 is subtracted.
__device__ __forceinline__ h8 i8x8_to_h8(u2 w)
{
    const uint32_t x0 = w.x ^ 0x80808080u, x1 = w.y ^ 0x80808080u;
    const uint32_t c = 0x64646464u;
    const uint32_t u[4] = {__builtin_amdgcn_perm(c, x0, 0x04010400u), __builtin_amdgcn_perm(c, x0, 0x04030402u),
                           __builtin_amdgcn_perm(c, x1, 0x04010400u), __builtin_amdgcn_perm(c, x1, 0x04030402u)};
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    h8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const h2 t = __builtin_bit_cast(h2, u[i]) - bias;
        r[2 * i] = t[0];
        r[2 * i + 1] = t[1];
    }
    return r;
}

// Eight Q4_0 nibbles n (the low nibbles of w's bytes when sh == 0, the high
// ones when sh == 4) -> eight exact fp16 values n - 8: 0x64 above the
// nibble makes the half 1024 + n, and the bias 1032 is subtracted.
__device__ __forceinline__ h8 u4x8_to_h8(u2 w, int sh)
{
    const uint32_t x0 = (w.x >> sh) & 0x0F0F0F0Fu, x1 = (w.y >> sh) & 0x0F0F0F0Fu;
    const uint32_t c = 0x64646464u;
    const uint32_t u[4] = {__builtin_amdgcn_perm(c, x0, 0x04010400u), __builtin_amdgcn_perm(c, x0, 0x04030402u),
                           __builtin_amdgcn_perm(c, x1, 0x04010400u), __builtin_amdgcn_perm(c, x1, 0x04030402u)};
    const h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    h8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const h2 t = __builtin_bit_cast(h2, u[i]) - bias;
        r[2 * i] = t[0];
        r[2 * i + 1] = t[1];
    }
    return r;
}

// Eight Q4_0 nibbles left in place -> eight exact fp16 values: the bytes of
// w masked by m (0x0F0F0F0F keeps the low nibbles n, 0xF0F0F0F0 the high
// ones as 16n) under 0x64 make the halves 1024 + n or 1024 + 16n, and the
// bias (1032 or 1152) leaves n - 8 or 16(n - 8).  A high-nibble operand so
// carries a factor 16 that the caller takes out of the other operand or of
// the accumulator, and needs no shift.
__device__ __forceinline__ h8 u4x8_masked_to_h8(u2 w, uint32_t m, h2 bias)
{
    const uint32_t x0 = w.x & m, x1 = w.y & m;
    const uint32_t c = 0x64646464u;
    const uint32_t u[4] = {__builtin_amdgcn_perm(c, x0, 0x04010400u), __builtin_amdgcn_perm(c, x0, 0x04030402u),
                           __builtin_amdgcn_perm(c, x1, 0x04010400u), __builtin_amdgcn_perm(c, x1, 0x04030402u)};
    h8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const h2 t = __builtin_bit_cast(h2, u[i]) - bias;
        r[2 * i] = t[0];
        r[2 * i + 1] = t[1];
    }
    return r;
}

// Eight Q4_0 nibbles -> eight fp16 subnormals n * 2^-24, exact: the mask m
// (0x000F000F: low nibbles n; 0x00F000F0: high nibbles in place, 16n) keeps
// one nibble of bytes 0 and 2 of a word in the low bits of its two halves,
// and the word shifted right by 8 gives bytes 1 and 3.  The operand order is
// bytes 0, 2, 1, 3, 4, 6, 5, 7 (the other operand of the product must follow
// it); the code offset 8 is left to the caller.  One AND per two halves, and
// one shift per four, against a permute and a packed subtract per two
// halves for the normal 1024 + n form.
__device__ __forceinline__ h8 u4x8_sub_to_h8(u2 w, uint32_t m)
{
    const u4 r = {w.x & m, (w.x >> 8) & m, w.y & m, (w.y >> 8) & m};
    return __builtin_bit_cast(h8, r);
}

// Eight int8 codes x -> eight fp16 subnormals (x + 128) * 2^-24, exact and in
// order: (x ^ 0x80) is x + 128 as an unsigned byte, placed in the low byte of
// a half whose high byte is 0.  The offset 128 is left to the caller.
__device__ __forceinline__ h8 i8x8_sub_to_h8(u2 w)
{
    const uint32_t x0 = w.x ^ 0x80808080u, x1 = w.y ^ 0x80808080u;
    const u4 r = {__builtin_amdgcn_perm(0u, x0, 0x0C010C00u), __builtin_amdgcn_perm(0u, x0, 0x0C030C02u),
                  __builtin_amdgcn_perm(0u, x1, 0x0C010C00u), __builtin_amdgcn_perm(0u, x1, 0x0C030C02u)};
    return __builtin_bit_cast(h8, r);
}

} // namespace mfma_ops
} // namespace gi
