// Shared definitions for the paged KV-cache library: page layout in HBM,
// bit-exact element conversions and launch-side helpers.
//
// Page layout (one allocation per layer; a block id addresses the same page
// in every layer's allocation, as one KVBlock holds every layer in
// pkg/engine/paged_kv.go:13-20):
//
//   f32 / f16   K  [kv_head][token_in_page][head_dim]      elements
//               V  [kv_head][head_dim][token_in_page]      elements
//   q8_0        K  int8 [kv_head][token][head_dim]
//               V  int8 [kv_head][head_dim][token]
//               KS fp16 [kv_head][token][head_dim/32]      block scales
//               VS fp16 [kv_head][head_dim/32][token]      block scales
//   q4_0        K  u8 [kv_head][token][head_dim/32][16]    byte j of a block:
//                                                          dim j | dim j+16 << 4
//               V  u8 [kv_head][head_dim/32][16][token]    the same pairs,
//                                                          token fastest
//               KS, VS fp16 as q8_0
//
// K is token-major so a (page, kv_head) K tile is one contiguous run whose
// rows feed the matrix-core A operand directly; V is stored dimension-major
// so that the same tile feeds the B operand of P*V with consecutive tokens
// per lane.  Gather converts back to the reference's contiguous
// [token][kv_dim] layout (kv.Key[l][t*kvDim + kvHead*headDim]).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gi {

enum KvType : int { KV_F32 = 0, KV_F16 = 1, KV_Q8_0 = 2, KV_Q4_0 = 3 };

struct PoolLayout {
    int kv_type;
    int num_layers;
    int num_kv_heads;
    int head_dim;
    int page_tokens;
    int64_t num_pages;
    int elt_bytes;      // 4, 2 or 1 (q4_0: 1, two values per byte)
    int64_t k_off;      // byte offsets inside one (layer, page) block
    int64_t v_off;
    int64_t ks_off;     // q8_0 / q4_0 only
    int64_t vs_off;     // q8_0 / q4_0 only
    int64_t page_bytes; // bytes of one (layer, page) block, 256-aligned
};

// Returns 0 and fills *out, or -1 when the shape is not supported.
inline int make_layout(int kv_type, int num_layers, int kvh, int hd, int P,
                       int64_t num_pages, PoolLayout *out)
{
    if (num_layers <= 0 || kvh <= 0 || hd <= 0 || P <= 0 || num_pages <= 0)
        return -1;
    if (kv_type != KV_F32 && kv_type != KV_F16 && kv_type != KV_Q8_0 && kv_type != KV_Q4_0)
        return -1;
    if (hd % 8 != 0)
        return -1;
    if ((kv_type == KV_Q8_0 || kv_type == KV_Q4_0) && hd % 32 != 0)
        return -1;
    PoolLayout L{};
    L.kv_type = kv_type;
    L.num_layers = num_layers;
    L.num_kv_heads = kvh;
    L.head_dim = hd;
    L.page_tokens = P;
    L.num_pages = num_pages;
    L.elt_bytes = kv_type == KV_F32 ? 4 : (kv_type == KV_F16 ? 2 : 1);
    int64_t tile = (int64_t)kvh * P * hd * L.elt_bytes;
    if (kv_type == KV_Q4_0)
        tile /= 2;
    L.k_off = 0;
    L.v_off = tile;
    int64_t end = 2 * tile;
    if (kv_type == KV_Q8_0 || kv_type == KV_Q4_0) {
        int64_t sc = (int64_t)kvh * P * (hd / 32) * 2;
        L.ks_off = end;
        L.vs_off = end + sc;
        end += 2 * sc;
    }
    L.page_bytes = (end + 255) / 256 * 256;
    *out = L;
    return 0;
}

// ---- element conversions (bit exact with pkg/quant/fp16.go) ---------------

// fp16 bits -> float, exact (pkg/quant/fp16.go:8-35 FP16ToFP32).  The
// hardware conversion is exact for every finite half and keeps NaN payloads
// the same way, but denormal halves must not be flushed: done in integer
// arithmetic so the float mode registers do not matter.
__device__ __host__ __forceinline__ float half_bits_to_float(uint32_t h)
{
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t f;
    if (ex == 0x1F) {
        f = sign | 0x7F800000u | (mant << 13);
    } else if (ex != 0) {
        f = sign | ((ex + 112u) << 23) | (mant << 13);
    } else if (mant == 0) {
        f = sign;
    } else {
        // subnormal half: value mant * 2^-24.  k = shifts that bring the
        // leading one to bit 10 (count of leading zeros within 11 bits);
        // the float exponent field is then 113 - k.
        int k = __builtin_clz(mant) - 21;
        mant = (mant << k) & 0x3FFu;
        f = sign | ((uint32_t)(113 - k) << 23) | (mant << 13);
    }
    return __builtin_bit_cast(float, f);
}

// float -> fp16 bits, dropping mantissa bits (pkg/quant/fp16.go:38-69
// FP32ToFP16).  Hardware conversions round to nearest even, so this is
// integer code.  NaN -> sign|0x7E00, |x| >= 65536 or Inf -> sign|0x7C00,
// |x| < 2^-25 -> signed zero.
__device__ __host__ __forceinline__ uint32_t float_to_half_bits_rtz(float v)
{
    uint32_t bits = __builtin_bit_cast(uint32_t, v);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int ex = (int)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x7FFFFFu;
    if (ex == 255)
        return sign | (mant ? 0x7E00u : 0x7C00u);
    ex -= 112;
    if (ex >= 31)
        return sign | 0x7C00u;
    if (ex <= 0) {
        if (ex < -10)
            return sign;
        return sign | (((mant | 0x800000u) >> (1 - ex)) >> 13);
    }
    return sign | ((uint32_t)ex << 10) | (mant >> 13);
}

// Q8_0 block scale from the block's largest magnitude (pkg/quant/quant.go:
// 418-435): scale = amax/127 (float division), truncated to fp16, widened
// back, inverse = 1/scale.  Both divisions are done in double and rounded
// once to float, which equals the correctly rounded float quotient because
// double carries more than 2*24+2 bits.  Returns the fp16 bits of the scale
// and the inverse through *inv (0 when the scale is 0, Inf or NaN-free zero).
__device__ __host__ __forceinline__ uint32_t q8_scale(float amax, float *inv)
{
    float scale = (float)((double)amax / 127.0);
    uint32_t d16 = 0;
    if (scale > 0.0f) {
        d16 = float_to_half_bits_rtz(scale);
        scale = half_bits_to_float(d16);
    }
    float iv = 0.0f;
    if (scale > 0.0f)
        iv = (float)(1.0 / (double)scale);
    *inv = iv;
    return d16;
}

// One Q8_0 element: clamp x*inv to [-128, 127] and round half away from
// zero (quant.go:440-449: math.Round then int8()).  NaN -> 0.
__device__ __host__ __forceinline__ int q8_quant(float x, float inv)
{
    if (!(inv > 0.0f))
        return 0;
    float v = x * inv;
    if (v > 127.0f)
        v = 127.0f;
    else if (v < -128.0f)
        v = -128.0f;
    if (v != v)
        return 0;
    float t = __builtin_truncf(v);
    float fr = v - t; // exact for |v| < 2^23
    if (fr >= 0.5f)
        t += 1.0f;
    else if (fr <= -0.5f)
        t -= 1.0f;
    return (int)t;
}

// Q4_0 block scale (pkg/quant/quant.go:478-490): scale = amax/7 in float,
// truncated to fp16 and widened back, inverse = 1/scale; the divisions are
// done in double and rounded once, as for q8_scale.
__device__ __host__ __forceinline__ uint32_t q4_scale(float amax, float *inv)
{
    float scale = (float)((double)amax / 7.0);
    uint32_t d16 = 0;
    if (scale > 0.0f) {
        d16 = float_to_half_bits_rtz(scale);
        scale = half_bits_to_float(d16);
    }
    float iv = 0.0f;
    if (scale > 0.0f)
        iv = (float)(1.0 / (double)scale);
    *inv = iv;
    return d16;
}

// One Q4_0 nibble (quant.go:494-502): int(math.Round(x*inv)) + 8 clamped to
// [0, 15], 8 when the inverse is 0.  Go's amd64 int() of a NaN is the
// minimum int64, which clamps to 0.  |x*inv| stays below 15 for finite x
// (the fp16 scale is at least half of amax/7), so the rounding is exact.
__device__ __host__ __forceinline__ int q4_quant(float x, float inv)
{
    if (!(inv > 0.0f))
        return 8;
    float v = x * inv;
    if (v != v)
        return 0;
    float t = __builtin_truncf(v);
    float fr = v - t;
    if (fr >= 0.5f)
        t += 1.0f;
    else if (fr <= -0.5f)
        t -= 1.0f;
    int q = (int)t + 8;
    return q < 0 ? 0 : (q > 15 ? 15 : q);
}

// |x| as an orderable key for the block maximum.  NaN inputs are skipped by
// the reference's `v > maxVal` compare (quant.go:420-423), so they map to 0.
__device__ __host__ __forceinline__ uint32_t abs_key(float x)
{
    uint32_t a = __builtin_bit_cast(uint32_t, x) & 0x7FFFFFFFu;
    return a > 0x7F800000u ? 0u : a;
}

// Power-of-two exponent e such that max_abs * 2^e <= 2^14, clamped to
// [-60, 60] (0 for a zero or non-finite input).  Multiplying by 2^e is exact,
// and it keeps both halves of an fp16 hi/lo split in the normal range, where
// each carries the full 11-bit significand.
__device__ __host__ __forceinline__ int pow2_exponent_for(float max_abs)
{
    uint32_t bits = __builtin_bit_cast(uint32_t, max_abs);
    int ex = (int)((bits >> 23) & 0xFF);
    if (ex == 0 || ex == 255)
        return 0;
    int ceil_log2 = ex - 127 + ((bits & 0x7FFFFFu) ? 1 : 0);
    int e = 14 - ceil_log2;
    return e < -60 ? -60 : (e > 60 ? 60 : e);
}

// Error flag bits raised by kernels into the handle's device status word.
enum : int { FLAG_BAD_PAGE = 1, FLAG_BAD_SLOT = 2, FLAG_BAD_POS = 4 };

} // namespace gi
