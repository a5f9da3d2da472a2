// Stores of one token's K/V elements into a page, in the page type's
// format: the per-element half of KVCache.Write (pkg/engine/kvcache.go:146-180)
// on the page layout of gi_common.h.  Shared by the append kernels and by the
// decode step that the matrix-core decode kernels fuse in front of their
// attention.
#pragma once

#include "gi_common.h"

namespace gi {

// 32-lane maximum of an unsigned key (lanes of one quantisation block).
__device__ __forceinline__ uint32_t max32(uint32_t x)
{
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) {
        uint32_t y = (uint32_t)__shfl_xor((int)x, m, 32);
        x = x > y ? x : y;
    }
    return x;
}

// Q4_0 quantise-and-store of element e of one token vector (slot s of page
// pg), called by all 32 lanes of the block's lane group: lane j < 16 writes
// byte j of the K and of the V block (element j low, element j + 16 high,
// quant.go:504), lane 0 the two fp16 scales.  ok == false only joins the
// shuffles.
__device__ __forceinline__ void quant_store_q4(const PoolLayout &L, uint8_t *pg, int s, int e, float kx,
                                               float vx, bool ok)
{
    const int hd = L.head_dim, nb = hd / 32, P = L.page_tokens;
    float kinv, vinv;
    uint32_t kd = q4_scale(__builtin_bit_cast(float, max32(abs_key(kx))), &kinv);
    uint32_t vd = q4_scale(__builtin_bit_cast(float, max32(abs_key(vx))), &vinv);
    const int kq = q4_quant(kx, kinv), vq = q4_quant(vx, vinv);
    const int kq_hi = __shfl_down(kq, 16, 32), vq_hi = __shfl_down(vq, 16, 32);
    if (!ok)
        return;
    const int kvh = e / hd, d = e - kvh * hd, blk = d >> 5, j = d & 31;
    if (j < 16) {
        pg[L.k_off + (((int64_t)kvh * P + s) * nb + blk) * 16 + j] = (uint8_t)(kq | (kq_hi << 4));
        pg[L.v_off + (((int64_t)kvh * nb + blk) * 16 + j) * P + s] = (uint8_t)(vq | (vq_hi << 4));
    }
    if (j == 0) {
        reinterpret_cast<uint16_t *>(pg + L.ks_off)[((int64_t)kvh * P + s) * nb + blk] = (uint16_t)kd;
        reinterpret_cast<uint16_t *>(pg + L.vs_off)[((int64_t)kvh * nb + blk) * P + s] = (uint16_t)vd;
    }
}

// Element d of kv head kvh of one token (K value kx, V value vx) into slot s
// of page pg: f32 copied, f16 truncated (FP32ToFP16, fp16.go:38-69), q8_0 and
// q4_0 quantised per 32-element block (QuantizeQ8_0 / QuantizeQ4_0,
// quant.go:407-521).  For the quantised types all 32 lanes of the element's
// block call it together; ok == false then only joins the shuffles.
template <int KT>
__device__ __forceinline__ void store_token_elem(const PoolLayout &L, uint8_t *pg, int s, int kvh, int d,
                                                 float kx, float vx, bool ok)
{
    const int hd = L.head_dim, P = L.page_tokens, nb = hd / 32;
    const int64_t ki = ((int64_t)kvh * P + s) * hd + d;
    const int64_t vi = ((int64_t)kvh * hd + d) * P + s;
    if constexpr (KT == KV_F32) {
        if (!ok)
            return;
        reinterpret_cast<float *>(pg + L.k_off)[ki] = kx;
        reinterpret_cast<float *>(pg + L.v_off)[vi] = vx;
    } else if constexpr (KT == KV_F16) {
        if (!ok)
            return;
        reinterpret_cast<uint16_t *>(pg + L.k_off)[ki] = (uint16_t)float_to_half_bits_rtz(kx);
        reinterpret_cast<uint16_t *>(pg + L.v_off)[vi] = (uint16_t)float_to_half_bits_rtz(vx);
    } else if constexpr (KT == KV_Q8_0) {
        float kinv, vinv;
        const uint32_t kd = q8_scale(__builtin_bit_cast(float, max32(abs_key(kx))), &kinv);
        const uint32_t vd = q8_scale(__builtin_bit_cast(float, max32(abs_key(vx))), &vinv);
        if (!ok)
            return;
        const int blk = d >> 5;
        reinterpret_cast<int8_t *>(pg + L.k_off)[ki] = (int8_t)q8_quant(kx, kinv);
        reinterpret_cast<int8_t *>(pg + L.v_off)[vi] = (int8_t)q8_quant(vx, vinv);
        if ((d & 31) == 0) {
            reinterpret_cast<uint16_t *>(pg + L.ks_off)[((int64_t)kvh * P + s) * nb + blk] = (uint16_t)kd;
            reinterpret_cast<uint16_t *>(pg + L.vs_off)[((int64_t)kvh * nb + blk) * P + s] = (uint16_t)vd;
        }
    } else {
        quant_store_q4(L, pg, s, kvh * hd + d, kx, vx, ok);
    }
}

} // namespace gi
