/*
 * oracle/cpu_ref.c -- CPU restatement of go-infer's paged-KV / attention
 * arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP path is
 * compared against (tests/, __graft_entry__.smoke() and the cpu_baseline leg
 * of bench.py).  No product code links, loads or calls it.
 *
 * The reference is Go (module go-inference).  Go is not available here, so
 * every routine below restates, in C11, the Go function cited beside it.
 * Built with -O2 -ffp-contract=off (see oracle/build.py) so that float
 * arithmetic is evaluated exactly as written with no fused multiply-add,
 * which is what Go's default amd64 code generation (GOAMD64=v1) does.
 *
 * Pinning (how each function is checked independently of this file):
 *   ref_fp32_to_fp16 / ref_fp16_to_fp32  -- numpy float16 conversion adjusted
 *       to round-toward-zero, all 65536 halves, boundary sweeps;
 *       pkg/quant/quant_test.go:10-19 restated.
 *   ref_quantize_q8_0 / ref_dequantize_q8_0 -- exact-rational closed form per
 *       element, max-element-maps-to-127 invariant, hand-built special cases;
 *       quant_test.go:129-143 and engine_test.go:251-273 restated.
 *   ref_dot_vec_f32 -- an input where the 8-wide chunk order gives a
 *       different float32 result from a sequential sum.
 *   ref_softmax -- kernels_test.go:23-37 restated, float64 closed form.
 *   ref_math_sqrt -- bit patterns of 1/sqrt(64) and 1/sqrt(128).
 *   ref_attention_* -- float64 textbook softmax(QK^T * scale) V in numpy,
 *       and prefill == per-token decode (engine_test.go:219-249 restated).
 *   ref_quantize_q4_0 / ref_dequantize_q4_0 -- exact-rational closed form
 *       per element, hand-built special cases (NaN -> nibble 0, Inf block ->
 *       all 8, ties away from zero, subnormal-scale clamps);
 *       quant_test.go:21-54, 145-160 and engine_test.go:275-297 restated.
 *   ref_apply_rope / ref_rope_table -- kernels_test.go:39-46 restated;
 *       cos/sin against a 50-digit evaluation of cos(pos * theta^(-2i/d));
 *       the rotation of (1, 0) lands at angle +pos*freq (sign and pairing);
 *       pair norms and the relative-position property of q.k.
 */
#define _POSIX_C_SOURCE 200809L /* pthread barriers under -std=c11 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- fp16 <-> fp32 ------------------------------------------------------ */

/* pkg/quant/fp16.go:8-35 FP16ToFP32: exact widening, subnormals normalised
 * by shifting, Inf/NaN keep their mantissa bits. */
float ref_fp16_to_fp32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (uint32_t)(h & 0x7C00u) >> 10;
    uint32_t mant = (uint32_t)(h & 0x03FFu);
    uint32_t f;
    if (ex == 0) {
        if (mant == 0) {
            f = sign;
        } else {
            ex = 1;
            while ((mant & 0x0400u) == 0) {
                mant <<= 1;
                ex--; /* unsigned wrap is intended: ex+(127-15) fixes it */
            }
            mant &= 0x03FFu;
            f = sign | ((ex + (127u - 15u)) << 23) | (mant << 13);
        }
    } else if (ex == 0x1F) {
        f = sign | 0x7F800000u | (mant << 13);
    } else {
        f = sign | ((ex + (127u - 15u)) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &f, 4);
    return out;
}

/* pkg/quant/fp16.go:38-69 FP32ToFP16: mantissa bits are dropped (round toward
 * zero); NaN -> sign|0x7E00, Inf and every |x| >= 65536 -> sign|0x7C00;
 * |x| < 2^-25 -> signed zero; subnormals shift the implicit-one mantissa. */
uint16_t ref_fp32_to_fp16(float val)
{
    uint32_t bits;
    memcpy(&bits, &val, 4);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int ex = (int)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x007FFFFFu;
    if (ex == 255) {
        if (mant != 0)
            return (uint16_t)(sign | 0x7E00u);
        return (uint16_t)(sign | 0x7C00u);
    }
    ex = ex - 127 + 15;
    if (ex >= 31)
        return (uint16_t)(sign | 0x7C00u);
    if (ex <= 0) {
        if (ex < -10)
            return (uint16_t)sign;
        mant = (mant | 0x00800000u) >> (1 - ex);
        return (uint16_t)(sign | (mant >> 13));
    }
    return (uint16_t)(sign | ((uint32_t)ex << 10) | (mant >> 13));
}

void ref_fp32_to_fp16_array(const float *src, uint16_t *dst, int64_t n)
{
    for (int64_t i = 0; i < n; i++)
        dst[i] = ref_fp32_to_fp16(src[i]);
}

void ref_fp16_to_fp32_array(const uint16_t *src, float *dst, int64_t n)
{
    for (int64_t i = 0; i < n; i++)
        dst[i] = ref_fp16_to_fp32(src[i]);
}

/* ---- Q8_0 ---------------------------------------------------------------- */

/* Go's math.Round: nearest integer, halves away from zero.  C's round() has
 * the same definition. */
static double go_round(double x) { return round(x); }

/* Go's int8(float64) conversion of a value already clamped to [-128, 127].
 * A NaN (NaN inputs pass the clamp untouched) converts to 0 on amd64, where
 * Go converts through CVTTSD2SQ and keeps the low byte; C leaves it
 * undefined, so it is spelled out. */
static int8_t go_int8(double x)
{
    if (x != x)
        return 0;
    return (int8_t)(int)x;
}

/* pkg/quant/quant.go:407-456 QuantizeQ8_0.  Blocks of 32; a short final
 * block is zero padded.  out must hold ((n+31)/32)*34 bytes. */
void ref_quantize_q8_0(const float *src, int64_t n, uint8_t *out)
{
    int64_t nblocks = (n + 31) / 32;
    memset(out, 0, (size_t)(nblocks * 34));
    for (int64_t b = 0; b < nblocks; b++) {
        int64_t start = b * 32;
        int64_t end = start + 32;
        if (end > n)
            end = n;
        float maxv = 0.0f;
        for (int64_t i = start; i < end; i++) {
            /* float32(math.Abs(float64(x))) == fabsf(x) exactly */
            float v = (float)fabs((double)src[i]);
            if (v > maxv)
                maxv = v;
        }
        float scale = maxv / 127.0f;
        uint16_t d16 = 0;
        if (scale > 0) {
            d16 = ref_fp32_to_fp16(scale);
            scale = ref_fp16_to_fp32(d16);
        }
        float inv = 0.0f;
        if (scale > 0)
            inv = 1.0f / scale;
        uint8_t *blk = out + b * 34;
        blk[0] = (uint8_t)(d16 & 0xFF); /* little endian */
        blk[1] = (uint8_t)(d16 >> 8);
        for (int i = 0; i < 32; i++) {
            int8_t q = 0;
            if (start + i < n && inv > 0) {
                float v = src[start + i] * inv;
                if (v > 127.0f)
                    v = 127.0f;
                else if (v < -128.0f)
                    v = -128.0f;
                q = go_int8(go_round((double)v));
            }
            blk[2 + i] = (uint8_t)q;
        }
    }
}

/* pkg/quant/quant.go:196-213 DequantizeQ8_0: out = float32(int8 q) * d. */
void ref_dequantize_q8_0(const uint8_t *data, int64_t n, float *out)
{
    int64_t nblocks = n / 32;
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = data + b * 34;
        float d = ref_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < 32; j++)
            out[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

/* ---- Q4_0 ---------------------------------------------------------------- */

/* Go's int(float64) on amd64 (CVTTSD2SQ): truncation toward zero, and the
 * "integer indefinite" 0x8000000000000000 for NaN and for values outside
 * int64 -- C leaves both undefined, so they are spelled out. */
static int64_t go_int(double x)
{
    if (x != x || x >= 9223372036854775808.0 || x < -9223372036854775808.0)
        return INT64_MIN;
    return (int64_t)x;
}

/* One Q4_0 element (quant.go:481-502): int(math.Round(float64(x*inv))) + 8,
 * clamped to [0, 15]; an element past the vector's end, or a zero inverse,
 * gives 8.  A NaN product converts to INT64_MIN, so it clamps to 0. */
static int q4_element(const float *src, int64_t idx, int64_t n, float inv)
{
    if (idx >= n || !(inv > 0))
        return 8;
    float v = src[idx] * inv;
    int64_t q = go_int(go_round((double)v));
    if (q != INT64_MIN)
        q += 8;
    if (q < 0)
        q = 0;
    else if (q > 15)
        q = 15;
    return (int)q;
}

/* pkg/quant/quant.go:458-521 QuantizeQ4_0: per block of 32, amax as in
 * Q8_0, scale = amax / 7 (float32), truncated to fp16 and widened back,
 * inv = 1 / scale; byte j of the block's 16 holds element j in its low
 * nibble and element j + 16 in its high nibble.  out must hold
 * ((n+31)/32)*18 bytes. */
void ref_quantize_q4_0(const float *src, int64_t n, uint8_t *out)
{
    int64_t nblocks = (n + 31) / 32;
    for (int64_t b = 0; b < nblocks; b++) {
        int64_t start = b * 32;
        int64_t end = start + 32;
        if (end > n)
            end = n;
        float maxv = 0.0f;
        for (int64_t i = start; i < end; i++) {
            float v = (float)fabs((double)src[i]);
            if (v > maxv)
                maxv = v;
        }
        float scale = maxv / 7.0f;
        uint16_t d16 = 0;
        if (scale > 0) {
            d16 = ref_fp32_to_fp16(scale);
            scale = ref_fp16_to_fp32(d16);
        }
        float inv = 0.0f;
        if (scale > 0)
            inv = 1.0f / scale;
        uint8_t *blk = out + b * 18;
        blk[0] = (uint8_t)(d16 & 0xFF);
        blk[1] = (uint8_t)(d16 >> 8);
        for (int j = 0; j < 16; j++) {
            int q0 = q4_element(src, start + j, n, inv);
            int q1 = q4_element(src, start + j + 16, n, inv);
            blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

/* pkg/quant/quant.go:96-116 DequantizeQ4_0: element j = (low nibble of byte
 * j - 8) * d, element j + 16 = (high nibble - 8) * d. */
void ref_dequantize_q4_0(const uint8_t *data, int64_t n, float *out)
{
    int64_t nblocks = n / 32;
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = data + b * 18;
        float d = ref_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < 16; j++) {
            int x0 = (int)(blk[2 + j] & 0x0F) - 8;
            int x1 = (int)((blk[2 + j] >> 4) & 0x0F) - 8;
            out[b * 32 + j] = (float)x0 * d;
            out[b * 32 + j + 16] = (float)x1 * d;
        }
    }
}

/* ---- dot / softmax / scale ---------------------------------------------- */

/* pkg/quant/quant.go:548-567 DotVecF32: 8-wide chunks summed left to right,
 * each chunk added to the running sum, then a scalar tail. */
float ref_dot_vec_f32(const float *x, const float *w, int n)
{
    float sum = 0.0f;
    int i = 0;
    for (; i <= n - 8; i += 8) {
        float c = x[i] * w[i];
        c = c + x[i + 1] * w[i + 1];
        c = c + x[i + 2] * w[i + 2];
        c = c + x[i + 3] * w[i + 3];
        c = c + x[i + 4] * w[i + 4];
        c = c + x[i + 5] * w[i + 5];
        c = c + x[i + 6] * w[i + 6];
        c = c + x[i + 7] * w[i + 7];
        sum += c;
    }
    for (; i < n; i++)
        sum += x[i] * w[i];
    return sum;
}

/* pkg/math/kernels.go:48-70 Softmax: two passes, exp evaluated in float64
 * and rounded to float32, float32 running sum, multiply by 1/sum. */
void ref_softmax(float *x, int n)
{
    if (n <= 0)
        return;
    float maxv = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > maxv)
            maxv = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        float v = (float)exp((double)(x[i] - maxv));
        x[i] = v;
        sum += v;
    }
    if (sum > 0) {
        float inv = 1.0f / sum;
        for (int i = 0; i < n; i++)
            x[i] *= inv;
    }
}

/* pkg/engine/forward.go:771-780 math_sqrt: ten Newton steps from x/2. */
double ref_math_sqrt(double x)
{
    if (x <= 0)
        return 0;
    double z = x / 2;
    for (int i = 0; i < 10; i++)
        z = (z + x / z) / 2;
    return z;
}

/* pkg/engine/forward.go:33 attnScale = float32(1.0 / math_sqrt(headDim)). */
float ref_attn_scale(int head_dim)
{
    return (float)(1.0 / ref_math_sqrt((double)head_dim));
}

/* ---- attention over a contiguous per-layer cache ------------------------ */

/* pkg/engine/forward.go:242-267 (decode).  kc/vc are [L][kv_dim] float32 as
 * indexed by kv.Key[l][t*kvDim + kvHead*headDim]; q/out are [H][hd].
 * q-head h reads kv head h / (H/KVH) (forward.go:249, config.go:59-64).
 * scores must hold L floats. */
/* One q-head of forward.go:243-266: out zeroed (243-245), scores over the
 * first L tokens of kv head kvh (252-255), Softmax, then the weighted V sum
 * in token order (259-266). */
static void attend_head(const float *qh, const float *kc, const float *vc,
                        float *oh, int kvh, int kv_dim, int hd, int L,
                        float scale, float *scores)
{
    for (int d = 0; d < hd; d++)
        oh[d] = 0.0f;
    for (int t = 0; t < L; t++)
        scores[t] = ref_dot_vec_f32(qh, kc + (int64_t)t * kv_dim + kvh * hd, hd) * scale;
    ref_softmax(scores, L);
    for (int t = 0; t < L; t++) {
        const float *vt = vc + (int64_t)t * kv_dim + kvh * hd;
        float wgt = scores[t];
        for (int d = 0; d < hd; d++)
            oh[d] += wgt * vt[d];
    }
}

void ref_attention_decode(const float *q, const float *kc, const float *vc,
                          float *out, int H, int KVH, int hd, int L,
                          float scale, float *scores)
{
    int kv_dim = KVH * hd;
    int kv_mul = H / KVH;
    for (int h = 0; h < H; h++)
        attend_head(q + (int64_t)h * hd, kc, vc, out + (int64_t)h * hd, h / kv_mul,
                    kv_dim, hd, L, scale, scores);
}

/* pkg/engine/forward.go:547-577 (chunked prefill, causal).  The chunk's own
 * K/V are already stored (forward.go:527-545).  Token b of the chunk attends
 * over activeContext = min(start_pos+b+1, max_seq) cached tokens.  q/out are
 * [chunk][H][hd].  scores must hold min(start_pos+chunk, max_seq) floats. */
void ref_attention_prefill(const float *q, const float *kc, const float *vc,
                           float *out, int H, int KVH, int hd, int start_pos,
                           int chunk, int max_seq, float scale, float *scores)
{
    for (int b = 0; b < chunk; b++) {
        int active = start_pos + b + 1;
        if (active > max_seq)
            active = max_seq;
        ref_attention_decode(q + (int64_t)b * H * hd, kc, vc,
                             out + (int64_t)b * H * hd, H, KVH, hd, active,
                             scale, scores);
    }
}

/* ---- KVCache.Write / Get on one contiguous layer ------------------------- */

/* Stored-format bytes per token vector for kv type t (0 f32, 1 f16, 2 q8_0,
 * 3 q4_0).  Q8_0 is ((kvDim+31)/32)*34, Q4_0 ((kvDim+31)/32)*18
 * (pkg/engine/kvcache.go:92-105, 152, 164). */
int64_t ref_bytes_per_vec(int kv_type, int kv_dim)
{
    if (kv_type == 0)
        return (int64_t)kv_dim * 4;
    if (kv_type == 1)
        return (int64_t)kv_dim * 2;
    if (kv_type == 3)
        return (int64_t)((kv_dim + 31) / 32) * 18;
    return (int64_t)((kv_dim + 31) / 32) * 34;
}

/* pkg/engine/kvcache.go:146-180 Write for one layer.  f32: copy; q8_0 /
 * q4_0: QuantizeQ8_0 / QuantizeQ4_0 over the whole kvDim vector.  fp16 (no reference type; the
 * reference's only f32->f16 routine is FP32ToFP16, fp16.go:38-69) stores the
 * truncated halves.  Out-of-range slots are ignored (kvcache.go:147-149).
 * cache is [max_seq][bytes_per_vec]. */
void ref_kv_write(int kv_type, int kv_dim, int max_seq, uint8_t *kcache,
                  uint8_t *vcache, int slot, const float *k, const float *v)
{
    if (slot < 0 || slot >= max_seq)
        return;
    int64_t bpv = ref_bytes_per_vec(kv_type, kv_dim);
    uint8_t *kd = kcache + (int64_t)slot * bpv;
    uint8_t *vd = vcache + (int64_t)slot * bpv;
    if (kv_type == 0) {
        memcpy(kd, k, (size_t)bpv);
        memcpy(vd, v, (size_t)bpv);
    } else if (kv_type == 1) {
        ref_fp32_to_fp16_array(k, (uint16_t *)kd, kv_dim);
        ref_fp32_to_fp16_array(v, (uint16_t *)vd, kv_dim);
    } else if (kv_type == 3) {
        ref_quantize_q4_0(k, kv_dim, kd);
        ref_quantize_q4_0(v, kv_dim, vd);
    } else {
        ref_quantize_q8_0(k, kv_dim, kd);
        ref_quantize_q8_0(v, kv_dim, vd);
    }
}

/* pkg/engine/kvcache.go:183-214 Get, widened to float32 for n tokens:
 * the attention loops read exactly these values. */
void ref_kv_widen(int kv_type, int kv_dim, const uint8_t *src, int64_t n_tok,
                  float *dst)
{
    int64_t bpv = ref_bytes_per_vec(kv_type, kv_dim);
    for (int64_t t = 0; t < n_tok; t++) {
        const uint8_t *s = src + t * bpv;
        float *d = dst + t * kv_dim;
        if (kv_type == 0)
            memcpy(d, s, (size_t)bpv);
        else if (kv_type == 1)
            ref_fp16_to_fp32_array((const uint16_t *)s, d, kv_dim);
        else if (kv_type == 3)
            ref_dequantize_q4_0(s, kv_dim, d);
        else
            ref_dequantize_q8_0(s, kv_dim, d);
    }
}

/* ---- paged pool in the reference layout ---------------------------------- */

/* pkg/engine/paged_kv.go:13-38 KVBlock: one block holds every layer,
 * Key[layer][token_idx*kvDim].  Here a pool of stored-format bytes laid out
 * [block][layer][token_in_block][bytes_per_vec] for K and V separately.
 * ref_paged_store writes token vectors at (block_id, slot) for one layer,
 * ref_paged_gather materialises logical tokens [0, n_tok) of one layer from a
 * block table into the contiguous [n_tok][bytes_per_vec] layout that
 * KVCache indexes (token t -> block_table[t/bs], slot t%bs). */
void ref_paged_store(int kv_type, int num_layers, int block_size, int kv_dim,
                     uint8_t *kpool, uint8_t *vpool, int layer, int n_tok,
                     const int32_t *block_ids, const int32_t *slots,
                     const float *k, const float *v)
{
    int64_t bpv = ref_bytes_per_vec(kv_type, kv_dim);
    for (int i = 0; i < n_tok; i++) {
        int64_t off = (((int64_t)block_ids[i] * num_layers + layer) * block_size + slots[i]) * bpv;
        ref_kv_write(kv_type, kv_dim, 1, kpool + off, vpool + off, 0,
                     k + (int64_t)i * kv_dim, v + (int64_t)i * kv_dim);
    }
}

void ref_paged_gather(int kv_type, int num_layers, int block_size, int kv_dim,
                      const uint8_t *kpool, const uint8_t *vpool, int layer,
                      const int32_t *block_table, int n_tok, uint8_t *kout,
                      uint8_t *vout)
{
    int64_t bpv = ref_bytes_per_vec(kv_type, kv_dim);
    for (int t = 0; t < n_tok; t++) {
        int64_t off = (((int64_t)block_table[t / block_size] * num_layers + layer) * block_size + t % block_size) * bpv;
        memcpy(kout + (int64_t)t * bpv, kpool + off, (size_t)bpv);
        memcpy(vout + (int64_t)t * bpv, vpool + off, (size_t)bpv);
    }
}

/* Decode attention for a batch of sequences whose caches are stored-format
 * contiguous [L_b][bytes_per_vec] arrays concatenated in kcat/vcat (token
 * offsets tok_off[b]).  Widens per a8/a7 then runs ref_attention_decode.
 * Used as the CPU baseline of the decode step.  wk/wv must hold
 * max(L)*kv_dim floats, scores max(L). */
void ref_decode_batch(int kv_type, const float *q, const uint8_t *kcat,
                      const uint8_t *vcat, const int64_t *tok_off,
                      const int32_t *seq_lens, int batch, float *out, int H,
                      int KVH, int hd, float scale, float *wk, float *wv,
                      float *scores)
{
    int kv_dim = KVH * hd;
    int64_t bpv = ref_bytes_per_vec(kv_type, kv_dim);
    for (int b = 0; b < batch; b++) {
        int L = seq_lens[b];
        ref_kv_widen(kv_type, kv_dim, kcat + tok_off[b] * bpv, L, wk);
        ref_kv_widen(kv_type, kv_dim, vcat + tok_off[b] * bpv, L, wv);
        ref_attention_decode(q + (int64_t)b * H * hd, wk, wv,
                             out + (int64_t)b * H * hd, H, KVH, hd, L, scale,
                             scores);
    }
}

/* ---- the same loops on several host threads ------------------------------ */

/* Work is split by (query, q-head) row, the split the reference's threaded
 * attention uses (pkg/engine/forward.go:1342-1378 hands heads to
 * goroutines).  Every row is computed by attend_head exactly as in the
 * one-thread functions above, so the results are bit-identical to theirs;
 * only the order in which rows finish differs.  Return 0, or -1 when a
 * thread or a buffer cannot be had. */

struct mt_job {
    const float *q, *kc, *vc;
    float *out;
    int H, KVH, hd, start, chunk, max_seq;
    float scale;
    int next; /* next row, taken with an atomic add */
    int failed;
};

static void *mt_prefill_worker(void *arg)
{
    struct mt_job *j = (struct mt_job *)arg;
    int kv_dim = j->KVH * j->hd, kv_mul = j->H / j->KVH;
    int cap = j->start + j->chunk < j->max_seq ? j->start + j->chunk : j->max_seq;
    float *scores = (float *)malloc(sizeof(float) * (size_t)(cap > 0 ? cap : 1));
    if (!scores) {
        __atomic_store_n(&j->failed, 1, __ATOMIC_RELAXED);
        return NULL;
    }
    const int rows = j->chunk * j->H;
    for (;;) {
        int r = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
        if (r >= rows)
            break;
        int b = r / j->H, h = r % j->H;
        int active = j->start + b + 1;
        if (active > j->max_seq)
            active = j->max_seq;
        int64_t off = ((int64_t)b * j->H + h) * j->hd;
        attend_head(j->q + off, j->kc, j->vc, j->out + off, h / kv_mul, kv_dim, j->hd, active,
                    j->scale, scores);
    }
    free(scores);
    return NULL;
}

static int run_threads(void *(*fn)(void *), void *arg, int nthreads)
{
    if (nthreads < 1)
        nthreads = 1;
    pthread_t *t = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    if (!t)
        return -1;
    int started = 0, rc = 0;
    for (; started < nthreads - 1; started++)
        if (pthread_create(&t[started], NULL, fn, arg) != 0) {
            rc = -1;
            break;
        }
    fn(arg); /* the calling thread works too */
    for (int i = 0; i < started; i++)
        pthread_join(t[i], NULL);
    free(t);
    return rc;
}

/* ref_attention_prefill on nthreads threads (rows taken dynamically, since
 * causal rows differ in length). */
int ref_attention_prefill_mt(const float *q, const float *kc, const float *vc,
                             float *out, int H, int KVH, int hd, int start_pos,
                             int chunk, int max_seq, float scale, int nthreads)
{
    struct mt_job j = {q, kc, vc, out, H, KVH, hd, start_pos, chunk, max_seq, scale, 0, 0};
    int rc = run_threads(mt_prefill_worker, &j, nthreads);
    return rc || j.failed ? -1 : 0;
}

/* ref_attention_decode on nthreads threads: one query at position L-1. */
int ref_attention_decode_mt(const float *q, const float *kc, const float *vc,
                            float *out, int H, int KVH, int hd, int L,
                            float scale, int nthreads)
{
    return ref_attention_prefill_mt(q, kc, vc, out, H, KVH, hd, L - 1, 1, L, scale, nthreads);
}

struct mt_batch {
    int kv_type, batch, H, KVH, hd, nthreads;
    const float *q;
    const uint8_t *kcat, *vcat;
    const int64_t *tok_off;
    const int32_t *seq_lens;
    float *out, *wk, *wv, scale;
    pthread_mutex_t mu;
    pthread_cond_t go;
    int ready; /* set once every thread that will run has started */
    pthread_barrier_t bar;
    int next_tid;
    int failed;
};

static void *mt_batch_worker(void *arg)
{
    struct mt_batch *j = (struct mt_batch *)arg;
    pthread_mutex_lock(&j->mu);
    while (!j->ready)
        pthread_cond_wait(&j->go, &j->mu);
    pthread_mutex_unlock(&j->mu);
    const int tid = __atomic_fetch_add(&j->next_tid, 1, __ATOMIC_RELAXED);
    const int n = j->nthreads, kv_dim = j->KVH * j->hd, kv_mul = j->H / j->KVH;
    const int64_t bpv = ref_bytes_per_vec(j->kv_type, kv_dim);
    int lmax = 1;
    for (int b = 0; b < j->batch; b++)
        if (j->seq_lens[b] > lmax)
            lmax = j->seq_lens[b];
    float *scores = (float *)malloc(sizeof(float) * (size_t)lmax);
    if (!scores)
        __atomic_store_n(&j->failed, 1, __ATOMIC_RELAXED);
    for (int b = 0; b < j->batch; b++) {
        const int L = j->seq_lens[b];
        /* widen this thread's share of the sequence's tokens */
        const int64_t t0 = (int64_t)L * tid / n, t1 = (int64_t)L * (tid + 1) / n;
        ref_kv_widen(j->kv_type, kv_dim, j->kcat + (j->tok_off[b] + t0) * bpv, t1 - t0,
                     j->wk + t0 * kv_dim);
        ref_kv_widen(j->kv_type, kv_dim, j->vcat + (j->tok_off[b] + t0) * bpv, t1 - t0,
                     j->wv + t0 * kv_dim);
        pthread_barrier_wait(&j->bar);
        for (int h = tid; scores && h < j->H; h += n) {
            int64_t off = ((int64_t)b * j->H + h) * j->hd;
            attend_head(j->q + off, j->wk, j->wv, j->out + off, h / kv_mul, kv_dim, j->hd, L,
                        j->scale, scores);
        }
        /* every row of this sequence is done before its buffers are reused */
        pthread_barrier_wait(&j->bar);
    }
    free(scores);
    return NULL;
}

/* ref_decode_batch on up to nthreads threads: each sequence is widened by
 * all threads (a share of its tokens each), then its q-heads are split over
 * them.  wk/wv must hold max(L)*kv_dim floats.  Returns the number of
 * threads that ran (fewer than asked if some could not be started), or -1. */
int ref_decode_batch_mt(int kv_type, const float *q, const uint8_t *kcat,
                        const uint8_t *vcat, const int64_t *tok_off,
                        const int32_t *seq_lens, int batch, float *out, int H,
                        int KVH, int hd, float scale, float *wk, float *wv,
                        int nthreads)
{
    if (nthreads < 1)
        nthreads = 1;
    struct mt_batch j;
    memset(&j, 0, sizeof j);
    j.kv_type = kv_type;
    j.batch = batch;
    j.H = H;
    j.KVH = KVH;
    j.hd = hd;
    j.q = q;
    j.kcat = kcat;
    j.vcat = vcat;
    j.tok_off = tok_off;
    j.seq_lens = seq_lens;
    j.out = out;
    j.wk = wk;
    j.wv = wv;
    j.scale = scale;
    pthread_t *t = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    if (!t)
        return -1;
    pthread_mutex_init(&j.mu, NULL);
    pthread_cond_init(&j.go, NULL);
    /* threads wait at the gate until the barrier is sized for those that
     * actually started */
    int started = 0;
    for (; started < nthreads - 1; started++)
        if (pthread_create(&t[started], NULL, mt_batch_worker, &j) != 0)
            break;
    j.nthreads = started + 1;
    int rc = pthread_barrier_init(&j.bar, NULL, (unsigned)j.nthreads) == 0 ? 0 : -1;
    if (rc) {
        /* the workers still pass the gate; with no sequences they only
         * allocate and exit */
        j.batch = 0;
    }
    pthread_mutex_lock(&j.mu);
    j.ready = 1;
    pthread_cond_broadcast(&j.go);
    pthread_mutex_unlock(&j.mu);
    mt_batch_worker(&j);
    for (int k = 0; k < started; k++)
        pthread_join(t[k], NULL);
    free(t);
    if (rc == 0)
        pthread_barrier_destroy(&j.bar);
    pthread_cond_destroy(&j.go);
    pthread_mutex_destroy(&j.mu);
    return rc || j.failed ? -1 : j.nthreads;
}

/* ---- rotary position embedding ------------------------------------------- */

/* pkg/math/kernels.go:22-35 ApplyRoPE: for i < half = head_dim/2,
 * freq = 1 / theta^(2i/head_dim) and angle = pos*freq in float64, cos and sin
 * rounded to float32, then the pair (vec[i], vec[i+half]) is rotated in
 * float32 with each product rounded before the sum (no fused multiply-add). */
void ref_apply_rope(float *vec, int pos, int head_dim, float theta)
{
    int half = head_dim / 2;
    for (int i = 0; i < half; i++) {
        double freq = 1.0 / pow((double)theta, (double)(2 * i) / (double)head_dim);
        double val = (double)pos * freq;
        float c = (float)cos(val);
        float s = (float)sin(val);
        float v0 = vec[i];
        float v1 = vec[i + half];
        vec[i] = v0 * c - v1 * s;
        vec[i + half] = v0 * s + v1 * c;
    }
}

/* RoPE of every head of a [n_heads][head_dim] vector, as Forward applies it
 * per q head and per kv head (pkg/engine/forward.go:228-234, 527-539).  With
 * rope_dim < head_dim only the first rope_dim dims of each head turn, at
 * frequencies of rope_dim (ApplyRoPE(head[:ropeDim], pos, ropeDim, theta),
 * forward.go:945-977). */
void ref_rope_heads(float *x, int n_heads, int head_dim, int rope_dim, int pos, float theta)
{
    if (rope_dim <= 0 || rope_dim > head_dim)
        rope_dim = head_dim;
    for (int h = 0; h < n_heads; h++)
        ref_apply_rope(x + (int64_t)h * head_dim, pos, rope_dim, theta);
}

/* The float32 (cos, sin) pairs ApplyRoPE uses at positions [pos0, pos0+n_pos)
 * for rope_dim: out[(p - pos0) * (rope_dim/2) + i] = {cos, sin}. */
void ref_rope_table(float theta, int rope_dim, int pos0, int n_pos, float *out)
{
    int half = rope_dim / 2;
    for (int p = 0; p < n_pos; p++) {
        for (int i = 0; i < half; i++) {
            double freq = 1.0 / pow((double)theta, (double)(2 * i) / (double)rope_dim);
            double val = (double)(pos0 + p) * freq;
            out[2 * ((int64_t)p * half + i)] = (float)cos(val);
            out[2 * ((int64_t)p * half + i) + 1] = (float)sin(val);
        }
    }
}

/* ---- weight matrix times activations (the O-projection after attention) -- */

/* pkg/quant/quant.go:569-577 DotVecF16: sequential float32 sum of
 * x[i] * FP16ToFP32(w[i]). */
float ref_dot_vec_f16(const float *x, const uint16_t *w, int n)
{
    float sum = 0.0f;
    for (int i = 0; i < n; i++)
        sum += x[i] * ref_fp16_to_fp32(w[i]);
    return sum;
}

/* quant.go:320-339 DotVecQ8_0: per block of 32, blockSum += float32(q) * x in
 * order, then total += blockSum * d. */
float ref_dot_vec_q8_0(const float *x, const uint8_t *blocks, int n)
{
    float total = 0.0f;
    for (int b = 0; b < n / 32; b++) {
        const uint8_t *blk = blocks + (int64_t)b * 34;
        float d = ref_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8)));
        float bs = 0.0f;
        for (int j = 0; j < 32; j++)
            bs += (float)(int8_t)blk[2 + j] * x[b * 32 + j];
        total += bs * d;
    }
    return total;
}

/* quant.go:294-317 DotVecQ4_0: per block, blockSum += v0*x[j] + v1*x[j+16]
 * for byte j (v0 low nibble - 8, v1 high nibble - 8), then total +=
 * blockSum * d. */
float ref_dot_vec_q4_0(const float *x, const uint8_t *blocks, int n)
{
    float total = 0.0f;
    for (int b = 0; b < n / 32; b++) {
        const uint8_t *blk = blocks + (int64_t)b * 18;
        float d = ref_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8)));
        float bs = 0.0f;
        for (int j = 0; j < 16; j++) {
            float v0 = (float)((int)(blk[2 + j] & 0x0F) - 8);
            float v1 = (float)((int)((blk[2 + j] >> 4) & 0x0F) - 8);
            bs += v0 * x[b * 32 + j] + v1 * x[b * 32 + j + 16];
        }
        total += bs * d;
    }
    return total;
}

/* Bytes of one weight row of a GGML type (0 F32, 1 F16, 2 Q4_0, 8 Q8_0;
 * pkg/gguf/types.go:25-31), 0 for other types. */
int64_t ref_weight_row_bytes(int ggml_type, int cols)
{
    switch (ggml_type) {
    case 0: return (int64_t)cols * 4;
    case 1: return (int64_t)cols * 2;
    case 2: return (int64_t)(cols / 32) * 18;
    case 8: return (int64_t)(cols / 32) * 34;
    }
    return 0;
}

/* pkg/math/gemv.go:27-59 (MatMulF32), 62-96 (Q4_0), 98-132 (Q8_0), 206-240
 * (F16): y[r] = DotVec<type>(x, row r of w), for each of batch rows of x
 * (the batch of metal.MatMulBatch, pkg/metal/metal_darwin.go:849-880, is a
 * row-by-row repetition of the GEMV).  x [batch][cols], y [batch][rows]. */
void ref_matmul(int ggml_type, int batch, int rows, int cols, const uint8_t *w, const float *x,
                float *y)
{
    int64_t rb = ref_weight_row_bytes(ggml_type, cols);
    for (int b = 0; b < batch; b++) {
        const float *xb = x + (int64_t)b * cols;
        for (int r = 0; r < rows; r++) {
            const uint8_t *wr = w + (int64_t)r * rb;
            float v = 0.0f;
            switch (ggml_type) {
            case 0: v = ref_dot_vec_f32(xb, (const float *)wr, cols); break;
            case 1: v = ref_dot_vec_f16(xb, (const uint16_t *)wr, cols); break;
            case 2: v = ref_dot_vec_q4_0(xb, wr, cols); break;
            case 8: v = ref_dot_vec_q8_0(xb, wr, cols); break;
            }
            y[(int64_t)b * rows + r] = v;
        }
    }
}
