// Chunked-prefill causal attention on the matrix cores (fp16, q8_0, q4_0 and f32 pages).
//
// Semantics: pkg/engine/forward.go:547-577 -- the chunk's K/V are already in
// the pages; query i of sequence b sits at position start_pos[b] + i and
// attends tokens [0, start_pos[b] + i + 1).
//
// Layout of the work follows the decode kernel (decode_mfma.hip): a wave
// computes S^T = K Q^T on 16x16x32 f16 MFMA tiles whose columns are 16
// (query, head) pairs of one kv head -- 16/G queries x G heads -- and feeds
// P back as the A operand of O += P V without moving it between lanes.  Each
// wave owns its columns for the whole context (no cross-wave merge); the four
// waves of a workgroup take consecutive column groups, so they stream the same
// K/V blocks and share them through the caches.  Query and P are split into
// fp16 hi + lo halves, so results keep float32 accuracy.  The LDS-staged
// kernels share one block of K and V among the waves of a workgroup; the
// ping-pong kernels (attn_prefill_pp, attn_prefill_ppq) put two waves on
// every SIMD that alternate between products and softmax.
//
// q8_0 pages stay exact: int8 values are exact in fp16 (converted with a
// byte permute: 0x64XX is 1024 + XX).  The LDS-staged kernel turns value x
// scale into exact hi + lo half pairs; the direct kernel multiplies each
// 32-wide k-step's partial scores by its K block scale and folds the V block
// scale of each 32 dimensions into P for the products of those dimensions.
#include "gi_common.h"
#include "gi_kernels.h"
#include "mfma_ops.h"

#include <math.h>
#include <type_traits>

namespace gi {

namespace mfma_prefill {

using mfma_ops::f4;
using mfma_ops::h2;
using mfma_ops::h8;
using mfma_ops::i8x8_to_h8;
using mfma_ops::u2;
using mfma_ops::u4;
using mfma_ops::split_pair;
using mfma_ops::u4x8_to_h8;

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float maxnum(float a, float b) { return __builtin_elementwise_maximumnum(a, b); }
__device__ __forceinline__ float maxnum3(float a, float b, float c) { return maxnum(maxnum(a, b), c); }
// Maximum over lanes l, l ^ 16 and l ^ 32 partners, as mfma_ops::max_xor16 /
// max_xor32, with maximumNumber.
__device__ __forceinline__ float max_xor16n(float x)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return maxnum(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}
__device__ __forceinline__ float max_xor32n(float x)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return maxnum(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}

__device__ __forceinline__ f4 mfma(h8 a, h8 b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h8 ld16(const uint8_t *p)
{
    return __builtin_nontemporal_load(reinterpret_cast<const h8 *>(p));
}

__device__ __forceinline__ void split_hilo(float x, _Float16 &hi, _Float16 &lo)
{
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// Eight values x = hi + lo, hi and lo fp16.  hi comes from one packed
// round-toward-zero conversion per pair, so the register the MFMA reads is
// the very value lo was computed against (with floating-point contraction a
// plain (_Float16)x can be evaluated twice with different roundings when x is
// a product, and the halves then no longer sum to x).
// neg1 is -1 (mfma_ops::opaque_neg1), so that each remainder x - hi is one
// mixed-precision multiply-add reading hi in place.
__device__ __forceinline__ void split8(const float *x, h8 &hi, h8 &lo, float neg1)
{
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const h2 h = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(x[2 * k], x[2 * k + 1]));
        hi[2 * k] = h[0];
        hi[2 * k + 1] = h[1];
        lo[2 * k] = (_Float16)fmaf((float)h[0], neg1, x[2 * k]);
        lo[2 * k + 1] = (_Float16)fmaf((float)h[1], neg1, x[2 * k + 1]);
    }
}

template <int HD, int KT, int NCG>
__global__ __launch_bounds__(256) void attn_prefill(PrefillArgs a)
{
    constexpr int KK = HD / 32, NB = HD / 16;
    const PoolLayout &L = a.L;
    const int kvh = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int H = a.num_heads, G = H / L.num_kv_heads, P = L.page_tokens;
    const int start = a.start_pos[b];
    const int chunk = a.chunk_len;
    const int32_t *bt = a.block_tables + (int64_t)b * a.max_blocks;
    const int mapped = a.max_blocks * P; // tokens the block table covers

    // Columns of group cg of this wave: global column c -> query c / G,
    // head kvh*G + c % G.
    int col0[NCG];
    int qlen[NCG];      // tokens this lane's column attends (>= 1)
    bool qvalid[NCG];
    int wave_len = 0;   // tokens any column of this wave attends
#pragma unroll
    for (int cg = 0; cg < NCG; cg++) {
        col0[cg] = ((blockIdx.x * 4 + w) * NCG + cg) * 16;
        const int qi = (col0[cg] + j) / G;
        qvalid[cg] = qi < chunk;
        int len = start + min(qi, chunk - 1) + 1;
        if (len > mapped) {
            if (j == 0 && g == 0 && a.status)
                atomicOr(a.status, FLAG_BAD_SLOT);
            len = mapped;
        }
        qlen[cg] = len;
        const int last = (col0[cg] + 15) / G;
        int wl = start + min(last, chunk - 1) + 1;
        wave_len = max(wave_len, min(wl, mapped));
    }
    if (col0[0] / G >= chunk)
        return; // wave entirely past the chunk (uniform per wave)

    // Q^T operands, hi and lo: column j of group cg, k-slot (g, v) of step kk
    // is dimension 32*kk + 8*g + v.  Each column is scaled by 2^qe (qe from
    // its largest |q|) so both halves stay normal fp16; the scores are
    // scaled back through c2s.
    h8 qh[NCG][KK], ql[NCG][KK];
    float c2s[NCG];
#pragma unroll
    for (int cg = 0; cg < NCG; cg++) {
        const int c = col0[cg] + j;
        const int qi = min(c / G, chunk - 1);
        const float *qp = a.q + (((int64_t)b * chunk + qi) * H + kvh * G + c % G) * HD;
        float qv[KK][8];
        float mq = 0.0f;
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
#pragma unroll
            for (int v = 0; v < 8; v++) {
                qv[kk][v] = qp[32 * kk + 8 * g + v];
                mq = fmaxf(mq, fabsf(qv[kk][v]));
            }
        mq = fmaxf(mq, __shfl_xor(mq, 16));
        mq = fmaxf(mq, __shfl_xor(mq, 32));
        const int qe = pow2_exponent_for(mq);
        const float up = ldexpf(1.0f, qe);
        c2s[cg] = a.scale * kLog2e * ldexpf(1.0f, -qe);
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
#pragma unroll
            for (int v = 0; v < 8; v++) {
                _Float16 hi, lo;
                split_hilo(qv[kk][v] * up, hi, lo);
                qh[cg][kk][v] = hi;
                ql[cg][kk][v] = lo;
            }
    }

    // q8_0: P is multiplied by V-block scale / vnorm[db], where vnorm is a
    // running power of two >= every V scale seen for that dimension block, so
    // the folded probabilities stay within [0, 2^14] and their hi/lo halves
    // stay normal fp16; the accumulators hold O / vnorm and are rescaled
    // exactly when it grows.
    float vnorm[HD / 32];
#pragma unroll
    for (int db = 0; db < HD / 32; db++)
        vnorm[db] = 0.0f;
    float m2[NCG], lsum[NCG];
    f4 o[NCG][NB];
#pragma unroll
    for (int cg = 0; cg < NCG; cg++) {
        m2[cg] = -INFINITY;
        lsum[cg] = 0.0f;
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
            o[cg][nb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    const int eb = KT == KV_F16 ? 2 : 1; // bytes per stored element
    const int64_t koff = L.k_off + (int64_t)kvh * P * HD * eb;
    const int64_t voff = L.v_off + (int64_t)kvh * HD * P * eb;
    const int64_t ksoff = L.ks_off + (int64_t)kvh * P * (HD / 32) * 2;
    const int64_t vsoff = L.vs_off + (int64_t)kvh * (HD / 32) * P * 2;
    const int tk0 = 8 * (j >> 2) + (j & 3), tk1 = tk0 + 4; // K rows of tiles 0/1

    for (int base = 0; base < wave_len; base += 32) {
        int64_t pA = bt[base / P];
        int64_t pB = base + 16 < wave_len ? (int64_t)bt[(base + 16) / P] : pA;
        bool ok = pA >= 0 && pA < L.num_pages && pB >= 0 && pB < L.num_pages;
        if (!ok) {
            if (j == 0 && g == 0 && a.status)
                atomicOr(a.status, FLAG_BAD_PAGE);
            if (!(pA >= 0 && pA < L.num_pages))
                pA = 0;
            if (!(pB >= 0 && pB < L.num_pages))
                pB = 0;
        }
        const uint8_t *gA = a.base + pA * L.page_bytes, *gB = a.base + pB * L.page_bytes;
        const uint8_t *g0 = tk0 < 16 ? gA : gB, *g1 = tk1 < 16 ? gA : gB, *gv = g < 2 ? gA : gB;
        const int s0 = (base + tk0) % P, s1 = (base + tk1) % P, sv = (base + 8 * g) % P;

        // ---- K tiles ----
        h8 k0[KK], k1[KK];
        float ksc0[KK][4], ksc1[KK][4]; // q8_0: scale of (row token, k-step)
#pragma unroll
        for (int kk = 0; kk < KK; kk++) {
            if (KT == KV_F16) {
                k0[kk] = ld16(g0 + koff + ((int64_t)s0 * HD + 32 * kk + 8 * g) * 2);
                k1[kk] = ld16(g1 + koff + ((int64_t)s1 * HD + 32 * kk + 8 * g) * 2);
            } else {
                k0[kk] = i8x8_to_h8(*reinterpret_cast<const u2 *>(g0 + koff + (int64_t)s0 * HD + 32 * kk + 8 * g));
                k1[kk] = i8x8_to_h8(*reinterpret_cast<const u2 *>(g1 + koff + (int64_t)s1 * HD + 32 * kk + 8 * g));
            }
        }
        if (KT == KV_Q8_0) {
            // output row 4g + r of tile 0 is token 8g + r, of tile 1 8g + 4 + r
            const uint16_t *ks = reinterpret_cast<const uint16_t *>(gv + ksoff) + (int64_t)sv * (HD / 32);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int kk = 0; kk < KK; kk++) {
                    ksc0[kk][r] = half_bits_to_float(ks[r * (HD / 32) + kk]);
                    ksc1[kk][r] = half_bits_to_float(ks[(4 + r) * (HD / 32) + kk]);
                }
        }
        // ---- V tiles: dimension 16*nb + j, tokens 8g .. 8g+7 ----
        h8 vv[NB];
        float vsc[HD / 32][8]; // q8_0: V scale of (dimension block, token)
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            if (KT == KV_F16)
                vv[nb] = ld16(gv + voff + ((int64_t)(16 * nb + j) * P + sv) * 2);
            else
                vv[nb] = i8x8_to_h8(*reinterpret_cast<const u2 *>(gv + voff + (int64_t)(16 * nb + j) * P + sv));
        }
        if (KT == KV_Q8_0) {
            const uint16_t *vs = reinterpret_cast<const uint16_t *>(gv + vsoff);
#pragma unroll
            for (int db = 0; db < HD / 32; db++)
#pragma unroll
                for (int i = 0; i < 8; i++)
                    vsc[db][i] = half_bits_to_float(vs[(int64_t)db * P + sv + i]);
        }
        if (KT == KV_Q8_0) {
#pragma unroll
            for (int db = 0; db < HD / 32; db++) {
                float mv = vsc[db][0];
#pragma unroll
                for (int i = 1; i < 8; i++)
                    mv = fmaxf(mv, vsc[db][i]);
                mv = fmaxf(mv, __shfl_xor(mv, 16));
                mv = fmaxf(mv, __shfl_xor(mv, 32));
                // smallest power of two >= mv (mv is a widened half: finite
                // or Inf, never NaN)
                uint32_t bits = __builtin_bit_cast(uint32_t, mv);
                if (bits & 0x7FFFFFu)
                    bits = (bits & 0xFF800000u) + 0x800000u;
                const float pw = __builtin_bit_cast(float, bits);
                if (pw > vnorm[db]) { // uniform across the wave
                    const float f = vnorm[db] / pw;
#pragma unroll
                    for (int cg = 0; cg < NCG; cg++)
#pragma unroll
                        for (int h = 0; h < 2; h++)
                            o[cg][2 * db + h] *= f;
                    vnorm[db] = pw;
                }
                const float inv = 1.0f / vnorm[db]; // exact: a power of two
#pragma unroll
                for (int i = 0; i < 8; i++)
                    vsc[db][i] *= inv;
            }
        }
        // tokens past the cached range: V zeroed so 0 * V stays 0
        if (base + 32 > wave_len || !ok) {
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (!(base + 8 * g + i < wave_len && ok))
#pragma unroll
                    for (int nb = 0; nb < NB; nb++)
                        vv[nb][i] = (_Float16)0.0f;
        }

#pragma unroll
        for (int cg = 0; cg < NCG; cg++) {
            // ---- scores ----
            f4 sa = {0.0f, 0.0f, 0.0f, 0.0f}, sb = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                if (KT == KV_F16) {
                    sa = mfma(k0[kk], qh[cg][kk], sa);
                    sa = mfma(k0[kk], ql[cg][kk], sa);
                    sb = mfma(k1[kk], qh[cg][kk], sb);
                    sb = mfma(k1[kk], ql[cg][kk], sb);
                } else {
                    f4 za = {0.0f, 0.0f, 0.0f, 0.0f}, zb = {0.0f, 0.0f, 0.0f, 0.0f};
                    za = mfma(k0[kk], qh[cg][kk], za);
                    za = mfma(k0[kk], ql[cg][kk], za);
                    zb = mfma(k1[kk], qh[cg][kk], zb);
                    zb = mfma(k1[kk], ql[cg][kk], zb);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        sa[r] = fmaf(za[r], ksc0[kk][r], sa[r]);
                        sb[r] = fmaf(zb[r], ksc1[kk][r], sb[r]);
                    }
                }
            }
            // lane: column j, tokens base + 8g + i (i < 8)
            float sc[8];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                sc[r] = sa[r] * c2s[cg];
                sc[4 + r] = sb[r] * c2s[cg];
            }
            const int lim = qlen[cg];
            if (base + 32 > lim || !ok) {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (!(base + 8 * g + i < lim && ok))
                        sc[i] = -INFINITY;
            }
            float mx = sc[0];
#pragma unroll
            for (int i = 1; i < 8; i++)
                mx = fmaxf(mx, sc[i]);
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mnew = fmaxf(m2[cg], mx);
            // A column whose tokens all lie ahead (possible only for a block
            // past its own limit, which it never reaches first) keeps -inf.
            const float alpha = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m2[cg] - mnew);
            m2[cg] = mnew;
            // p carries a factor 2^14 (so its lo half stays a normal fp16);
            // the running sum carries the same factor and it cancels at the end.
            const float msub = mnew - 14.0f;
            float p[8], ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                p[i] = mnew == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[i] - msub);
                ps += p[i];
            }
            lsum[cg] = lsum[cg] * alpha + ps;
            if (__any(alpha != 1.0f)) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float ar = __shfl(alpha, 4 * g + r);
#pragma unroll
                    for (int nb = 0; nb < NB; nb++)
                        o[cg][nb][r] *= ar;
                }
            }
            // ---- P * V ----
            if (KT == KV_F16) {
                h8 ph, pl;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    _Float16 hi, lo;
                    split_hilo(p[i], hi, lo);
                    ph[i] = hi;
                    pl[i] = lo;
                }
#pragma unroll
                for (int nb = 0; nb < NB; nb++) {
                    o[cg][nb] = mfma(ph, vv[nb], o[cg][nb]);
                    o[cg][nb] = mfma(pl, vv[nb], o[cg][nb]);
                }
            } else {
#pragma unroll
                for (int db = 0; db < HD / 32; db++) {
                    float x[8];
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        x[i] = p[i] * vsc[db][i];
                    h8 ph, pl;
                    split8(x, ph, pl, mfma_ops::opaque_neg1());
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        o[cg][2 * db + h] = mfma(ph, vv[2 * db + h], o[cg][2 * db + h]);
                        o[cg][2 * db + h] = mfma(pl, vv[2 * db + h], o[cg][2 * db + h]);
                    }
                }
            }
        }
    }

    // ---- normalise and store: output row 4g + r of group cg is column
    // col0 + 4g + r; its denominator lives in lane 4g + r ----
#pragma unroll
    for (int cg = 0; cg < NCG; cg++) {
        float lt = lsum[cg];
        lt += __shfl_xor(lt, 16);
        lt += __shfl_xor(lt, 32);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float l = __shfl(lt, 4 * g + r);
            const int c = col0[cg] + 4 * g + r;
            const int qi = c / G;
            if (qi >= chunk)
                continue;
            float *op = a.out + (((int64_t)b * chunk + qi) * H + kvh * G + c % G) * HD;
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                float x = o[cg][nb][r];
                if (KT == KV_Q8_0)
                    x *= vnorm[nb / 2];
                op[16 * nb + j] = x * inv;
            }
        }
    }
    (void)qvalid;
}


// ---------------------------------------------------------------------------
// LDS-staged form (pages of 16, 32 or 64 tokens).  A workgroup owns 4 x 16 x
// NCG (query, head) columns of one kv head -- NCG groups of 16 per wave, so
// each operand read from LDS feeds 2 NCG (q8_0: 3 NCG) products -- and streams
// the context in 64-token blocks through LDS: all 256 threads load a block with one 16-byte global
// load per chunk, convert it, and store it; every wave then reads its MFMA
// operands from LDS.  The next block's global loads are in flight while the
// current block is computed.
//
// Page ids come from one block-table load per lane (lane l: token l of a
// block), issued a block ahead; each chunk of a wave lies inside one page, so
// its page id is read out of that register as a wave-uniform value.  A 64-bit
// ballot of the same register marks the block's tokens that are cached and on
// a valid page.
//
// q8_0 K and V are dequantised while staging into exact pairs of fp16
// halves: hi = fp16(q * s) and lo = fma(q, s, -hi), whose exact value fits a
// half because q * s has at most 19 significant bits.  Q K^T and P V then take
// three products each (hi x hi, lo x hi, hi x lo).
constexpr int kTB = 64; // tokens per staged block
// Online softmax: p = 2^(score - m + kPExp) with the reference maximum m
// lagging the true one by at most kLazy, so p <= 2^14 stays well inside fp16.
constexpr float kPExp = 6.0f, kLazy = 8.0f;

template <int HD, int KT, int NW = 4>
struct StageRegs {
    // 16-byte chunks per thread and block (NW waves stage it): f32 K rows /
    // V columns of 4 elements, fp16 of 8, int8 K rows / V columns of 16
    // elements, or q4_0 K rows of 32 nibbles (one quantisation block) / V
    // byte rows of 16 tokens (two dimensions each).
    // The chunks of K (and as many of V) are spread over ST threads, the
    // first ST of the workgroup (at most four waves, f32 pages every wave);
    // the others stage nothing.  With 8 waves, four staging q8_0 blocks at two chunks each
    // measured 381 against 369 TFLOP/s for all eight at one (two staging
    // waves at four chunks each spill).
    static constexpr bool QUANT = KT == KV_Q8_0 || KT == KV_Q4_0;
    static constexpr int CH = kTB * HD / (KT == KV_F32 ? 4 : KT == KV_F16 ? 8 : KT == KV_Q8_0 ? 16 : 32);
    static constexpr int SMAX = KT == KV_F32 ? 64 * NW : 256;
    static constexpr int ST = CH < SMAX ? CH : SMAX;
    static constexpr int NC = CH / ST;
    static_assert(ST % 64 == 0 && NC * ST == CH, "whole waves stage whole blocks");
    u4 k[NC], v[NC];
    int64_t kpage[QUANT ? NC : 1]; // quantised pages: page of each chunk (wave-uniform)
    int64_t vpage[QUANT ? NC : 1];
};

// Swizzled geometry of one staged block in LDS, shared by both staged
// kernels.  K: segments of 512/HD token rows (1 KiB, rows unpadded inside),
// each followed by 4096/HD bytes of padding, the low two bits of a row's
// 16-byte chunk index XORed with row % 4; V: [dimension][kTB] halves with the
// 16-byte chunk index XORed with dimension % 8.  The MFMA operand reads of a
// quarter-wave then fall on distinct banks.
template <int HD>
struct SwzGeom {
    static constexpr int KROWS = 512 / HD;             // K rows per segment
    static constexpr int KSEGB = 1024 + 4096 / HD;     // bytes per K segment, padded
    static constexpr int KBYTES = kTB / KROWS * KSEGB; // bytes of one K plane
    static constexpr int VBYTES = HD * kTB * 2;        // bytes of one V plane
    // byte offsets of chunk c (8 halves) of K row `row` / of V dimension `dim`
    __device__ static int koff(int row, int c) { return row / KROWS * KSEGB + row % KROWS * HD * 2 + 16 * (c ^ (row & 3)); }
    __device__ static int voff(int dim, int c) { return (dim * kTB + 8 * (c ^ (dim & 7))) * 2; }
    // byte offsets of element `col` of K row `row` / token `t` of V dimension `dim`
    __device__ static int kel(int row, int col) { return koff(row, col >> 3) + (col & 7) * 2; }
    __device__ static int vel(int dim, int t) { return voff(dim, t >> 3) + (t & 7) * 2; }
};

// Quantised and f32 K and V are stored as hi + lo fp16 pairs (exact for
// quantised pages, 2^-23 relative for f32 ones), in the swizzled geometry.
// KC (quantised pages): K is stored as its integer codes instead, exact in
// fp16, with the block scales beside them ([token][32-dimension block], fp16
// bits); V keeps its hi + lo planes.
template <int HD, int KT, int NBUF, bool KC = false>
struct Lds {
    static constexpr bool Q8 = KT != KV_F16;
    static constexpr bool KLO = Q8 && !KC;
    using G = SwzGeom<HD>;
    __attribute__((aligned(16))) uint8_t k[NBUF][G::KBYTES];
    __attribute__((aligned(16))) uint8_t v[NBUF][G::VBYTES];
    __attribute__((aligned(16))) uint8_t kl[KLO ? NBUF : 1][KLO ? G::KBYTES : 1]; // K lo
    __attribute__((aligned(16))) uint8_t vl[Q8 ? NBUF : 1][Q8 ? G::VBYTES : 1];   // V lo
    __attribute__((aligned(16))) uint16_t ks[KC ? NBUF : 1][KC ? kTB * (HD / 32) : 1];
};

// Chunk -> (token, column) of K and (page segment, code row, token group)
// of V inside one block.  K chunks hold EK dimensions of one token (f32 4,
// fp16 8, q8_0 16, q4_0 32); V chunks EV tokens of one code row (f32 4,
// fp16 8, quantised 16), a code row being a dimension (f32, fp16, q8_0) or the byte row of
// dimensions 32r' + r'' and 32r' + 16 + r'' (q4_0 row 16r' + r'').
template <int HD, int KT, int P>
struct ChunkMap {
    static constexpr int EK = KT == KV_F32 ? 4 : KT == KV_F16 ? 8 : KT == KV_Q8_0 ? 16 : 32;
    static constexpr int EV = KT == KV_F32 ? 4 : KT == KV_F16 ? 8 : 16;
    static constexpr int VROWS = KT == KV_Q4_0 ? HD / 2 : HD;
    static constexpr int KPR = HD / EK;  // K chunks per token row
    static constexpr int VPD = P / EV;   // V chunks per code row and page
    static constexpr int VPS = VROWS * VPD; // V chunks per page segment
    static_assert(VPS % 64 == 0 && (64 * EK / HD) <= P, "a wave's chunks must share one page");
    __device__ static int k_tok(int ch) { return ch / KPR; }
    __device__ static int k_col(int ch) { return EK * (ch % KPR); }
    __device__ static int v_seg(int ch) { return ch / VPS; }
    __device__ static int v_dim(int ch) { return (ch % VPS) / VPD; } // the code row
    __device__ static int v_tok(int ch) { return EV * ((ch % VPS) % VPD); } // within the page
};

// Page id of token `t` of the context (lane-wise), -1 past the cached range.
template <int P>
__device__ __forceinline__ int table_entry(const int32_t *bt, int t, int wg_len)
{
    return t < wg_len ? bt[t / P] : -1;
}

template <int HD, int KT, int P, int NW>
__device__ __forceinline__ void stage_load(const PrefillArgs &a, int kvh, int tid, int w, int tb,
                                           StageRegs<HD, KT, NW> &R)
{
    constexpr int NT = StageRegs<HD, KT, NW>::ST;
    if (NT < 64 * NW && tid >= NT) // wave-uniform
        return;
    using M = ChunkMap<HD, KT, P>;
    const PoolLayout &L = a.L;
    const int64_t np = L.num_pages;
    auto page = [&](int tok) -> int64_t { // wave-uniform
        const int pg = __builtin_amdgcn_readlane(tb, tok);
        return (pg >= 0 && pg < np) ? pg : 0;
    };
#pragma unroll
    for (int c = 0; c < R.NC; c++) {
        const int ch = tid + NT * c, ch0 = 64 * w + NT * c;
        const uint8_t *kp = a.base + page(M::k_tok(ch0)) * L.page_bytes + L.k_off;
        const int tk = M::k_tok(ch);
        const uint8_t *vp = a.base + page(M::v_seg(ch0) * P) * L.page_bytes;
        const int d = M::v_dim(ch), tv = M::v_tok(ch);
        if (KT == KV_F32) {
            R.k[c] = *reinterpret_cast<const u4 *>(kp + (((int64_t)kvh * P + tk % P) * HD + M::k_col(ch)) * 4);
            R.v[c] = *reinterpret_cast<const u4 *>(vp + L.v_off + (((int64_t)kvh * HD + d) * P + tv) * 4);
        } else if (KT == KV_F16) {
            R.k[c] = *reinterpret_cast<const u4 *>(kp + (((int64_t)kvh * P + tk % P) * HD + M::k_col(ch)) * 2);
            R.v[c] = *reinterpret_cast<const u4 *>(vp + L.v_off + (((int64_t)kvh * HD + d) * P + tv) * 2);
        } else if (KT == KV_Q8_0) {
            R.k[c] = *reinterpret_cast<const u4 *>(kp + ((int64_t)kvh * P + tk % P) * HD + M::k_col(ch));
            R.v[c] = *reinterpret_cast<const u4 *>(vp + L.v_off + ((int64_t)kvh * HD + d) * P + tv);
            R.kpage[c] = page(M::k_tok(ch0));
            R.vpage[c] = page(M::v_seg(ch0) * P);
        } else {
            // q4_0: K rows of HD/2 bytes, 16 per block; V byte rows of P bytes
            R.k[c] = *reinterpret_cast<const u4 *>(kp + ((int64_t)kvh * P + tk % P) * (HD / 2) + M::k_col(ch) / 2);
            R.v[c] = *reinterpret_cast<const u4 *>(vp + L.v_off + ((int64_t)kvh * (HD / 2) + d) * P + tv);
            R.kpage[c] = page(M::k_tok(ch0));
            R.vpage[c] = page(M::v_seg(ch0) * P);
        }
    }
}

// q8_0 element pairs: hi = fp16(q * s), lo = fma(q, s, -hi).  q * s has at
// most 19 significant bits, so lo holds the rest exactly and hi + lo == q * s.
__device__ __forceinline__ void dequant_pair(h8 q, h8 s, h8 &hi, h8 &lo)
{
    hi = q * s;
    lo = __builtin_elementwise_fma(q, s, -hi);
}

// Largest |K| and |V| of this thread's f32 chunks of a staged block, over the
// live tokens only (stale slots may hold anything).
template <int HD, int P, int NW>
__device__ __forceinline__ void f32_chunk_max(const StageRegs<HD, KV_F32, NW> &R, int tid, uint64_t vmask, float &mk,
                                              float &mv)
{
    using M = ChunkMap<HD, KV_F32, P>;
    constexpr int ST = StageRegs<HD, KV_F32, NW>::ST;
    mk = 0.0f;
    mv = 0.0f;
    if (ST < 64 * NW && tid >= ST)
        return;
#pragma unroll
    for (int c = 0; c < R.NC; c++) {
        const int ch = tid + ST * c;
        const bool klive = (vmask >> M::k_tok(ch)) & 1u;
        const int t0 = M::v_seg(ch) * P + M::v_tok(ch);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // words copied out first: hipcc's __builtin_bit_cast of an
            // ext_vector element reads element 0 whatever the index
            const uint32_t kw = R.k[c][i], vw = R.v[c][i];
            if (klive)
                mk = fmaxf(mk, fabsf(__builtin_bit_cast(float, kw)));
            if ((vmask >> (t0 + i)) & 1u)
                mv = fmaxf(mv, fabsf(__builtin_bit_cast(float, vw)));
        }
    }
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x)
{
    // (an update of 0 with in-row patterns: folds into the instruction using it)
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Maximum of a non-negative value over the wave, wave-uniform.
__device__ __forceinline__ float wave_max_nonneg(float x)
{
    x = fmaxf(x, dpp_f<0xB1>(x));  // quad_perm [1,0,3,2]
    x = fmaxf(x, dpp_f<0x4E>(x));  // quad_perm [2,3,0,1]
    x = fmaxf(x, dpp_f<0x141>(x)); // row_half_mirror
    x = fmaxf(x, dpp_f<0x140>(x)); // row_mirror
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    const uint32_t m = max(max(__builtin_amdgcn_readlane(b, 0), __builtin_amdgcn_readlane(b, 16)),
                           max(__builtin_amdgcn_readlane(b, 32), __builtin_amdgcn_readlane(b, 48)));
    return __builtin_bit_cast(float, m);
}

// Power-of-two operand scale of a block with largest magnitude m: the
// running scale `run` (0: none yet) is kept while m*run lies in [2^-2,
// 2^15), otherwise m is moved to [2^14, 2^15).
__device__ __forceinline__ float block_scale(float m, float run)
{
    const float r = run == 0.0f ? 1.0f : run;
    const float ms = m * r;
    if (m == 0.0f || (ms >= 0.25f && ms < 32768.0f))
        return r;
    int k = 14 - ((int)((__builtin_bit_cast(uint32_t, m) >> 23) & 0xFF) - 127);
    k = min(max(k, -126), 127);
    return __builtin_bit_cast(float, (uint32_t)(k + 127) << 23);
}

// 1 / x for a power of two x in [2^-126, 2^126].
__device__ __forceinline__ float pow2_recip(float x)
{
    return __builtin_bit_cast(float, 0x7F000000u - __builtin_bit_cast(uint32_t, x));
}

// Converts and stores a staged block.  `vmask` bit l: block token l is cached
// and on a valid page; V of other tokens is stored as zero (their scores are
// masked, and stale values must not reach O through 0 * NaN).
template <int HD, int KT, int P, int NBUF, int NW>
__device__ __forceinline__ void stage_store(const PrefillArgs &a, int kvh, int tid, int w, int buf,
                                            uint64_t vmask, const StageRegs<HD, KT, NW> &R,
                                            Lds<HD, KT, NBUF> &S, float ksc = 1.0f, float vsc = 1.0f, float neg1 = -1.0f)
{
    using M = ChunkMap<HD, KT, P>;
    using G = SwzGeom<HD>;
    // q8_0 block scales: one per K chunk, 16 per V chunk.  Loaded here rather
    // than with the chunk so that they hold no registers through the block's
    // compute (they are shared by many chunks and come from the caches).
    typedef StageRegs<HD, KT, NW> SR;
    constexpr int NT = SR::ST;
    if (NT < 64 * NW && tid >= NT) // wave-uniform
        return;
    constexpr int NCS = SR::QUANT ? SR::NC : 1;
    u4 vs[2 * NCS];
    _Float16 ks[NCS];
    if (SR::QUANT) {
#pragma unroll
        for (int c = 0; c < R.NC; c++) {
            const int ch = tid + NT * c;
            const u4 *sp = reinterpret_cast<const u4 *>(
                a.base + R.vpage[c] * a.L.page_bytes + a.L.vs_off +
                (((int64_t)kvh * (HD / 32) + M::v_dim(ch) / (KT == KV_Q4_0 ? 16 : 32)) * P + M::v_tok(ch)) * 2);
            vs[2 * c] = sp[0];
            vs[2 * c + 1] = sp[1];
            ks[c] = reinterpret_cast<const _Float16 *>(a.base + R.kpage[c] * a.L.page_bytes + a.L.ks_off)
                [((int64_t)kvh * P + M::k_tok(ch) % P) * (HD / 32) + M::k_col(ch) / 32];
        }
    }
#pragma unroll
    for (int c = 0; c < R.NC; c++) {
        const int ch = tid + NT * c;
        const int tk = M::k_tok(ch), col = M::k_col(ch);
        const int d = M::v_dim(ch), t0 = M::v_seg(ch) * P + M::v_tok(ch); // block-local token
        const uint32_t live = (uint32_t)(vmask >> t0) & ((1u << M::EV) - 1u);
        if (KT == KV_F32) {
            // K: 4 dimensions of token tk; V: tokens t0 .. t0+3 of dimension
            // d, dead tokens zeroed (their weights are 0)
            float kx[4], vx[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t kw = R.k[c][i], vw = R.v[c][i]; // (see f32_chunk_max)
                kx[i] = __builtin_bit_cast(float, kw);
                vx[i] = ((live >> i) & 1u) ? __builtin_bit_cast(float, vw) : 0.0f;
            }
            // the scales are workgroup-uniform and 1 for ordinary data
            if (ksc != 1.0f) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    kx[i] *= ksc;
            }
            if (vsc != 1.0f) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    vx[i] *= vsc;
            }
            uint32_t kh[2], kl[2], vh[2], vl[2];
            split_pair(kx[0], kx[1], kh[0], kl[0], neg1);
            split_pair(kx[2], kx[3], kh[1], kl[1], neg1);
            split_pair(vx[0], vx[1], vh[0], vl[0], neg1);
            split_pair(vx[2], vx[3], vh[1], vl[1], neg1);
            *reinterpret_cast<u2 *>(&S.k[buf][G::kel(tk, col)]) = u2{kh[0], kh[1]};
            *reinterpret_cast<u2 *>(&S.kl[buf][G::kel(tk, col)]) = u2{kl[0], kl[1]};
            *reinterpret_cast<u2 *>(&S.v[buf][G::vel(d, t0)]) = u2{vh[0], vh[1]};
            *reinterpret_cast<u2 *>(&S.vl[buf][G::vel(d, t0)]) = u2{vl[0], vl[1]};
        } else if (KT == KV_F16) {
            *reinterpret_cast<u4 *>(&S.k[buf][G::kel(tk, col)]) = R.k[c];
            u4 vv = R.v[c];
            if (live != 0xFFu) {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (!((live >> i) & 1u))
                        vv[i / 2] &= (i & 1) ? 0x0000FFFFu : 0xFFFF0000u;
            }
            *reinterpret_cast<u4 *>(&S.v[buf][G::vel(d, t0)]) = vv;
        } else if (KT == KV_Q4_0) {
            // K: the chunk is one block; low nibbles are dimensions col ..
            // col + 15, high nibbles col + 16 .. col + 31
            const h8 ksp = ks[c]; // splat
#pragma unroll
            for (int m = 0; m < 4; m++) {
                h8 hi, lo;
                const u2 w = u2{R.k[c][2 * (m & 1)], R.k[c][2 * (m & 1) + 1]};
                dequant_pair(u4x8_to_h8(w, 4 * (m >> 1)), ksp, hi, lo);
                *reinterpret_cast<h8 *>(&S.k[buf][G::kel(tk, col + 8 * m)]) = hi;
                *reinterpret_cast<h8 *>(&S.kl[buf][G::kel(tk, col + 8 * m)]) = lo;
            }
            // V: byte row d = 16 db + r holds dimension 32 db + r (low
            // nibble) and 32 db + 16 + r (high nibble) of 16 tokens
            const int dl = 32 * (d >> 4) + (d & 15);
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const u2 w = u2{R.v[c][2 * half], R.v[c][2 * half + 1]};
                const uint32_t lv = live >> (8 * half);
#pragma unroll
                for (int nib = 0; nib < 2; nib++) {
                    h8 hi, lo;
                    dequant_pair(u4x8_to_h8(w, 4 * nib), __builtin_bit_cast(h8, vs[2 * c + half]), hi, lo);
                    if ((lv & 0xFFu) != 0xFFu) {
#pragma unroll
                        for (int i = 0; i < 8; i++)
                            if (!((lv >> i) & 1u)) {
                                hi[i] = (_Float16)0.0f;
                                lo[i] = (_Float16)0.0f;
                            }
                    }
                    *reinterpret_cast<h8 *>(&S.v[buf][G::vel(dl + 16 * nib, t0 + 8 * half)]) = hi;
                    *reinterpret_cast<h8 *>(&S.vl[buf][G::vel(dl + 16 * nib, t0 + 8 * half)]) = lo;
                }
            }
        } else {
            const h8 ksp = ks[c]; // splat
#pragma unroll
            for (int half = 0; half < 2; half++) {
                h8 hi, lo;
                dequant_pair(i8x8_to_h8(u2{R.k[c][2 * half], R.k[c][2 * half + 1]}), ksp, hi, lo);
                *reinterpret_cast<h8 *>(&S.k[buf][G::kel(tk, col + 8 * half)]) = hi;
                *reinterpret_cast<h8 *>(&S.kl[buf][G::kel(tk, col + 8 * half)]) = lo;
            }
#pragma unroll
            for (int half = 0; half < 2; half++) {
                h8 hi, lo;
                dequant_pair(i8x8_to_h8(u2{R.v[c][2 * half], R.v[c][2 * half + 1]}),
                             __builtin_bit_cast(h8, vs[2 * c + half]), hi, lo);
                const uint32_t lv = live >> (8 * half);
                if ((lv & 0xFFu) != 0xFFu) {
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        if (!((lv >> i) & 1u)) {
                            hi[i] = (_Float16)0.0f;
                            lo[i] = (_Float16)0.0f;
                        }
                }
                *reinterpret_cast<h8 *>(&S.v[buf][G::vel(d, t0 + 8 * half)]) = hi;
                *reinterpret_cast<h8 *>(&S.vl[buf][G::vel(d, t0 + 8 * half)]) = lo;
            }
        }
    }
}

// One plane (K or V) of a quantised block staged by the NT = 256 threads of
// one wave group: its chunks (ChunkMap; q8_0 two per thread, q4_0 one) and
// their pages (wave-uniform: a wave's chunks share one page).
template <int HD, int KT>
struct PlaneRegs {
    static constexpr int NT = 256;
    static constexpr int CH = kTB * HD / (KT == KV_Q8_0 ? 16 : 32);
    static constexpr int NC = CH / NT;
    static_assert(NC * NT == CH, "whole chunks per thread");
    u4 x[NC];
    int64_t page[NC];
};

// Loads the K (PLANE 0) or V (PLANE 1) chunks of thread st (0..255) of the
// block whose page ids are in tb (lane l: token l).
template <int PLANE, int HD, int KT, int P>
__device__ __forceinline__ void plane_load(const PrefillArgs &a, int kvh, int st, int tb, PlaneRegs<HD, KT> &R)
{
    using M = ChunkMap<HD, KT, P>;
    constexpr int NT = PlaneRegs<HD, KT>::NT;
    const PoolLayout &L = a.L;
    const int64_t np = L.num_pages;
    auto page = [&](int tok) -> int64_t { // wave-uniform
        const int pg = __builtin_amdgcn_readlane(tb, tok);
        return (pg >= 0 && pg < np) ? pg : 0;
    };
    constexpr int RB = KT == KV_Q4_0 ? HD / 2 : HD; // bytes of a K row / V code rows of a head
#pragma unroll
    for (int c = 0; c < R.NC; c++) {
        const int ch = st + NT * c, ch0 = 64 * (st >> 6) + NT * c;
        if (PLANE == 0) {
            R.page[c] = page(M::k_tok(ch0));
            const uint8_t *kp = a.base + R.page[c] * L.page_bytes + L.k_off;
            R.x[c] = *reinterpret_cast<const u4 *>(kp + ((int64_t)kvh * P + M::k_tok(ch) % P) * RB +
                                                   M::k_col(ch) / (KT == KV_Q4_0 ? 2 : 1));
        } else {
            R.page[c] = page(M::v_seg(ch0) * P);
            const uint8_t *vp = a.base + R.page[c] * L.page_bytes + L.v_off;
            R.x[c] = *reinterpret_cast<const u4 *>(vp + ((int64_t)kvh * (KT == KV_Q4_0 ? HD / 2 : HD) + M::v_dim(ch)) * P +
                                                   M::v_tok(ch));
        }
    }
}

// Block scales of the chunks in PlaneRegs: K, one fp16 scale per chunk (the
// chunk lies in one 32-dimension block of one token); V, the 16 token scales
// of each chunk's dimension block.  Loaded apart from the codes, so that
// their latency passes under other work before plane_store needs them.
template <int HD, int KT>
struct PlaneScales {
    static constexpr int NC = PlaneRegs<HD, KT>::NC;
    uint32_t k[NC];
    u4 v[2 * NC];
};

template <int PLANE, int HD, int KT, int P>
__device__ __forceinline__ void plane_scales(const PrefillArgs &a, int kvh, int st, const PlaneRegs<HD, KT> &R,
                                             PlaneScales<HD, KT> &C)
{
    using M = ChunkMap<HD, KT, P>;
    constexpr int NT = PlaneRegs<HD, KT>::NT;
    const PoolLayout &L = a.L;
#pragma unroll
    for (int c = 0; c < R.NC; c++) {
        const int ch = st + NT * c;
        if (PLANE == 0) {
            const int tk = M::k_tok(ch), col = M::k_col(ch);
            C.k[c] = reinterpret_cast<const uint16_t *>(a.base + R.page[c] * L.page_bytes + L.ks_off)
                [((int64_t)kvh * P + tk % P) * (HD / 32) + col / 32];
        } else {
            const int d = M::v_dim(ch);
            const u4 *sp = reinterpret_cast<const u4 *>(
                a.base + R.page[c] * L.page_bytes + L.vs_off +
                (((int64_t)kvh * (HD / 32) + d / (KT == KV_Q4_0 ? 16 : 32)) * P + M::v_tok(ch)) * 2);
            C.v[2 * c] = sp[0];
            C.v[2 * c + 1] = sp[1];
        }
    }
}

// Dequantises the chunks of plane_load, with the scales plane_scales loaded
// for them, into exact hi + lo fp16 planes of buffer `buf` (the layout
// stage_store writes); V of tokens whose `vmask` bit is clear is stored as
// zero.  KC: K is stored as exact fp16 codes, with its scales in S.ks.
template <int PLANE, int HD, int KT, int P, int NBUF, bool KC>
__device__ __forceinline__ void plane_store(const PrefillArgs &a, int kvh, int st, int buf, uint64_t vmask,
                                            const PlaneRegs<HD, KT> &R, const PlaneScales<HD, KT> &C,
                                            Lds<HD, KT, NBUF, KC> &S)
{
    using M = ChunkMap<HD, KT, P>;
    using G = SwzGeom<HD>;
    constexpr int NT = PlaneRegs<HD, KT>::NT;
    const PoolLayout &L = a.L;
#pragma unroll
    for (int c = 0; c < R.NC; c++) {
        const int ch = st + NT * c;
        if (PLANE == 0) {
            const int tk = M::k_tok(ch), col = M::k_col(ch);
            if (KC) {
                // the codes, and the scale once per 32-dimension block
                if (KT == KV_Q4_0) {
#pragma unroll
                    for (int m = 0; m < 4; m++) {
                        const u2 w = u2{R.x[c][2 * (m & 1)], R.x[c][2 * (m & 1) + 1]};
                        *reinterpret_cast<h8 *>(&S.k[buf][G::kel(tk, col + 8 * m)]) = u4x8_to_h8(w, 4 * (m >> 1));
                    }
                } else {
#pragma unroll
                    for (int half = 0; half < 2; half++)
                        *reinterpret_cast<h8 *>(&S.k[buf][G::kel(tk, col + 8 * half)]) =
                            i8x8_to_h8(u2{R.x[c][2 * half], R.x[c][2 * half + 1]});
                }
                if (col % 32 == 0)
                    S.ks[buf][tk * (HD / 32) + col / 32] = (uint16_t)C.k[c];
                continue;
            }
            const _Float16 kscale = __builtin_bit_cast(_Float16, (uint16_t)C.k[c]);
            const h8 ksp = kscale; // splat
            if (KT == KV_Q4_0) {
                // the chunk is one block: low nibbles are dimensions col ..
                // col + 15, high nibbles col + 16 .. col + 31
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    h8 hi, lo;
                    const u2 w = u2{R.x[c][2 * (m & 1)], R.x[c][2 * (m & 1) + 1]};
                    dequant_pair(u4x8_to_h8(w, 4 * (m >> 1)), ksp, hi, lo);
                    *reinterpret_cast<h8 *>(&S.k[buf][G::kel(tk, col + 8 * m)]) = hi;
                    *reinterpret_cast<h8 *>(&S.kl[buf][G::kel(tk, col + 8 * m)]) = lo;
                }
            } else {
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    h8 hi, lo;
                    dequant_pair(i8x8_to_h8(u2{R.x[c][2 * half], R.x[c][2 * half + 1]}), ksp, hi, lo);
                    *reinterpret_cast<h8 *>(&S.k[buf][G::kel(tk, col + 8 * half)]) = hi;
                    *reinterpret_cast<h8 *>(&S.kl[buf][G::kel(tk, col + 8 * half)]) = lo;
                }
            }
        } else {
            const int d = M::v_dim(ch), t0 = M::v_seg(ch) * P + M::v_tok(ch); // block-local token
            const uint32_t live = (uint32_t)(vmask >> t0) & 0xFFFFu;
            const u4 vs[2] = {C.v[2 * c], C.v[2 * c + 1]};
            // q4_0: byte row d = 16 db + r holds dimension 32 db + r (low
            // nibble) and 32 db + 16 + r (high nibble) of 16 tokens
            const int dl = KT == KV_Q4_0 ? 32 * (d >> 4) + (d & 15) : d;
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const u2 w = u2{R.x[c][2 * half], R.x[c][2 * half + 1]};
                const uint32_t lv = live >> (8 * half);
#pragma unroll
                for (int nib = 0; nib < (KT == KV_Q4_0 ? 2 : 1); nib++) {
                    h8 hi, lo;
                    dequant_pair(KT == KV_Q4_0 ? u4x8_to_h8(w, 4 * nib) : i8x8_to_h8(w),
                                 __builtin_bit_cast(h8, vs[half]), hi, lo);
                    if ((lv & 0xFFu) != 0xFFu) {
#pragma unroll
                        for (int i = 0; i < 8; i++)
                            if (!((lv >> i) & 1u)) {
                                hi[i] = (_Float16)0.0f;
                                lo[i] = (_Float16)0.0f;
                            }
                    }
                    *reinterpret_cast<h8 *>(&S.v[buf][G::vel(dl + 16 * nib, t0 + 8 * half)]) = hi;
                    *reinterpret_cast<h8 *>(&S.vl[buf][G::vel(dl + 16 * nib, t0 + 8 * half)]) = lo;
                }
            }
        }
    }
}

// MFMA operand addresses.  A lane's K operand of tile (h, t) and k-step kk
// is row 32h + 8(j/4) + j%4 + 4t, 16-byte chunk 4kk + g; its V operand of
// half h and output tile nb is dimension 16nb + j, chunk 4h + g.  Each
// layout splits these addresses into a per-lane base, computed once per
// block, and a compile-time offset, so that the reads use immediate offsets.

// Register-staged layout: the swizzled geometry (SwzGeom), hi and lo planes.
template <int HD, int KT, int NBUF, bool KC>
__device__ __forceinline__ const uint8_t *k_lane(const Lds<HD, KT, NBUF, KC> &S, int buf, int j, int g, bool lo)
{
    // row 8(j/4) + j%4 (+ 32h + 4t): segment and row inside it
    using G = SwzGeom<HD>;
    constexpr int KR = G::KROWS;
    const int seg = KR == 4 ? 2 * (j >> 2) : (j >> 2);
    return (lo ? S.kl[buf] : S.k[buf]) + seg * G::KSEGB + (j & 3) * HD * 2 + 16 * (g ^ (j & 3));
}
template <int HD, int KT, int NBUF, bool KC>
__device__ __forceinline__ const uint8_t *v_lane(const Lds<HD, KT, NBUF, KC> &S, int buf, int h, int j, int g,
                                                 bool lo)
{
    return (lo ? S.vl[buf] : S.v[buf]) + (j * kTB + 8 * ((4 * h + g) ^ (j & 7))) * 2;
}
template <int HD, int KT, int NBUF, bool KC>
__device__ constexpr int k_const(const Lds<HD, KT, NBUF, KC> *, int h, int t, int kk)
{
    constexpr int KR = SwzGeom<HD>::KROWS, SB = SwzGeom<HD>::KSEGB;
    return (KR == 4 ? (8 * h + t) * SB : 4 * h * SB + 4 * t * HD * 2) + 64 * kk;
}
template <int HD, int KT, int NBUF, bool KC>
__device__ constexpr int v_const(const Lds<HD, KT, NBUF, KC> *, int nb)
{
    return 16 * nb * kTB * 2;
}

// Layout written by direct global->LDS loads (fp16 pages): the swizzled
// geometry (SwzGeom), whose K segments are exactly what one 1 KiB load
// instruction fills in lane order.
template <int HD>
struct LdsDirect {
    static constexpr int KROWS = SwzGeom<HD>::KROWS, KSEGB = SwzGeom<HD>::KSEGB, KBYTES = SwzGeom<HD>::KBYTES;
    __attribute__((aligned(16))) uint8_t k[2][KBYTES];
    __attribute__((aligned(16))) _Float16 v[2][HD * kTB]; // [dim][kTB], chunk c at c ^ (dim & 7)
    __device__ static int koff(int row, int c) { return SwzGeom<HD>::koff(row, c); }
};
template <int HD>
__device__ __forceinline__ const uint8_t *k_lane(const LdsDirect<HD> &S, int buf, int j, int g, bool)
{
    // row 8(j/4) + j%4 (+ 32h + 4t): segment and row inside it
    constexpr int KR = LdsDirect<HD>::KROWS;
    const int seg = KR == 4 ? 2 * (j >> 2) : (j >> 2);
    return &S.k[buf][seg * LdsDirect<HD>::KSEGB + (j & 3) * HD * 2 + 16 * (g ^ (j & 3))];
}
template <int HD>
__device__ __forceinline__ const uint8_t *v_lane(const LdsDirect<HD> &S, int buf, int h, int j, int g, bool)
{
    return reinterpret_cast<const uint8_t *>(&S.v[buf][j * kTB + 8 * ((4 * h + g) ^ (j & 7))]);
}
template <int HD>
__device__ constexpr int k_const(const LdsDirect<HD> *, int h, int t, int kk)
{
    constexpr int KR = LdsDirect<HD>::KROWS, SB = LdsDirect<HD>::KSEGB;
    return (KR == 4 ? (8 * h + t) * SB : 4 * h * SB + 4 * t * HD * 2) + 64 * kk;
}
template <int HD>
__device__ constexpr int v_const(const LdsDirect<HD> *, int nb)
{
    return 16 * nb * kTB * 2;
}

__device__ __forceinline__ h8 ld_frag(const uint8_t *p, int off)
{
    return *reinterpret_cast<const h8 *>(p + off);
}

// Schedule of a run of NF operand steps, each R reads from LDS feeding M
// products: the reads of the first RA steps, then for each step the reads RA
// steps ahead followed by its products, so that a read has RA steps of
// products to land (the scheduler would otherwise sink every read next to
// its products and wait out the LDS latency each time).
// VM > 0: one global load after the products of every VM-th step (from
// step 0), so that the load instructions, which hold the wave while the
// address unit takes them, issue between products.
template <int NF, int M, int R, int RA, int VM = 0>
__device__ __forceinline__ void read_ahead_order()
{
    __builtin_amdgcn_sched_group_barrier(0x100, RA * R, 0);
#pragma unroll
    for (int f = 0; f < NF; f++) {
        if (f + RA < NF)
            __builtin_amdgcn_sched_group_barrier(0x100, R, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, M, 0);
        if (VM > 0 && f % VM == 0)
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
}

// No extra work between the products of pv_block.
struct NoLoads {
    static constexpr int N = 0;
    __device__ void operator()(int) const {}
};

// Per-wave attention state over NCG column groups of 16 (query, head)
// columns: Q^T operands, running maximum and sum, and the O accumulators.
template <int HD, int KT, int NCG>
struct WaveAttn {
    static constexpr int KK = HD / 32, NB = HD / 16;
    h8 qh[NCG][KK], ql[NCG][KK];
    float c2s[NCG], m2[NCG], lsum[NCG];
    // f32 pages: 1 / the K operand scale of this lane's tokens of half h of
    // the current block (tokens 32h + 8g .. 32h + 8g + 7)
    float kinv[2] = {1.0f, 1.0f};
    // f32 ping-pong kernel: the power-of-two V operand scale that O tiles
    // 2q and 2q + 1 (dimensions 32q .. 32q + 31) are held in
    float vso[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    float neg1;        // -1, opaque to the optimiser (split8)
    f4 o[NCG][NB];
    int qlen[NCG];

    // Loads Q of columns col0 + 16 cg + j, split into hi + lo halves scaled
    // per column by 2^qe.  ONE_PASS: every column group's values are loaded
    // at once and kept in registers (one memory round trip at the kernel's
    // start, where every workgroup reads its Q together); otherwise two
    // passes per group, the second from the caches, so that only 8 values
    // are live at a time next to the split halves.
    template <bool ONE_PASS = false>
    __device__ __forceinline__ void init(const PrefillArgs &a, int b, int kvh, int col0, int start,
                                         int mapped, bool active, int j, int g)
    {
        const int H = a.num_heads, G = H / a.L.num_kv_heads, chunk = a.chunk_len;
        neg1 = mfma_ops::opaque_neg1();
        if (ONE_PASS) {
            f4 xq[NCG][KK][2];
#pragma unroll
            for (int cg = 0; cg < NCG; cg++) {
                const int c = col0 + 16 * cg + j;
                const int qi = min(c / G, chunk - 1);
                qlen[cg] = min(start + qi + 1, mapped);
                const float *qp = a.q + (((int64_t)b * chunk + qi) * H + kvh * G + c % G) * HD;
#pragma unroll
                for (int kk = 0; kk < KK; kk++)
#pragma unroll
                    for (int hv = 0; hv < 2; hv++)
                        xq[cg][kk][hv] = active ? *reinterpret_cast<const f4 *>(qp + 32 * kk + 8 * g + 4 * hv) : f4{};
            }
#pragma unroll
            for (int cg = 0; cg < NCG; cg++) {
                float mq = 0.0f;
#pragma unroll
                for (int kk = 0; kk < KK; kk++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        mq = fmaxf(mq, fmaxf(fabsf(xq[cg][kk][0][v]), fabsf(xq[cg][kk][1][v])));
                mq = fmaxf(mq, __shfl_xor(mq, 16));
                mq = fmaxf(mq, __shfl_xor(mq, 32));
                const int qe = pow2_exponent_for(mq);
                const float up = ldexpf(1.0f, qe);
                c2s[cg] = a.scale * kLog2e * ldexpf(1.0f, -qe);
#pragma unroll
                for (int kk = 0; kk < KK; kk++) {
                    float x[8];
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        x[v] = xq[cg][kk][0][v] * up;
                        x[4 + v] = xq[cg][kk][1][v] * up;
                    }
                    split8(x, qh[cg][kk], ql[cg][kk], neg1);
                }
                m2[cg] = -INFINITY;
                lsum[cg] = 0.0f;
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    o[cg][nb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            return;
        }
#pragma unroll
        for (int cg = 0; cg < NCG; cg++) {
            const int c = col0 + 16 * cg + j;
            const int qi = min(c / G, chunk - 1);
            qlen[cg] = min(start + qi + 1, mapped);
            const float *qp = a.q + (((int64_t)b * chunk + qi) * H + kvh * G + c % G) * HD;
            // two passes over q (the second from the caches), so that only
            // 8 of its values are live at a time next to the split halves
            float mq = 0.0f;
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const f4 x0 = active ? *reinterpret_cast<const f4 *>(qp + 32 * kk + 8 * g) : f4{};
                const f4 x1 = active ? *reinterpret_cast<const f4 *>(qp + 32 * kk + 8 * g + 4) : f4{};
#pragma unroll
                for (int v = 0; v < 4; v++)
                    mq = fmaxf(mq, fmaxf(fabsf(x0[v]), fabsf(x1[v])));
            }
            mq = fmaxf(mq, __shfl_xor(mq, 16));
            mq = fmaxf(mq, __shfl_xor(mq, 32));
            const int qe = pow2_exponent_for(mq);
            const float up = ldexpf(1.0f, qe);
            c2s[cg] = a.scale * kLog2e * ldexpf(1.0f, -qe);
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const f4 x0 = active ? *reinterpret_cast<const f4 *>(qp + 32 * kk + 8 * g) : f4{};
                const f4 x1 = active ? *reinterpret_cast<const f4 *>(qp + 32 * kk + 8 * g + 4) : f4{};
                float x[8];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    x[v] = x0[v] * up;
                    x[4 + v] = x1[v] * up;
                }
                split8(x, qh[cg][kk], ql[cg][kk], neg1);
            }
            m2[cg] = -INFINITY;
            lsum[cg] = 0.0f;
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
                o[cg][nb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }

    // Online softmax of column 16 cg + j over this lane's 16 tokens of a
    // block (sv[8h + v]: token 32h + 8g + v), producing P as fp16 hi + lo per
    // half.  Scores in log2 units are s * c2s (c2s > 0).  The reference
    // maximum m2 is raised only when a block's maximum passes it by more than
    // kLazy, so O and l are rarely rescaled; every p = 2^(s c2s - m2 + kPExp)
    // is at most 2^(kPExp + kLazy).  Returns whether any column of the wave
    // grew, in which case the caller rescales O by `alpha`.
    template <bool FULL>
    __device__ __forceinline__ bool softmax16(int cg, float (&sv)[16], int base, uint64_t mask, h8 &ph0,
                                              h8 &pl0, h8 &ph1, h8 &pl1, float &alpha, int g)
    {
        if (!FULL) {
            const uint32_t lm = (uint32_t)(mask >> (8 * g));
            const uint32_t hm = (uint32_t)(mask >> (32 + 8 * g));
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int tl = 32 * (i / 8) + 8 * g + (i % 8);
                const uint32_t bit = ((i < 8 ? lm : hm) >> (i % 8)) & 1u;
                if (!(bit && base + tl < qlen[cg]))
                    sv[i] = -INFINITY;
            }
        }
        // maximumNumber (IEEE 754-2019) compiles to v_max3_f32 with no
        // canonicalising moves of the product results that fmaxf needs
        float mx;
        if constexpr (KT == KV_F32) {
            // the two halves may carry different K scales
            const float a0 = maxnum3(maxnum3(sv[0], sv[1], sv[2]), maxnum3(sv[3], sv[4], sv[5]), maxnum(sv[6], sv[7]));
            const float a1 =
                maxnum3(maxnum3(sv[8], sv[9], sv[10]), maxnum3(sv[11], sv[12], sv[13]), maxnum(sv[14], sv[15]));
            mx = maxnum(a0 * kinv[0], a1 * kinv[1]);
        } else {
            float m3[5];
#pragma unroll
            for (int i = 0; i < 5; i++)
                m3[i] = maxnum3(sv[3 * i], sv[3 * i + 1], sv[3 * i + 2]);
            mx = maxnum3(maxnum3(m3[0], m3[1], m3[2]), maxnum3(m3[3], m3[4], sv[15]), sv[15]);
        }
        mx = max_xor32n(max_xor16n(mx));
        mx *= c2s[cg];
        const bool grow = mx > m2[cg] + kLazy;
        const float mref = grow ? mx : m2[cg];
        alpha = grow ? __builtin_amdgcn_exp2f(m2[cg] - mref) : 1.0f;
        m2[cg] = mref;
        const float msub = mref == -INFINITY ? 0.0f : mref - kPExp;
        float p[16];
        float ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            p[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], c2s[cg] * kinv[i / 8], -msub));
            ps += p[i];
        }
        lsum[cg] = lsum[cg] * alpha + ps;
        split8(&p[0], ph0, pl0, neg1);
        split8(&p[8], ph1, pl1, neg1);
        return __any(grow);
    }

    // O rows (columns 4g + r of each group) times the alpha of their column.
    __device__ __forceinline__ void rescale(const float (&alpha)[NCG], int g)
    {
#pragma unroll
        for (int cg = 0; cg < NCG; cg++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float ar = __shfl(alpha[cg], 4 * g + r);
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    o[cg][nb][r] *= ar;
            }
    }

    // One 64-token block from LDS buffer `buf`.  `mask` bit l: block token l
    // is cached and on a valid page.  FULL: every token of the block is valid
    // for every column of the wave (a separate instantiation, with no masking
    // code).
    template <bool FULL, class LDS>
    __device__ __forceinline__ void block(const LDS &S, int buf, int base, uint64_t mask, int j, int g)
    {
        // ---- scores: tiles (h, t), row j = token 32h + 8(j/4) + j%4 + 4t ----
        const uint8_t *kp = k_lane(S, buf, j, g, false);
        const uint8_t *klp = KT != KV_F16 ? k_lane(S, buf, j, g, true) : kp;
        f4 s[NCG][2][2];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int t = 0; t < 2; t++) {
#pragma unroll
                for (int cg = 0; cg < NCG; cg++)
                    s[cg][h][t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int kk = 0; kk < KK; kk++) {
                    const int off = k_const(&S, h, t, kk);
                    const h8 ka = ld_frag(kp, off);
                    h8 kl;
                    if (KT != KV_F16)
                        kl = ld_frag(klp, off);
#pragma unroll
                    for (int cg = 0; cg < NCG; cg++) {
                        s[cg][h][t] = mfma(ka, qh[cg][kk], s[cg][h][t]);
                        s[cg][h][t] = mfma(ka, ql[cg][kk], s[cg][h][t]);
                        if (KT != KV_F16)
                            s[cg][h][t] = mfma(kl, qh[cg][kk], s[cg][h][t]);
                    }
                }
            }

        // ---- online softmax of each column over this lane's 16 tokens ----
        h8 ph[2][NCG], pl[2][NCG];
        float alpha[NCG];
        bool grow = false;
#pragma unroll
        for (int cg = 0; cg < NCG; cg++) {
            float sv[16]; // [8h + v]: token 32h + 8g + v
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        sv[8 * h + 4 * t + r] = s[cg][h][t][r];
            grow |= softmax16<FULL>(cg, sv, base, mask, ph[0][cg], pl[0][cg], ph[1][cg], pl[1][cg],
                                    alpha[cg], g);
        }
        if (grow)
            rescale(alpha, g);

        // ---- P V, V operand: dimension 16nb + j, tokens 32h + 8g .. +7 ----
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint8_t *vp = v_lane(S, buf, h, j, g, false);
            const uint8_t *vlp = KT != KV_F16 ? v_lane(S, buf, h, j, g, true) : vp;
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                const h8 vb = ld_frag(vp, v_const(&S, nb));
                h8 vl;
                if (KT != KV_F16)
                    vl = ld_frag(vlp, v_const(&S, nb));
#pragma unroll
                for (int cg = 0; cg < NCG; cg++) {
                    o[cg][nb] = mfma(ph[h][cg], vb, o[cg][nb]);
                    o[cg][nb] = mfma(pl[h][cg], vb, o[cg][nb]);
                    if (KT != KV_F16)
                        o[cg][nb] = mfma(ph[h][cg], vl, o[cg][nb]);
                }
            }
        }
    }

    // ---- the three stages of block(), for the ping-pong kernels ----
    // The operand fragments are read from LDS RA steps ahead of their
    // products, so that the products of one group of waves run back to back
    // while the other group is on the vector ALU.  fp16 pages take two
    // products per operand pair; P V on staged quantised pages three (hi x
    // hi, lo x hi, hi x lo), their scores two (qk_block_kc).
    static constexpr bool LOP = KT != KV_F16;      // lo plane of V
    static constexpr int NPR = LOP ? 3 : 2;        // P V products per pair
    static constexpr int NRD = LOP ? 2 : 1;        // V fragment reads per step
    static constexpr int RA = LOP ? 1 : 2;         // steps read ahead

    // Score tiles of the block in K buffer kb: fp16 pages (two products per
    // pair, Q hi and lo against K), or f32 pages, whose K is staged as hi +
    // lo planes (three: hi x hi, hi x Q lo, lo x Q hi).  Quantised pages use
    // qk_block_kc.
    template <class LDS>
    __device__ __forceinline__ void qk_block(const LDS &S, int kb, f4 (&s)[NCG][2][2], int j, int g) const
    {
        static_assert(KT == KV_F16 || KT == KV_F32, "fp16 K operands, or f32 K as hi + lo planes");
        constexpr bool KLP = KT == KV_F32;
        const uint8_t *kp = k_lane(S, kb, j, g, false);
        const uint8_t *klp = KLP ? k_lane(S, kb, j, g, true) : kp;
        constexpr int NF = 4 * KK; // steps: (h, t, kk), kk fastest
        auto off = [&](int f) { return k_const(&S, f / (2 * KK), (f / KK) % 2, f % KK); };
        h8 kh[RA + 1], kl[RA + 1];
#pragma unroll
        for (int f = 0; f < RA; f++) {
            kh[f] = ld_frag(kp, off(f));
            if (KLP)
                kl[f] = ld_frag(klp, off(f));
        }
#pragma unroll
        for (int f = 0; f < NF; f++) {
            const int h = f / (2 * KK), t = (f / KK) % 2, kk = f % KK;
            if (f + RA < NF) {
                kh[(f + RA) % (RA + 1)] = ld_frag(kp, off(f + RA));
                if (KLP)
                    kl[(f + RA) % (RA + 1)] = ld_frag(klp, off(f + RA));
            }
            const h8 ka = kh[f % (RA + 1)];
            if (kk == 0)
#pragma unroll
                for (int cg = 0; cg < NCG; cg++)
                    s[cg][h][t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int cg = 0; cg < NCG; cg++) {
                s[cg][h][t] = mfma(ka, qh[cg][kk], s[cg][h][t]);
                s[cg][h][t] = mfma(ka, ql[cg][kk], s[cg][h][t]);
                if (KLP)
                    s[cg][h][t] = mfma(kl[f % (RA + 1)], qh[cg][kk], s[cg][h][t]);
            }
        }
        read_ahead_order<NF, (KLP ? 3 : 2) * NCG, KLP ? 2 : 1, RA>();
    }

    // f32 pages: this lane's K scale factors for the block in buffer kb,
    // from the per-wave scales of its four 16-token groups (ks: LDS, 4
    // floats).  Half h of the lane's tokens lies in group 2h + g / 2.
    __device__ __forceinline__ void k_units(const float *ks, int g)
    {
        kinv[0] = pow2_recip(ks[g >> 1]);
        kinv[1] = pow2_recip(ks[2 + (g >> 1)]);
    }

    // f32 pages: moves O tiles 2q, 2q + 1 to the V scale of dimension group
    // q of the block about to be multiplied in (vs: LDS, 4 floats; exact
    // powers of two).  The scales rarely move, so the check is one uniform
    // branch per block.
    __device__ __forceinline__ void v_units(const float *vs)
    {
        static_assert(NB == 8, "four dimension groups of two tiles (head_dim 128)");
        const f4 v4 = *reinterpret_cast<const f4 *>(vs);
        float v[4];
        bool moved = false;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            v[q] = v4[q];
            moved |= v[q] != vso[q];
        }
        if (__builtin_amdgcn_readfirstlane((int)moved)) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float r = v[q] * pow2_recip(vso[q]);
#pragma unroll
                for (int cg = 0; cg < NCG; cg++) {
                    o[cg][2 * q] *= r;
                    o[cg][2 * q + 1] *= r;
                }
                vso[q] = v[q];
            }
        }
    }

    // f32 pages: O back from the V scales it is held in (before finish).
    __device__ __forceinline__ void v_units_out()
    {
#pragma unroll
        for (int cg = 0; cg < NCG; cg++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
                o[cg][nb] *= pow2_recip(vso[nb / 2]);
    }

    // Score tiles of the block in K buffer kb from exact K codes (Lds with
    // KC): per k-step a fresh pair of products (Q hi and lo against the
    // codes of one 32-dimension block), then one mixed-precision FMA per
    // score with the block scale of its token, so that QK^T takes two
    // products per pair instead of three.  A lane's score rows 4g + r of
    // tile (h, t) are tokens 32h + 8g + 4t + r; their scales are read from
    // LDS once per tile, a step ahead of its first products.
    template <class LDS>
    __device__ __forceinline__ void qk_block_kc(const LDS &S, int kb, f4 (&s)[NCG][2][2], int j, int g) const
    {
        const uint8_t *kp = k_lane(S, kb, j, g, false);
        const uint8_t *sp = reinterpret_cast<const uint8_t *>(&S.ks[kb][8 * g * KK]);
        constexpr int NF = 4 * KK, RK = 1; // steps: (h, t, kk), kk fastest; read one step ahead
        auto off = [&](int f) { return k_const(&S, f / (2 * KK), (f / KK) % 2, f % KK); };
        // tile (h, t) = f / KK: its 4 tokens x KK scales, 8 bytes per token
        auto soff = [&](int tile) { return (32 * (tile / 2) + 4 * (tile % 2)) * KK * 2; };
        static_assert(KK == 4, "four scales per token fill 8 bytes");
        h8 kh[RK + 1];
        u4 sc[2][2];
        kh[0] = ld_frag(kp, off(0));
        sc[0][0] = *reinterpret_cast<const u4 *>(sp + soff(0));
        sc[0][1] = *reinterpret_cast<const u4 *>(sp + soff(0) + 16);
        f4 z[NCG];
#pragma unroll
        for (int f = 0; f < NF; f++) {
            const int h = f / (2 * KK), t = (f / KK) % 2, kk = f % KK, tile = f / KK;
            if (f + RK < NF)
                kh[(f + RK) % (RK + 1)] = ld_frag(kp, off(f + RK));
            if (kk == KK - 1 && tile + 1 < 4) {
                sc[(tile + 1) & 1][0] = *reinterpret_cast<const u4 *>(sp + soff(tile + 1));
                sc[(tile + 1) & 1][1] = *reinterpret_cast<const u4 *>(sp + soff(tile + 1) + 16);
            }
            const h8 ka = kh[f % (RK + 1)];
#pragma unroll
            for (int cg = 0; cg < NCG; cg++) {
                z[cg] = mfma(ka, qh[cg][kk], f4{0.0f, 0.0f, 0.0f, 0.0f});
                z[cg] = mfma(ka, ql[cg][kk], z[cg]);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                // scale of token row r, block kk: half (r * KK + kk) of the tile's 32 bytes
                const uint32_t wv = sc[tile & 1][r / 2][(r % 2) * 2 + kk / 2];
                const h2 hv = __builtin_bit_cast(h2, wv);
                const float ksc = (float)hv[kk % 2];
#pragma unroll
                for (int cg = 0; cg < NCG; cg++)
                    s[cg][h][t][r] = fmaf(z[cg][r], ksc, kk == 0 ? 0.0f : s[cg][h][t][r]);
            }
        }
    }

    // Online softmax of the block at `base`: the scores in st are replaced by
    // P in place (st[cg][h][0] holds the hi halves of P half h, st[cg][h][1]
    // the lo halves), so that one register array carries a block between
    // the stages; O is rescaled where a column's reference maximum grew.
    template <bool FULL>
    __device__ __forceinline__ void softmax_block(f4 (&st)[NCG][2][2], int base, uint64_t mask, int g)
    {
        float alpha[NCG];
        bool grow = false;
#pragma unroll
        for (int cg = 0; cg < NCG; cg++) {
            float sv[16];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        sv[8 * h + 4 * t + r] = st[cg][h][t][r];
            h8 ph0, pl0, ph1, pl1;
            grow |= softmax16<FULL>(cg, sv, base, mask, ph0, pl0, ph1, pl1, alpha[cg], g);
            st[cg][0][0] = __builtin_bit_cast(f4, ph0);
            st[cg][0][1] = __builtin_bit_cast(f4, pl0);
            st[cg][1][0] = __builtin_bit_cast(f4, ph1);
            st[cg][1][1] = __builtin_bit_cast(f4, pl1);
        }
        if (grow)
            rescale(alpha, g);
    }

    // O += P V over the block in V buffer vb, P as softmax_block left it.
    // `loads` (N > 0): N global loads, load c issued after the products of
    // step c * (steps / N).
    template <class LDS, class LD = NoLoads>
    __device__ __forceinline__ void pv_block(const LDS &S, int vb, const f4 (&st)[NCG][2][2], int j, int g,
                                             const LD &loads = LD{})
    {
        const uint8_t *vp[2] = {v_lane(S, vb, 0, j, g, false), v_lane(S, vb, 1, j, g, false)};
        const uint8_t *vlp[2] = {LOP ? v_lane(S, vb, 0, j, g, true) : vp[0], LOP ? v_lane(S, vb, 1, j, g, true) : vp[1]};
        constexpr int NF = 2 * NB; // steps: (h, nb), nb fastest
        h8 vh[RA + 1], vl[RA + 1];
#pragma unroll
        for (int f = 0; f < RA; f++) {
            vh[f] = ld_frag(vp[f / NB], v_const(&S, f % NB));
            if (LOP)
                vl[f] = ld_frag(vlp[f / NB], v_const(&S, f % NB));
        }
#pragma unroll
        for (int f = 0; f < NF; f++) {
            const int h = f / NB, nb = f % NB;
            if (f + RA < NF) {
                vh[(f + RA) % (RA + 1)] = ld_frag(vp[(f + RA) / NB], v_const(&S, (f + RA) % NB));
                if (LOP)
                    vl[(f + RA) % (RA + 1)] = ld_frag(vlp[(f + RA) / NB], v_const(&S, (f + RA) % NB));
            }
            const h8 vv = vh[f % (RA + 1)];
#pragma unroll
            for (int cg = 0; cg < NCG; cg++) {
                const h8 phh = __builtin_bit_cast(h8, st[cg][h][0]);
                o[cg][nb] = mfma(phh, vv, o[cg][nb]);
                o[cg][nb] = mfma(__builtin_bit_cast(h8, st[cg][h][1]), vv, o[cg][nb]);
                if (LOP)
                    o[cg][nb] = mfma(phh, vl[f % (RA + 1)], o[cg][nb]);
            }
            if constexpr (LD::N > 0)
                if (f % (NF / LD::N) == 0)
                    loads(f / (NF / LD::N));
        }
        read_ahead_order<NF, NPR * NCG, NRD, RA, (LD::N > 0 ? NF / LD::N : 0)>();
    }

    // O of every column times f (an exact power of two).
    __device__ __forceinline__ void scale_o(float f)
    {
#pragma unroll
        for (int cg = 0; cg < NCG; cg++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
                o[cg][nb] *= f;
    }

    __device__ __forceinline__ void finish(const PrefillArgs &a, int b, int kvh, int col0, int j, int g)
    {
        const int H = a.num_heads, G = H / a.L.num_kv_heads, chunk = a.chunk_len;
#pragma unroll
        for (int cg = 0; cg < NCG; cg++) {
            float lt = lsum[cg];
            lt += __shfl_xor(lt, 16);
            lt += __shfl_xor(lt, 32);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float l = __shfl(lt, 4 * g + r);
                const int c = col0 + 16 * cg + 4 * g + r;
                const int qi = c / G;
                if (qi >= chunk)
                    continue;
                float *op = a.out + (((int64_t)b * chunk + qi) * H + kvh * G + c % G) * HD;
                const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    op[16 * nb + j] = o[cg][nb][r] * inv;
            }
        }
    }
};

// Work split shared by the staged kernels: the workgroup's columns, the
// context each wave and the workgroup must cover, and the block-table reads.
// A tile is the NW * 16 * NCG consecutive columns of one workgroup.  PAIRED
// (the ping-pong kernels): the first half of the waves take their columns
// from tile wx and the second half from tile T - 1 - wx (T tiles), so that a
// short causal range and a long one share each SIMD and every workgroup gets
// about the same work; each half then decides alone which blocks it sees
// whole (wg_full is per half).
template <int P, int NCG, int NW = 4, bool PAIRED = false>
struct PrefillWork {
    int wx, kvh, b, tid, lane, w, j, g, start, mapped, col0, wave_len, wg_full, wg_len;
    bool wave_active;
    const int32_t *bt;

    __device__ __forceinline__ PrefillWork(const PrefillArgs &a)
    {
        constexpr int WCOLS = 16 * NCG;
        wx = gridDim.x - 1 - blockIdx.x; // heaviest (latest-query) workgroups first
        kvh = blockIdx.y;
        b = blockIdx.z;
        tid = threadIdx.x;
        lane = tid & 63;
        w = __builtin_amdgcn_readfirstlane(tid >> 6);
        j = lane & 15;
        g = lane >> 4;
        const int G = a.num_heads / a.L.num_kv_heads, chunk = a.chunk_len;
        start = a.start_pos[b];
        bt = a.block_tables + (int64_t)b * a.max_blocks;
        mapped = a.max_blocks * P;
        auto len = [&](int col) { return min(start + min(col / G, chunk - 1) + 1, mapped); };
        if (PAIRED) {
            const int ta = wx, tb = gridDim.x - 1 - wx; // tiles of the two halves
            const int t = w < NW / 2 ? ta : tb;
            col0 = (t * NW + w) * WCOLS;
            // shortest column of this half
            wg_full = min(start + (t * NW + (w < NW / 2 ? 0 : NW / 2)) * WCOLS / G + 1, mapped);
            wg_len = max(len((ta * NW + NW / 2) * WCOLS - 1), len((tb * NW + NW) * WCOLS - 1));
        } else {
            col0 = (wx * NW + w) * WCOLS;
            wg_full = min(start + wx * NW * WCOLS / G + 1, mapped); // shortest column of the workgroup
            wg_len = len(wx * NW * WCOLS + NW * WCOLS - 1);
        }
        wave_len = len(col0 + WCOLS - 1);
        wave_active = col0 / G < chunk;
        if (start + chunk > mapped && tid == 0 && a.status)
            atomicOr(a.status, FLAG_BAD_SLOT);
    }

    // Whether the block at `base` is whole for every column of the workgroup
    // (PAIRED: of this wave's half): all its tokens valid and before the
    // shortest column's end.
    __device__ __forceinline__ bool block_full(int base, uint64_t mask) const
    {
        return mask == ~0ull && base + kTB <= wg_full;
    }

    // Page id of block token `lane` of the block at `base` (-1 past wg_len).
    __device__ __forceinline__ int table(int base) const { return table_entry<P>(bt, base + lane, wg_len); }

    // Ballot of the block's valid tokens; flags page ids outside the pool.
    __device__ __forceinline__ uint64_t valid_mask(const PrefillArgs &a, int tb, int base) const
    {
        const bool ok = tb >= 0 && tb < a.L.num_pages;
        const bool bad = base + lane < wg_len && !ok;
        if (__ballot(bad) && w == 0 && lane == 0 && a.status)
            atomicOr(a.status, FLAG_BAD_PAGE);
        return __ballot(ok);
    }
};

// NW waves per workgroup share its staging: 4, or 8 (two per SIMD in one
// workgroup, so that one workgroup per CU holds two staging buffers).
template <int HD, int KT, int P, int NBUF, int NCG, int NW>
__global__ __launch_bounds__(64 * NW) void attn_prefill_lds(PrefillArgs a)
{
    constexpr bool F32 = KT == KV_F32;
    static_assert(!F32 || NBUF == 1, "f32 pages exchange block maxima at the single-buffer barrier");
    const PrefillWork<P, NCG, NW> W(a);
    __shared__ Lds<HD, KT, NBUF> S;
    __shared__ float s_bmax[NW][2]; // f32 pages: per-wave |K|, |V| maxima of the block being staged
    WaveAttn<HD, KT, NCG> A;
    A.init(a, W.b, W.kvh, W.col0, W.start, W.mapped, W.wave_active, W.j, W.g);

    StageRegs<HD, KT, NW> R;
    // f32 pages: power-of-two operand scales of the staged block (running,
    // workgroup-uniform), of the block in LDS, and the scale O is held in
    float ksc_run = 0.0f, vsc_run = 0.0f, ksc_cur = 1.0f, vsc_cur = 1.0f, vsc_o = 0.0f;
    // all threads: the staged block's maxima over the workgroup (one
    // barrier), then its scales
    auto f32_scales = [&](uint64_t vmask) {
        if constexpr (F32) {
            float mk, mv;
            f32_chunk_max<HD, P, NW>(R, W.tid, vmask, mk, mv);
            mk = wave_max_nonneg(mk);
            mv = wave_max_nonneg(mv);
            if (W.lane == 0) {
                s_bmax[W.w][0] = mk;
                s_bmax[W.w][1] = mv;
            }
            __syncthreads();
            mk = s_bmax[0][0];
            mv = s_bmax[0][1];
#pragma unroll
            for (int x = 1; x < NW; x++) {
                mk = fmaxf(mk, s_bmax[x][0]);
                mv = fmaxf(mv, s_bmax[x][1]);
            }
            ksc_run = block_scale(mk, ksc_run);
            vsc_run = block_scale(mv, vsc_run);
        }
    };
    int tb = W.table(0);
    uint64_t mask_c = W.valid_mask(a, tb, 0);
    stage_load<HD, KT, P, NW>(a, W.kvh, W.tid, W.w, tb, R);
    tb = W.table(kTB);
    f32_scales(mask_c);
    stage_store<HD, KT, P, NBUF, NW>(a, W.kvh, W.tid, W.w, 0, mask_c, R, S, ksc_run, vsc_run, A.neg1);
    ksc_cur = ksc_run;
    vsc_cur = vsc_run;
    __syncthreads();

    // One staged block; FULL: no column of the workgroup needs masking.
    int base = 0, it = 0;
    auto step = [&](auto full) {
        constexpr bool FULL = decltype(full)::value;
        const int buf = NBUF == 2 ? (it & 1) : 0;
        const bool more = base + kTB < W.wg_len;
        uint64_t mask_n = 0;
        if (more) {
            mask_n = W.valid_mask(a, tb, base + kTB);
            stage_load<HD, KT, P, NW>(a, W.kvh, W.tid, W.w, tb, R);
            tb = W.table(base + 2 * kTB);
        }
        if constexpr (F32) {
            // scores of this block carry its K scale; O moves to its V
            // scale (exact powers of two)
            A.kinv[0] = A.kinv[1] = pow2_recip(ksc_cur);
            if (vsc_o != 0.0f && vsc_o != vsc_cur)
                A.scale_o(vsc_cur * pow2_recip(vsc_o));
            vsc_o = vsc_cur;
        }
        if (W.wave_active && base < W.wave_len)
            A.template block<FULL>(S, buf, base, mask_c, W.j, W.g);
        if (more) {
            if (F32)
                f32_scales(mask_n); // its barrier also frees the single buffer
            else if (NBUF == 1)
                __syncthreads();
            stage_store<HD, KT, P, NBUF, NW>(a, W.kvh, W.tid, W.w, NBUF == 2 ? (buf ^ 1) : 0, mask_n, R, S,
                                         ksc_run, vsc_run, A.neg1);
        }
        mask_c = mask_n;
        ksc_cur = ksc_run;
        vsc_cur = vsc_run;
        __syncthreads();
        base += kTB;
        it++;
    };
    // blocks every column of the workgroup sees whole, then the rest (the
    // causal diagonal, the partial last block, and any block after a page
    // id outside the pool)
    while (base < W.wg_len && W.block_full(base, mask_c))
        step(std::true_type{});
    while (base < W.wg_len)
        step(std::false_type{});
    if (W.wave_active) {
        if (F32 && vsc_o != 0.0f)
            A.scale_o(pow2_recip(vsc_o));
        A.finish(a, W.b, W.kvh, W.col0, W.j, W.g);
    }
}

// Direct global->LDS loads of one fp16 block: issue_k the K plane into K
// buffer `buf`, issue_v the V plane into V buffer `buf`; NW waves share each
// (HD / (8 NW) loads per wave).  K: 1 KiB segments of 512/HD tokens (one page
// each); V: segments of 8 dimensions x 64 tokens, where lane l always fetches
// logical chunk (l & 7) ^ ((l >> 3) & 7), i.e. the same 8 tokens of every
// segment.
template <int HD, int P, int NW = 4>
__device__ __forceinline__ void issue_k(const PrefillArgs &a, int kvh, int w, int lane, int tb, LdsDirect<HD> &S,
                                        int buf)
{
    const PoolLayout &L = a.L;
    const int64_t np = L.num_pages;
    constexpr int KROWS = LdsDirect<HD>::KROWS, KSEG = kTB / KROWS;
    static_assert(KSEG % NW == 0, "whole K segments per wave");
#pragma unroll
    for (int q = 0; q < KSEG / NW; q++) {
        const int seg = NW * q + w;
        const int row = seg * KROWS + lane / (HD / 8);
        const int c = (lane % (HD / 8)) ^ (row & 3);
        const int pr = __builtin_amdgcn_readlane(tb, seg * KROWS);
        const int64_t pg = (pr >= 0 && pr < np) ? pr : 0;
        const uint8_t *src = a.base + pg * L.page_bytes + L.k_off +
                             (((int64_t)kvh * P + row % P) * HD + 8 * c) * 2;
        __builtin_amdgcn_global_load_lds(
            src, (__attribute__((address_space(3))) void *)&S.k[buf][seg * LdsDirect<HD>::KSEGB], 16, 0, 0);
    }
}

template <int HD, int P, int NW = 4>
__device__ __forceinline__ void issue_v(const PrefillArgs &a, int kvh, int w, int lane, int tb, LdsDirect<HD> &S,
                                        int buf)
{
    const PoolLayout &L = a.L;
    const int64_t np = L.num_pages;
    constexpr int VSEG = HD / 8;
    static_assert(VSEG % NW == 0, "whole V segments per wave");
    const int vtok = 8 * ((lane & 7) ^ ((lane >> 3) & 7));
    const int vr = __shfl(tb, vtok);
    const int64_t vpg = (vr >= 0 && vr < np) ? vr : 0;
    const uint8_t *vsrc = a.base + vpg * L.page_bytes + L.v_off + (int64_t)(vtok % P) * 2;
#pragma unroll
    for (int q = 0; q < VSEG / NW; q++) {
        const int seg = NW * q + w;
        const int d = 8 * seg + (lane >> 3);
        __builtin_amdgcn_global_load_lds(vsrc + ((int64_t)kvh * HD + d) * P * 2,
                                         (__attribute__((address_space(3))) void *)&S.v[buf][seg * 8 * kTB],
                                         16, 0, 0);
    }
}

// Zeroes V of the tokens whose `vmask` bit is clear (past the cached range or
// on an invalid page) after a direct load; their scores are masked, and stale
// values must not reach O through 0 * NaN.
template <int HD, int NT = 256>
__device__ __forceinline__ void zero_dead_v(LdsDirect<HD> &S, int buf, uint64_t vmask, int tid)
{
    for (int e = tid; e < HD * (kTB / 8); e += NT) {
        const int d = e / (kTB / 8), c = e % (kTB / 8);
        const uint32_t live = (uint32_t)(vmask >> (8 * c)) & 0xFFu;
        if (live == 0xFFu)
            continue;
        u4 *p = reinterpret_cast<u4 *>(&S.v[buf][d * kTB + 8 * (c ^ (d & 7))]);
        u4 x = *p;
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (!((live >> i) & 1u))
                x[i / 2] &= (i & 1) ? 0x0000FFFFu : 0xFFFF0000u;
        *p = x;
    }
}

__device__ __forceinline__ void wait_direct_loads()
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// fp16 pages, two waves per SIMD in ping-pong.  The workgroup's 8 waves form
// two groups, A (waves 0-3) and B (waves 4-7), one wave of each per SIMD,
// offset by half a block: while one group issues its matrix-core products
// (P V of one block and Q K^T of the next, back to back, at raised wave
// priority) the other runs the online softmax between them on the vector
// ALU, and the roles swap at each barrier.  Per block n:
//   phase 1: A: P V (n - 1), scores (n)      B: softmax (n)
//   phase 2: A: softmax (n)                  B: P V (n), scores (n + 1)
// K and V have two LDS buffers each, filled by direct global->LDS loads that
// all 8 waves issue at the start of phase 2 (K of block n + 2, V of block
// n + 1) and wait for at the end of the next phase 1.  Each group runs its
// own copy of the loop (pp_loop<GB>), so that neither carries the other's
// live values; both pass the same barriers.
template <int HD, int P, int NCG>
struct PingPong {
    static constexpr int NW = 8;
    const PrefillArgs &a;
    const PrefillWork<P, NCG, NW, true> &W;
    LdsDirect<HD> &S;
    WaveAttn<HD, KV_F16, NCG> &A;

    // whether this wave computes on the block at `base`
    __device__ __forceinline__ bool live(int base) const { return W.wave_active && base < W.wave_len; }

    template <bool GB>
    __device__ __forceinline__ void run(int tbv, int tbk, uint64_t mask_c, uint64_t mask_n, int nblk)
    {
        f4 s[NCG][2][2]; // a block's scores, then its P (softmax_block)
        if (GB && live(0))
            A.qk_block(S, 0, s, W.j, W.g);
        int n = 0;
        auto step = [&](auto full) {
            constexpr bool FULL = decltype(full)::value;
            const int base = n * kTB, cur = n & 1;
            // phase 1
            if (!GB) {
                __builtin_amdgcn_s_setprio(1);
                if (n > 0 && live(base - kTB))
                    A.pv_block(S, cur ^ 1, s, W.j, W.g);
                if (live(base))
                    A.qk_block(S, cur, s, W.j, W.g);
                __builtin_amdgcn_s_setprio(0);
            } else if (live(base)) {
                A.template softmax_block<FULL>(s, base, mask_c, W.g);
            }
            wait_direct_loads(); // K of block n + 1 and V of block n
            __syncthreads();
            if (mask_c != ~0ull) { // V of block n has tokens to zero
                zero_dead_v<HD, 64 * NW>(S, cur, mask_c, W.tid);
                __syncthreads();
            }
            // phase 2: group A issues the direct loads before its softmax,
            // which reads no LDS; B's products read LDS with none in flight
            if (!GB) {
                issue_k<HD, P, NW / 2>(a, W.kvh, W.w, W.lane, tbk, S, cur);     // block n + 2
                issue_v<HD, P, NW / 2>(a, W.kvh, W.w, W.lane, tbv, S, cur ^ 1); // block n + 1
            }
            const uint64_t mask_nn = W.valid_mask(a, tbk, base + 2 * kTB);
            tbv = tbk;
            tbk = W.table(base + 3 * kTB);
            if (!GB) {
                if (live(base))
                    A.template softmax_block<FULL>(s, base, mask_c, W.g);
            } else {
                __builtin_amdgcn_s_setprio(1);
                if (live(base))
                    A.pv_block(S, cur, s, W.j, W.g);
                if (live(base + kTB))
                    A.qk_block(S, cur ^ 1, s, W.j, W.g);
                __builtin_amdgcn_s_setprio(0);
            }
            __syncthreads();
            mask_c = mask_n;
            mask_n = mask_nn;
            n++;
        };
        while (n < nblk && W.block_full(n * kTB, mask_c))
            step(std::true_type{});
        while (n < nblk)
            step(std::false_type{});
        if (!GB && nblk > 0 && live((nblk - 1) * kTB))
            A.pv_block(S, (nblk - 1) & 1, s, W.j, W.g);
    }
};

template <int HD, int P, int NCG>
__global__ __launch_bounds__(512) void attn_prefill_pp(PrefillArgs a)
{
    constexpr int NW = PingPong<HD, P, NCG>::NW;
    const PrefillWork<P, NCG, NW, true> W(a);
    __shared__ LdsDirect<HD> S;
    WaveAttn<HD, KV_F16, NCG> A;
    const int nblk = (W.wg_len + kTB - 1) / kTB;

    // prologue: K and V of block 0, K of block 1, in flight while Q is
    // loaded and split
    const int tb = W.table(0);
    const int tbv = W.table(kTB); // block whose V is issued next
    issue_k<HD, P, NW>(a, W.kvh, W.w, W.lane, tb, S, 0);
    issue_v<HD, P, NW>(a, W.kvh, W.w, W.lane, tb, S, 0);
    issue_k<HD, P, NW>(a, W.kvh, W.w, W.lane, tbv, S, 1);
    const int tbk = W.table(2 * kTB); // block whose K is issued next
    A.template init<true>(a, W.b, W.kvh, W.col0, W.start, W.mapped, W.wave_active, W.j, W.g);
    const uint64_t mask_c = W.valid_mask(a, tb, 0);
    const uint64_t mask_n = W.valid_mask(a, tbv, kTB);
    wait_direct_loads();
    __syncthreads();
    if (mask_c != ~0ull) {
        zero_dead_v<HD, 64 * NW>(S, 0, mask_c, W.tid);
        __syncthreads();
    }
    PingPong<HD, P, NCG> pp{a, W, S, A};
    if (W.w >= NW / 2)
        pp.template run<true>(tbv, tbk, mask_c, mask_n, nblk);
    else
        pp.template run<false>(tbv, tbk, mask_c, mask_n, nblk);
    wait_direct_loads(); // loads issued past the end, before the workgroup's LDS is released
    if (W.wave_active)
        A.finish(a, W.b, W.kvh, W.col0, W.j, W.g);
}

// Quantised pages (q8_0, q4_0; head_dim 128), two waves per SIMD in
// ping-pong as attn_prefill_pp, with the blocks staged through registers
// into exact hi + lo fp16 planes (two LDS buffers each for K and V).  Each
// group stages one plane in its vector-ALU phase: B the K plane of block
// n + 1 in phase 1 of block n, A the V plane of block n + 1 in phase 2; the
// global loads of a plane go out one block before its conversion.  Per
// block n:
//   phase 1: A: P V (n - 1), scores (n)      B: softmax (n), K (n + 1) staged
//   phase 2: A: softmax (n), V (n + 1) staged B: P V (n), scores (n + 1)
template <int HD, int KT, int P, int NCG>
struct PingPongQ {
    static constexpr int NW = 8;
    const PrefillArgs &a;
    const PrefillWork<P, NCG, NW, true> &W;
    Lds<HD, KT, 2, true> &S;
    WaveAttn<HD, KT, NCG> &A;

    __device__ __forceinline__ bool live(int base) const { return W.wave_active && base < W.wave_len; }

    // GB: group B (stages K), else group A (stages V).  R holds this
    // group's plane of block 1; tb2 the page ids of block 2.
    template <bool GB>
    __device__ __forceinline__ void run(PlaneRegs<HD, KT> &R, int tb2, uint64_t mask_c, uint64_t mask_n, int nblk)
    {
        const int st = W.tid & 255;
        f4 s[NCG][2][2]; // a block's scores, then its P (softmax_block)
        if (GB && live(0))
            A.qk_block_kc(S, 0, s, W.j, W.g);
        int n = 0;
        auto step = [&](auto full) {
            constexpr bool FULL = decltype(full)::value;
            const int base = n * kTB, cur = n & 1;
            // phase 1
            if (!GB) {
                __builtin_amdgcn_s_setprio(1);
                if (n > 0 && live(base - kTB))
                    A.pv_block(S, cur ^ 1, s, W.j, W.g);
                if (live(base))
                    A.qk_block_kc(S, cur, s, W.j, W.g);
                __builtin_amdgcn_s_setprio(0);
            } else {
                PlaneScales<HD, KT> C;
                plane_scales<0, HD, KT, P>(a, W.kvh, st, R, C); // in flight during the softmax
                if (live(base))
                    A.template softmax_block<FULL>(s, base, mask_c, W.g);
                plane_store<0, HD, KT, P, 2>(a, W.kvh, st, cur ^ 1, 0, R, C, S); // K of block n + 1
                plane_load<0, HD, KT, P>(a, W.kvh, st, tb2, R);                   // K of block n + 2
            }
            __syncthreads();
            // phase 2
            if (!GB) {
                PlaneScales<HD, KT> C;
                plane_scales<1, HD, KT, P>(a, W.kvh, st, R, C); // in flight during the softmax
                if (live(base))
                    A.template softmax_block<FULL>(s, base, mask_c, W.g);
                plane_store<1, HD, KT, P, 2>(a, W.kvh, st, cur ^ 1, mask_n, R, C, S); // V of block n + 1
                plane_load<1, HD, KT, P>(a, W.kvh, st, tb2, R);                        // V of block n + 2
            } else {
                __builtin_amdgcn_s_setprio(1);
                if (live(base))
                    A.pv_block(S, cur, s, W.j, W.g);
                if (live(base + kTB))
                    A.qk_block_kc(S, cur ^ 1, s, W.j, W.g);
                __builtin_amdgcn_s_setprio(0);
            }
            const uint64_t mask_nn = W.valid_mask(a, tb2, base + 2 * kTB);
            tb2 = W.table(base + 3 * kTB);
            __syncthreads();
            mask_c = mask_n;
            mask_n = mask_nn;
            n++;
        };
        while (n < nblk && W.block_full(n * kTB, mask_c))
            step(std::true_type{});
        while (n < nblk)
            step(std::false_type{});
        if (!GB && nblk > 0 && live((nblk - 1) * kTB))
            A.pv_block(S, (nblk - 1) & 1, s, W.j, W.g);
    }
};

template <int HD, int KT, int P, int NCG>
__global__ __launch_bounds__(512) void attn_prefill_ppq(PrefillArgs a)
{
    constexpr int NW = PingPongQ<HD, KT, P, NCG>::NW;
    const PrefillWork<P, NCG, NW, true> W(a);
    __shared__ Lds<HD, KT, 2, true> S;
    WaveAttn<HD, KT, NCG> A;
    const int nblk = (W.wg_len + kTB - 1) / kTB;
    const bool gb = W.w >= NW / 2;
    const int st = W.tid & 255;

    // prologue: both planes of block 0 staged (B: K, A: V), and each group's
    // plane of block 1 loaded; block 0's loads are in flight while Q is
    // loaded and split
    const int tb0 = W.table(0), tb1 = W.table(kTB);
    PlaneRegs<HD, KT> R;
    PlaneScales<HD, KT> C;
    if (gb) {
        plane_load<0, HD, KT, P>(a, W.kvh, st, tb0, R);
        plane_scales<0, HD, KT, P>(a, W.kvh, st, R, C);
    } else {
        plane_load<1, HD, KT, P>(a, W.kvh, st, tb0, R);
        plane_scales<1, HD, KT, P>(a, W.kvh, st, R, C);
    }
    A.template init<true>(a, W.b, W.kvh, W.col0, W.start, W.mapped, W.wave_active, W.j, W.g);
    const uint64_t mask_c = W.valid_mask(a, tb0, 0);
    const uint64_t mask_n = W.valid_mask(a, tb1, kTB);
    if (gb) {
        plane_store<0, HD, KT, P, 2>(a, W.kvh, st, 0, 0, R, C, S);
        plane_load<0, HD, KT, P>(a, W.kvh, st, tb1, R);
    } else {
        plane_store<1, HD, KT, P, 2>(a, W.kvh, st, 0, mask_c, R, C, S);
        plane_load<1, HD, KT, P>(a, W.kvh, st, tb1, R);
    }
    const int tb2 = W.table(2 * kTB);
    __syncthreads();
    PingPongQ<HD, KT, P, NCG> pp{a, W, S, A};
    if (gb)
        pp.template run<true>(R, tb2, mask_c, mask_n, nblk);
    else
        pp.template run<false>(R, tb2, mask_c, mask_n, nblk);
    if (W.wave_active)
        A.finish(a, W.b, W.kvh, W.col0, W.j, W.g);
}

// f32 pages (head_dim 128): one plane of a 64-token block staged by the four
// waves of one group, eight 16-byte chunks per lane.  Wave ws holds K tokens
// 16ws .. 16ws + 15 (chunk c: token 16ws + 2c + l/32, dimensions 4(l%32) ..
// +3, so each load reads 1 KiB of one page), or V dimensions 32ws .. 32ws +
// 31 (chunk c: dimension 32ws + 4c + l/16, tokens 4(l%16) .. +3).
struct PlaneF32 {
    u4 x[8];
};

// This lane's address of chunk 0 of the K (PLANE 0) or V plane of the block
// whose page ids are in tb (lane l: token l); chunk c lies plane_step(c)
// floats further.
template <int PLANE, int P>
__device__ __forceinline__ const float *plane_ptr_f32(const PrefillArgs &a, int kvh, int ws, int lane, int tb)
{
    constexpr int HD = 128;
    const PoolLayout &L = a.L;
    const int64_t np = L.num_pages;
    if (PLANE == 0) {
        const int pr = __builtin_amdgcn_readlane(tb, 16 * ws);
        const int64_t pg = (pr >= 0 && pr < np) ? pr : 0;
        return reinterpret_cast<const float *>(a.base + pg * L.page_bytes + L.k_off) +
               ((int64_t)kvh * P + (16 * ws) % P) * HD + 4 * lane; // lane l: token l/32, dims 4(l%32)
    }
    const int t0 = 4 * (lane & 15);
    const int pr = __shfl(tb, t0);
    const int64_t pg = (pr >= 0 && pr < np) ? pr : 0;
    return reinterpret_cast<const float *>(a.base + pg * L.page_bytes + L.v_off) +
           ((int64_t)kvh * HD + 32 * ws + (lane >> 4)) * P + t0 % P;
}

template <int PLANE, int P>
__device__ constexpr int plane_step(int c)
{
    return PLANE == 0 ? 2 * c * 128 : 4 * c * P;
}

// The eight loads of a plane from plane_ptr_f32, one per call (pv_block
// spreads them between its products).
template <int PLANE, int P>
struct PlaneLoads {
    static constexpr int N = 8;
    const float *p;
    PlaneF32 &R;
    __device__ __forceinline__ void operator()(int c) const
    {
        R.x[c] = *reinterpret_cast<const u4 *>(p + plane_step<PLANE, P>(c));
    }
};

template <int PLANE, int P>
__device__ __forceinline__ void plane_load_f32(const PrefillArgs &a, int kvh, int ws, int lane, int tb, PlaneF32 &R)
{
    const PlaneLoads<PLANE, P> ld{plane_ptr_f32<PLANE, P>(a, kvh, ws, lane, tb), R};
#pragma unroll
    for (int c = 0; c < 8; c++)
        ld(c);
}

// Converts a plane of plane_load_f32 into the hi + lo fp16 planes of buffer
// `buf` (the layout stage_store writes), scaled by this wave's power-of-two
// operand scale, which it derives from the largest live magnitude with the
// running rule of block_scale (`run`: this wave's running scale, 0 at the
// start) and publishes in sc[ws].  `vmask` bit l: block token l is cached and
// on a valid page; stale slots take no part in the scale, and their V is
// stored as zero (their scores are masked, and stale values must not reach O
// through 0 * NaN).
template <int PLANE, int NBUF>
__device__ __forceinline__ void plane_store_f32(int ws, int lane, uint64_t vmask, const PlaneF32 &R, float &run,
                                                float *sc, float neg1, Lds<128, KV_F32, NBUF> &S, int buf)
{
    using G = SwzGeom<128>;
    float x[8][4];
#pragma unroll
    for (int c = 0; c < 8; c++) {
        // words copied out first: hipcc's __builtin_bit_cast of an
        // ext_vector element reads element 0 whatever the index
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            w[i] = R.x[c][i];
#pragma unroll
        for (int i = 0; i < 4; i++)
            x[c][i] = __builtin_bit_cast(float, w[i]);
    }
    // largest live magnitude: maximumNumber with |x| operands compiles to
    // v_max3_f32 with abs modifiers (two values per instruction); a block
    // with every token live (uniform branch) needs no masking
    float m = 0.0f;
    if (vmask == ~0ull) {
#pragma unroll
        for (int c = 0; c < 8; c++)
#pragma unroll
            for (int i = 0; i < 4; i += 2)
                m = maxnum3(m, fabsf(x[c][i]), fabsf(x[c][i + 1]));
    } else {
#pragma unroll
        for (int c = 0; c < 8; c++) {
            if (PLANE == 0) {
                const bool live = (vmask >> (16 * ws + 2 * c + (lane >> 5))) & 1u;
#pragma unroll
                for (int i = 0; i < 4; i++)
                    x[c][i] = live ? x[c][i] : 0.0f; // K of a dead token: its scores are masked
            } else {
                const uint32_t live = (uint32_t)(vmask >> (4 * (lane & 15))) & 0xFu;
#pragma unroll
                for (int i = 0; i < 4; i++)
                    x[c][i] = ((live >> i) & 1u) ? x[c][i] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 4; i += 2)
                m = maxnum3(m, fabsf(x[c][i]), fabsf(x[c][i + 1]));
        }
    }
    run = block_scale(wave_max_nonneg(m), run);
    if (lane == 0)
        sc[ws] = run;
    if (run != 1.0f) { // wave-uniform, and 1 for ordinary data
#pragma unroll
        for (int c = 0; c < 8; c++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                x[c][i] *= run;
    }
#pragma unroll
    for (int c = 0; c < 8; c++) {
        uint32_t hi[2], lo[2];
        split_pair(x[c][0], x[c][1], hi[0], lo[0], neg1);
        split_pair(x[c][2], x[c][3], hi[1], lo[1], neg1);
        if (PLANE == 0) {
            const int tk = 16 * ws + 2 * c + (lane >> 5), col = 4 * (lane & 31);
            *reinterpret_cast<u2 *>(&S.k[buf][G::kel(tk, col)]) = u2{hi[0], hi[1]};
            *reinterpret_cast<u2 *>(&S.kl[buf][G::kel(tk, col)]) = u2{lo[0], lo[1]};
        } else {
            const int d = 32 * ws + 4 * c + (lane >> 4), t0 = 4 * (lane & 15);
            *reinterpret_cast<u2 *>(&S.v[buf][G::vel(d, t0)]) = u2{hi[0], hi[1]};
            *reinterpret_cast<u2 *>(&S.vl[buf][G::vel(d, t0)]) = u2{lo[0], lo[1]};
        }
    }
}

// f32 pages (head_dim 128), two waves per SIMD in ping-pong as
// attn_prefill_ppq, with K and V staged through registers into hi + lo fp16
// planes (two LDS buffers each): group B converts the K plane of block n + 1
// at the start of phase 1 of block n, group A the V plane at the start of
// phase 2.  Each group loads its plane in its product phase before, one
// load instruction every other step of P V (a load holds the wave while the
// address unit takes it, about as long as a product), so that the 32
// staging registers are not live through the softmax.
// Every staging wave picks its own power-of-two scale (block_scale), so no
// barrier is spent on block maxima: a K scale covers 16 tokens (the softmax
// takes a factor per half of a lane's tokens, k_units), a V scale 32
// dimensions (two O tiles, v_units).  Per block n:
//   phase 1: A: P V (n - 1) with the loads of V (n + 1), scores (n)
//            B: convert K (n + 1), softmax (n)
//   phase 2: A: convert V (n + 1), softmax (n)
//            B: P V (n) with the loads of K (n + 2), scores (n + 1)
template <int HD, int P, int NCG>
struct PingPongF {
    static constexpr int NW = 8;
    const PrefillArgs &a;
    const PrefillWork<P, NCG, NW, true> &W;
    Lds<HD, KV_F32, 2> &S;
    float (&sc)[2][2][4]; // [plane][buffer][staging wave]
    WaveAttn<HD, KV_F32, NCG> &A;

    __device__ __forceinline__ bool live(int base) const { return W.wave_active && base < W.wave_len; }

    __device__ __forceinline__ void scores(int kb, f4 (&s)[NCG][2][2]) { A.qk_block(S, kb, s, W.j, W.g); }
    __device__ __forceinline__ void pv(int vb, const f4 (&s)[NCG][2][2])
    {
        A.v_units(sc[1][vb]);
        A.pv_block(S, vb, s, W.j, W.g);
    }
    // P V with a plane's loads issued between its products (or alone when
    // this wave has no P V to do)
    template <int PLANE>
    __device__ __forceinline__ void pv_loads(bool do_pv, int vb, const f4 (&s)[NCG][2][2], int tb, PlaneF32 &R)
    {
        const PlaneLoads<PLANE, P> ld{plane_ptr_f32<PLANE, P>(a, W.kvh, W.w & 3, W.lane, tb), R};
        if (do_pv) {
            A.v_units(sc[1][vb]);
            A.pv_block(S, vb, s, W.j, W.g, ld);
        } else {
#pragma unroll
            for (int c = 0; c < 8; c++)
                ld(c);
        }
    }
    template <bool FULL>
    __device__ __forceinline__ void softmax(int kb, f4 (&s)[NCG][2][2], int base, uint64_t mask)
    {
        A.k_units(sc[0][kb], W.g);
        A.template softmax_block<FULL>(s, base, mask, W.g);
    }

    // GB: group B (stages K), else group A (stages V).  R: B holds the K
    // plane of block 1; tbn: the page ids of the block whose plane this
    // group loads next (B: block 2, A: block 1); run: this wave's running
    // scale.
    template <bool GB>
    __device__ __forceinline__ void run(PlaneF32 &R, float &run, int tbn, uint64_t mask_c, uint64_t mask_n,
                                        int nblk)
    {
        const int ws = W.w & 3;
        f4 s[NCG][2][2]; // a block's scores, then its P (softmax_block)
        if (GB && live(0))
            scores(0, s);
        int n = 0;
        auto step = [&](auto full) {
            constexpr bool FULL = decltype(full)::value;
            const int base = n * kTB, cur = n & 1;
            int tb2; // page ids of block n + 2
            // phase 1
            if (!GB) {
                __builtin_amdgcn_s_setprio(1);
                tb2 = W.table(base + 2 * kTB); // before the plane's loads: the mask below waits for it alone
                pv_loads<1>(n > 0 && live(base - kTB), cur ^ 1, s, tbn, R); // P V (n - 1), loads of V (n + 1)
                tbn = tb2;
                if (live(base))
                    scores(cur, s);
                __builtin_amdgcn_s_setprio(0);
            } else {
                plane_store_f32<0, 2>(ws, W.lane, mask_n, R, run, sc[0][cur ^ 1], A.neg1, S, cur ^ 1); // K (n + 1)
                if (live(base))
                    softmax<FULL>(cur, s, base, mask_c);
            }
            __syncthreads();
            // phase 2
            if (!GB) {
                plane_store_f32<1, 2>(ws, W.lane, mask_n, R, run, sc[1][cur ^ 1], A.neg1, S, cur ^ 1); // V (n + 1)
                if (live(base))
                    softmax<FULL>(cur, s, base, mask_c);
            } else {
                __builtin_amdgcn_s_setprio(1);
                tb2 = tbn;
                tbn = W.table(base + 3 * kTB);
                pv_loads<0>(live(base), cur, s, tb2, R); // P V (n), loads of K (n + 2)
                if (live(base + kTB))
                    scores(cur ^ 1, s);
                __builtin_amdgcn_s_setprio(0);
            }
            const uint64_t mask_nn = W.valid_mask(a, tb2, base + 2 * kTB);
            __syncthreads();
            mask_c = mask_n;
            mask_n = mask_nn;
            n++;
        };
        while (n < nblk && W.block_full(n * kTB, mask_c))
            step(std::true_type{});
        while (n < nblk)
            step(std::false_type{});
        if (!GB && nblk > 0 && live((nblk - 1) * kTB))
            pv((nblk - 1) & 1, s);
    }
};

template <int HD, int P, int NCG>
__global__ __launch_bounds__(512) void attn_prefill_ppf(PrefillArgs a)
{
    static_assert(HD == 128, "f32 ping-pong staging maps head_dim 128");
    constexpr int NW = PingPongF<HD, P, NCG>::NW;
    const PrefillWork<P, NCG, NW, true> W(a);
    __shared__ Lds<HD, KV_F32, 2> S;
    __shared__ __attribute__((aligned(16))) float sc[2][2][4];
    WaveAttn<HD, KV_F32, NCG> A;
    const int nblk = (W.wg_len + kTB - 1) / kTB;
    const bool gb = W.w >= NW / 2;
    const int ws = W.w & 3;

    // prologue: both planes of block 0 staged (B: K, A: V), and B's plane of
    // block 1 loaded; block 0's loads are in flight while Q is loaded and
    // split
    const int tb0 = W.table(0), tb1 = W.table(kTB), tb2 = W.table(2 * kTB);
    PlaneF32 R;
    float run = 0.0f;
    if (gb)
        plane_load_f32<0, P>(a, W.kvh, ws, W.lane, tb0, R);
    else
        plane_load_f32<1, P>(a, W.kvh, ws, W.lane, tb0, R);
    A.template init<true>(a, W.b, W.kvh, W.col0, W.start, W.mapped, W.wave_active, W.j, W.g);
    const uint64_t mask_c = W.valid_mask(a, tb0, 0);
    const uint64_t mask_n = W.valid_mask(a, tb1, kTB);
    if (gb) {
        plane_store_f32<0, 2>(ws, W.lane, mask_c, R, run, sc[0][0], A.neg1, S, 0);
        plane_load_f32<0, P>(a, W.kvh, ws, W.lane, tb1, R);
    } else {
        plane_store_f32<1, 2>(ws, W.lane, mask_c, R, run, sc[1][0], A.neg1, S, 0);
    }
    __syncthreads();
    PingPongF<HD, P, NCG> pp{a, W, S, sc, A};
    if (gb)
        pp.template run<true>(R, run, tb2, mask_c, mask_n, nblk);
    else
        pp.template run<false>(R, run, tb1, mask_c, mask_n, nblk);
    if (W.wave_active) {
        A.v_units_out();
        A.finish(a, W.b, W.kvh, W.col0, W.j, W.g);
    }
}

} // namespace mfma_prefill

bool mfma_prefill_supported(const PoolLayout &L, int num_heads)
{
    // q4_0 and f32: the staged kernel only (pages of 16/32/64 tokens; q4_0
    // with head_dim 128)
    const bool staged = L.page_tokens == 16 || L.page_tokens == 32 || L.page_tokens == 64;
    if (L.kv_type == KV_Q4_0 && (L.head_dim != 128 || !staged))
        return false;
    if (L.kv_type == KV_F32 && !staged)
        return false;
    if (L.page_tokens % 16 != 0 || (L.head_dim != 64 && L.head_dim != 128))
        return false;
    if (num_heads % L.num_kv_heads)
        return false;
    const int G = num_heads / L.num_kv_heads;
    return G == 1 || G == 2 || G == 4 || G == 8 || G == 16;
}

// Column groups per wave: two share each K/V block's loads and conversion
// when registers allow (head_dim 64); head_dim 128 keeps one so that two
// waves fit per SIMD.
template <int HD>
constexpr int prefill_ncg()
{
    return HD == 64 ? 2 : 1;
}

// The register-staged kernel (attn_prefill_lds) now serves f32 pages at
// head_dim 64 (8-wave workgroups over one buffer: their block maxima are
// exchanged at its barrier, every wave staging) and q8_0 pages at head_dim
// 64 (4-wave workgroups over one buffer).  fp16 pages, and f32 and the
// quantised pages at head_dim 128, run the ping-pong kernels.
template <int HD, int KT>
constexpr int kPrefillWaves = KT == KV_F32 ? 8 : 4;

// Column groups per wave: two halve the LDS reads per matrix-core product;
// taken where the kernel then still fits two waves per SIMD (256 VGPRs).
// f32 pages take one: with their staging spread over 8 waves (four 16-byte
// chunks per thread) the kernel then fits two waves per SIMD (234 VGPRs),
// where two groups over 4 waves held one (397 VGPRs): 203 against 153
// TFLOP/s on the Llama-3-8B 4096-token prefill.
template <int HD, int KT, int P>
constexpr int prefill_lds_ncg()
{
    return KT == KV_F32 ? 1 : (HD == 64 || P == 16 || (KT != KV_F16 && P == 32)) ? 2 : 1;
}

// The ping-pong kernels hold two column groups per wave.
constexpr int kPrefillPingPongNcg = 2;
// The f32 ping-pong kernel holds one column group per wave: its staging
// keeps a plane's 32 KiB (32 VGPRs per thread) in flight beside each wave's
// state, 223 VGPRs with one group, and two groups spill 524.
constexpr int kPrefillF32Ncg = 1;

template <int HD, int KT>
static void launch_lds(const PrefillArgs &a, hipStream_t st)
{
    using namespace mfma_prefill;
    constexpr int NBUF = 1;
    constexpr int NW = kPrefillWaves<HD, KT>;
    const int G = a.num_heads / a.L.num_kv_heads;
    const int64_t cols = (int64_t)a.chunk_len * G;
    auto grid = [&](int ncg, int nw) {
        const int64_t per_wg = nw * 16 * ncg;
        return dim3((unsigned)((cols + per_wg - 1) / per_wg), a.L.num_kv_heads, a.batch);
    };
    if constexpr (KT == KV_F16) {
        constexpr int NCG = kPrefillPingPongNcg;
        switch (a.L.page_tokens) {
        case 16:
            hipLaunchKernelGGL((attn_prefill_pp<HD, 16, NCG>), grid(NCG, 8), dim3(512), 0, st, a);
            break;
        case 32:
            hipLaunchKernelGGL((attn_prefill_pp<HD, 32, NCG>), grid(NCG, 8), dim3(512), 0, st, a);
            break;
        default:
            hipLaunchKernelGGL((attn_prefill_pp<HD, 64, NCG>), grid(NCG, 8), dim3(512), 0, st, a);
            break;
        }
    } else if constexpr (KT == KV_F32 && HD == 128) {
        constexpr int NCG = kPrefillF32Ncg;
        switch (a.L.page_tokens) {
        case 16:
            hipLaunchKernelGGL((attn_prefill_ppf<HD, 16, NCG>), grid(NCG, 8), dim3(512), 0, st, a);
            break;
        case 32:
            hipLaunchKernelGGL((attn_prefill_ppf<HD, 32, NCG>), grid(NCG, 8), dim3(512), 0, st, a);
            break;
        default:
            hipLaunchKernelGGL((attn_prefill_ppf<HD, 64, NCG>), grid(NCG, 8), dim3(512), 0, st, a);
            break;
        }
    } else if constexpr ((KT == KV_Q8_0 || KT == KV_Q4_0) && HD == 128) {
        constexpr int NCG = kPrefillPingPongNcg;
        switch (a.L.page_tokens) {
        case 16:
            hipLaunchKernelGGL((attn_prefill_ppq<HD, KT, 16, NCG>), grid(NCG, 8), dim3(512), 0, st, a);
            break;
        case 32:
            hipLaunchKernelGGL((attn_prefill_ppq<HD, KT, 32, NCG>), grid(NCG, 8), dim3(512), 0, st, a);
            break;
        default:
            hipLaunchKernelGGL((attn_prefill_ppq<HD, KT, 64, NCG>), grid(NCG, 8), dim3(512), 0, st, a);
            break;
        }
    } else {
#define GI_PFL(PT)                                                                           \
    hipLaunchKernelGGL((attn_prefill_lds<HD, KT, PT, NBUF, prefill_lds_ncg<HD, KT, PT>(), NW>), \
                       grid(prefill_lds_ncg<HD, KT, PT>(), NW), dim3(64 * NW), 0, st, a)
    switch (a.L.page_tokens) {
    case 16:
        GI_PFL(16);
        break;
    case 32:
        GI_PFL(32);
        break;
    default:
        GI_PFL(64);
        break;
    }
#undef GI_PFL
    }
}

hipError_t launch_prefill_mfma(const PrefillArgs &a, hipStream_t st)
{
    using namespace mfma_prefill;
    const int G = a.num_heads / a.L.num_kv_heads;
    const int64_t cols = (int64_t)a.chunk_len * G;
    const int P = a.L.page_tokens;
    if (P == 16 || P == 32 || P == 64) {
        if (a.L.head_dim == 128) {
            if (a.L.kv_type == KV_F16)
                launch_lds<128, KV_F16>(a, st);
            else if (a.L.kv_type == KV_Q4_0)
                launch_lds<128, KV_Q4_0>(a, st);
            else if (a.L.kv_type == KV_F32)
                launch_lds<128, KV_F32>(a, st);
            else
                launch_lds<128, KV_Q8_0>(a, st);
        } else {
            if (a.L.kv_type == KV_F16)
                launch_lds<64, KV_F16>(a, st);
            else if (a.L.kv_type == KV_F32)
                launch_lds<64, KV_F32>(a, st);
            else
                launch_lds<64, KV_Q8_0>(a, st);
        }
        return hipGetLastError();
    }
    const int per_wg = 4 * 16 * (a.L.head_dim == 64 ? prefill_ncg<64>() : prefill_ncg<128>());
    dim3 grid((unsigned)((cols + per_wg - 1) / per_wg), a.L.num_kv_heads, a.batch);
#define GI_PF(HD, KT) \
    hipLaunchKernelGGL((attn_prefill<HD, KT, prefill_ncg<HD>()>), grid, dim3(256), 0, st, a)
    if (a.L.head_dim == 128) {
        if (a.L.kv_type == KV_F16)
            GI_PF(128, KV_F16);
        else
            GI_PF(128, KV_Q8_0);
    } else {
        if (a.L.kv_type == KV_F16)
            GI_PF(64, KV_F16);
        else
            GI_PF(64, KV_Q8_0);
    }
#undef GI_PF
    return hipGetLastError();
}

} // namespace gi
