// Chunked-prefill causal attention on the matrix cores (fp16 and q8_0 pages).
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
// fp16 hi + lo halves, so results keep float32 accuracy.
//
// q8_0 pages stay exact: int8 values are exact in fp16 (converted with a
// byte permute: 0x64XX is 1024 + XX), the K block scale of each 32-wide
// k-step multiplies that step's partial scores, and the V block scale of
// each 32 dimensions is folded into P for the products of those dimensions.
#include "gi_common.h"
#include "gi_kernels.h"

#include <math.h>

namespace gi {

namespace mfma_prefill {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f4 mfma(h8 a, h8 b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h8 ld16(const uint8_t *p)
{
    return __builtin_nontemporal_load(reinterpret_cast<const h8 *>(p));
}

// Eight int8 values -> eight exact fp16 values.  (x ^ 0x80) is x + 128 as an
// unsigned byte; 0x64 in the high byte makes the half 1024 + (x + 128);
// subtracting 1152 leaves x.
__device__ __forceinline__ h8 i8x8_to_h8(uint2 w)
{
    const uint32_t x0 = w.x ^ 0x80808080u, x1 = w.y ^ 0x80808080u;
    const uint32_t c = 0x64646464u;
    uint32_t u[4] = {__builtin_amdgcn_perm(c, x0, 0x04010400u), __builtin_amdgcn_perm(c, x0, 0x04030402u),
                     __builtin_amdgcn_perm(c, x1, 0x04010400u), __builtin_amdgcn_perm(c, x1, 0x04030402u)};
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    h8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        h2 t = __builtin_bit_cast(h2, u[i]) - bias;
        r[2 * i] = t[0];
        r[2 * i + 1] = t[1];
    }
    return r;
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
__device__ __forceinline__ void split8(const float *x, h8 &hi, h8 &lo)
{
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const h2 h = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(x[2 * k], x[2 * k + 1]));
        hi[2 * k] = h[0];
        hi[2 * k + 1] = h[1];
        lo[2 * k] = (_Float16)(x[2 * k] - (float)h[0]);
        lo[2 * k + 1] = (_Float16)(x[2 * k + 1] - (float)h[1]);
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
                k0[kk] = i8x8_to_h8(*reinterpret_cast<const uint2 *>(g0 + koff + (int64_t)s0 * HD + 32 * kk + 8 * g));
                k1[kk] = i8x8_to_h8(*reinterpret_cast<const uint2 *>(g1 + koff + (int64_t)s1 * HD + 32 * kk + 8 * g));
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
                vv[nb] = i8x8_to_h8(*reinterpret_cast<const uint2 *>(gv + voff + (int64_t)(16 * nb + j) * P + sv));
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
            const float alpha = mnew == -INFINITY ? 1.0f : exp2f(m2[cg] - mnew);
            m2[cg] = mnew;
            // p carries a factor 2^14 (so its lo half stays a normal fp16);
            // the running sum carries the same factor and it cancels at the end.
            float p[8], ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                p[i] = mnew == -INFINITY ? 0.0f : exp2f(sc[i] - mnew + 14.0f);
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
                    split8(x, ph, pl);
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
// LDS-staged form.  A workgroup owns 4 x NCG x 16 (query, head) columns of one
// kv head and streams the context in 64-token blocks through double-buffered
// LDS: all 256 threads load a block (one 16-byte global load per chunk,
// int8 converted to exact fp16 on the way), then every wave reads its MFMA
// operands from LDS.  The next block's global loads are in flight while the
// current block is computed.  Used when the page size divides 64.
constexpr int kTB = 64; // tokens per staged block

template <int HD, int KT>
struct StageRegs {
    // 16-byte chunks per thread: fp16 K and V rows of 8 elements, or int8 K
    // rows / V columns of 16 elements.
    static constexpr int NC = KT == KV_F16 ? HD / 32 : HD / 64;
    u4 k[NC], v[NC];
    uint32_t ks[HD / 64 > 0 ? HD / 64 : 1]; // q8_0: K scales of one token, packed halves
    uint32_t vs;                            // q8_0: one V scale (low half)
};

template <int HD, int KT>
struct Lds {
    __attribute__((aligned(16))) _Float16 k[2][kTB][HD + 8]; // token-major K, rows padded
    __attribute__((aligned(16))) _Float16 v[2][HD][kTB + 8]; // dimension-major V
    __attribute__((aligned(16))) float ksc[2][kTB][HD / 32]; // q8_0 K scales
    __attribute__((aligned(16))) float vsc[2][HD / 32][kTB]; // q8_0 V scales
    uint8_t valid[2][kTB];                                   // token on a page inside the pool
};

template <int HD, int KT>
__device__ __forceinline__ void stage_load(const PrefillArgs &a, const int32_t *bt, int base,
                                           int wg_len, int kvh, int tid, StageRegs<HD, KT> &R)
{
    const PoolLayout &L = a.L;
    const int P = L.page_tokens;
    auto page_of = [&](int t) -> int64_t {
        if (t >= wg_len)
            return -1;
        int64_t pg = bt[t / P];
        return (pg >= 0 && pg < L.num_pages) ? pg : -1;
    };
#pragma unroll
    for (int c = 0; c < R.NC; c++) {
        const int ch = tid + 256 * c;
        if (KT == KV_F16) {
            // K: token ch / (HD/8), 8 elements at column 8*(ch % (HD/8))
            const int tok = ch / (HD / 8), col = ch % (HD / 8);
            const int t = base + tok;
            const int64_t pg = page_of(t);
            R.k[c] = pg < 0 ? u4{0, 0, 0, 0}
                            : __builtin_nontemporal_load(reinterpret_cast<const u4 *>(
                                  a.base + pg * L.page_bytes + L.k_off +
                                  (((int64_t)kvh * P + t % P) * HD + 8 * col) * 2));
            // V: page segment, dimension, group of 8 tokens
            const int per_seg = HD * P / 8;
            const int seg = ch / per_seg, rem = ch % per_seg;
            const int d = rem / (P / 8), tg = rem % (P / 8);
            const int tv = base + seg * P + 8 * tg;
            const int64_t pv = page_of(tv);
            R.v[c] = pv < 0 ? u4{0, 0, 0, 0}
                            : __builtin_nontemporal_load(reinterpret_cast<const u4 *>(
                                  a.base + pv * L.page_bytes + L.v_off +
                                  (((int64_t)kvh * HD + d) * P + 8 * tg) * 2));
        } else {
            const int tok = ch / (HD / 16), col = ch % (HD / 16);
            const int t = base + tok;
            const int64_t pg = page_of(t);
            R.k[c] = pg < 0 ? u4{0, 0, 0, 0}
                            : __builtin_nontemporal_load(reinterpret_cast<const u4 *>(
                                  a.base + pg * L.page_bytes + L.k_off +
                                  ((int64_t)kvh * P + t % P) * HD + 16 * col));
            const int per_seg = HD * P / 16;
            const int seg = ch / per_seg, rem = ch % per_seg;
            const int d = rem / (P / 16), tg = rem % (P / 16);
            const int tv = base + seg * P + 16 * tg;
            const int64_t pv = page_of(tv);
            R.v[c] = pv < 0 ? u4{0, 0, 0, 0}
                            : __builtin_nontemporal_load(reinterpret_cast<const u4 *>(
                                  a.base + pv * L.page_bytes + L.v_off +
                                  ((int64_t)kvh * HD + d) * P + 16 * tg));
        }
    }
    if (KT == KV_Q8_0) {
        if (tid < kTB) {
            const int t = base + tid;
            const int64_t pg = page_of(t);
            const uint16_t *src = reinterpret_cast<const uint16_t *>(
                a.base + (pg < 0 ? 0 : pg) * L.page_bytes + L.ks_off) +
                ((int64_t)kvh * P + t % P) * (HD / 32);
#pragma unroll
            for (int i = 0; i < HD / 64; i++)
                R.ks[i] = pg < 0 ? 0u : (uint32_t)src[2 * i] | ((uint32_t)src[2 * i + 1] << 16);
        }
        if (tid < kTB * (HD / 32)) {
            const int db = tid / kTB, tok = tid % kTB;
            const int t = base + tok;
            const int64_t pg = page_of(t);
            R.vs = pg < 0 ? 0u
                          : reinterpret_cast<const uint16_t *>(a.base + pg * L.page_bytes + L.vs_off)
                                [((int64_t)kvh * (HD / 32) + db) * P + t % P];
        }
    }
}

template <int HD, int KT>
__device__ __forceinline__ void stage_store(const PrefillArgs &a, const int32_t *bt, int base,
                                            int wg_len, int tid, int buf,
                                            const StageRegs<HD, KT> &R, Lds<HD, KT> &S)
{
    const PoolLayout &L = a.L;
    const int P = L.page_tokens;
#pragma unroll
    for (int c = 0; c < R.NC; c++) {
        const int ch = tid + 256 * c;
        if (KT == KV_F16) {
            const int tok = ch / (HD / 8), col = ch % (HD / 8);
            *reinterpret_cast<u4 *>(&S.k[buf][tok][8 * col]) = R.k[c];
            const int per_seg = HD * P / 8;
            const int seg = ch / per_seg, rem = ch % per_seg;
            const int d = rem / (P / 8), tg = rem % (P / 8);
            const int t0 = seg * P + 8 * tg; // block-local first token
            u4 vv = R.v[c];
            if (base + t0 + 8 > wg_len) {
                // tokens past the cached range read as zero
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (base + t0 + i >= wg_len)
                        vv[i / 2] &= (i & 1) ? 0x0000FFFFu : 0xFFFF0000u;
            }
            *reinterpret_cast<u4 *>(&S.v[buf][d][t0]) = vv;
        } else {
            const int tok = ch / (HD / 16), col = ch % (HD / 16);
            const h8 lo8 = i8x8_to_h8(uint2{R.k[c][0], R.k[c][1]});
            const h8 hi8 = i8x8_to_h8(uint2{R.k[c][2], R.k[c][3]});
            *reinterpret_cast<h8 *>(&S.k[buf][tok][16 * col]) = lo8;
            *reinterpret_cast<h8 *>(&S.k[buf][tok][16 * col + 8]) = hi8;
            const int per_seg = HD * P / 16;
            const int seg = ch / per_seg, rem = ch % per_seg;
            const int d = rem / (P / 16), tg = rem % (P / 16);
            const int t0 = seg * P + 16 * tg;
            h8 v0 = i8x8_to_h8(uint2{R.v[c][0], R.v[c][1]});
            h8 v1 = i8x8_to_h8(uint2{R.v[c][2], R.v[c][3]});
            if (base + t0 + 16 > wg_len) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (base + t0 + i >= wg_len)
                        v0[i] = (_Float16)0.0f;
                    if (base + t0 + 8 + i >= wg_len)
                        v1[i] = (_Float16)0.0f;
                }
            }
            *reinterpret_cast<h8 *>(&S.v[buf][d][t0]) = v0;
            *reinterpret_cast<h8 *>(&S.v[buf][d][t0 + 8]) = v1;
        }
    }
    if (tid < kTB) {
        const int t = base + tid;
        bool ok = t < wg_len;
        if (ok) {
            const int64_t pg = bt[t / P];
            ok = pg >= 0 && pg < L.num_pages;
            if (!ok && a.status)
                atomicOr(a.status, FLAG_BAD_PAGE);
        }
        S.valid[buf][tid] = ok ? 1 : 0;
        if (KT == KV_Q8_0) {
#pragma unroll
            for (int i = 0; i < HD / 64; i++) {
                S.ksc[buf][tid][2 * i] = half_bits_to_float(R.ks[i] & 0xFFFFu);
                S.ksc[buf][tid][2 * i + 1] = half_bits_to_float(R.ks[i] >> 16);
            }
        }
    }
    if (KT == KV_Q8_0 && tid < kTB * (HD / 32))
        S.vsc[buf][tid / kTB][tid % kTB] = half_bits_to_float(R.vs);
}

template <int HD, int KT, int NCG>
__global__ __launch_bounds__(256) void attn_prefill_lds(PrefillArgs a)
{
    constexpr int KK = HD / 32, NB = HD / 16, NDB = HD / 32;
    const PoolLayout &L = a.L;
    const int kvh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int H = a.num_heads, G = H / L.num_kv_heads, P = L.page_tokens;
    const int start = a.start_pos[b];
    const int chunk = a.chunk_len;
    const int32_t *bt = a.block_tables + (int64_t)b * a.max_blocks;
    const int mapped = a.max_blocks * P;

    __shared__ Lds<HD, KT> S;

    int col0[NCG], qlen[NCG];
    int wave_len = 0;
#pragma unroll
    for (int cg = 0; cg < NCG; cg++) {
        col0[cg] = ((blockIdx.x * 4 + w) * NCG + cg) * 16;
        const int qi = min((col0[cg] + j) / G, chunk - 1);
        qlen[cg] = min(start + qi + 1, mapped);
        wave_len = max(wave_len, min(start + min((col0[cg] + 15) / G, chunk - 1) + 1, mapped));
    }
    if (start + chunk > mapped && tid == 0 && a.status)
        atomicOr(a.status, FLAG_BAD_SLOT);
    const int wg_last = (blockIdx.x * 4 * NCG + 4 * NCG) * 16 - 1;
    const int wg_len = min(start + min(wg_last / G, chunk - 1) + 1, mapped);
    const bool wave_active = col0[0] / G < chunk;

    // Q^T operands (hi, lo) scaled per column by 2^qe.
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
                qv[kk][v] = wave_active ? qp[32 * kk + 8 * g + v] : 0.0f;
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
    float vnorm[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++)
        vnorm[db] = 0.0f;

    StageRegs<HD, KT> R;
    stage_load<HD, KT>(a, bt, 0, wg_len, kvh, tid, R);
    stage_store<HD, KT>(a, bt, 0, wg_len, tid, 0, R, S);
    __syncthreads();

    for (int base = 0, it = 0; base < wg_len; base += kTB, it++) {
        const int buf = it & 1;
        const bool more = base + kTB < wg_len;
        if (more)
            stage_load<HD, KT>(a, bt, base + kTB, wg_len, kvh, tid, R);

        if (wave_active && base < wave_len) {
            // ---- scores: tiles (h, t), row j = token 32h + 8(j/4) + j%4 + 4t ----
            f4 s[NCG][2][2];
#pragma unroll
            for (int cg = 0; cg < NCG; cg++)
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int t = 0; t < 2; t++)
                        s[cg][h][t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const int row = 32 * h + 8 * (j >> 2) + (j & 3) + 4 * t;
                    float ks[4][KK]; // q8_0: scale of output row token 32h + 8g + 4t + r
                    if (KT == KV_Q8_0) {
#pragma unroll
                        for (int r = 0; r < 4; r++)
#pragma unroll
                            for (int kk = 0; kk < KK; kk++)
                                ks[r][kk] = S.ksc[buf][32 * h + 8 * g + 4 * t + r][kk];
                    }
#pragma unroll
                    for (int kk = 0; kk < KK; kk++) {
                        const h8 ka = *reinterpret_cast<const h8 *>(&S.k[buf][row][32 * kk + 8 * g]);
#pragma unroll
                        for (int cg = 0; cg < NCG; cg++) {
                            if (KT == KV_F16) {
                                s[cg][h][t] = mfma(ka, qh[cg][kk], s[cg][h][t]);
                                s[cg][h][t] = mfma(ka, ql[cg][kk], s[cg][h][t]);
                            } else {
                                f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                                z = mfma(ka, qh[cg][kk], z);
                                z = mfma(ka, ql[cg][kk], z);
#pragma unroll
                                for (int r = 0; r < 4; r++)
                                    s[cg][h][t][r] = fmaf(z[r], ks[r][kk], s[cg][h][t][r]);
                            }
                        }
                    }
                }

            // q8_0: running power-of-two normaliser of each V block's scales
            float vmul[NDB];
            if (KT == KV_Q8_0) {
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    float mv = 0.0f;
#pragma unroll
                    for (int h = 0; h < 2; h++)
#pragma unroll
                        for (int v = 0; v < 8; v++)
                            mv = fmaxf(mv, S.vsc[buf][db][32 * h + 8 * g + v]);
                    mv = fmaxf(mv, __shfl_xor(mv, 16));
                    mv = fmaxf(mv, __shfl_xor(mv, 32));
                    uint32_t bits = __builtin_bit_cast(uint32_t, mv);
                    if (bits & 0x7FFFFFu)
                        bits = (bits & 0xFF800000u) + 0x800000u;
                    const float pw = __builtin_bit_cast(float, bits);
                    if (pw > vnorm[db]) {
                        const float f = vnorm[db] / pw;
#pragma unroll
                        for (int cg = 0; cg < NCG; cg++)
#pragma unroll
                            for (int hh = 0; hh < 2; hh++)
                                o[cg][2 * db + hh] *= f;
                        vnorm[db] = pw;
                    }
                    vmul[db] = vnorm[db] > 0.0f ? 1.0f / vnorm[db] : 0.0f;
                }
            }

            // ---- online softmax per column ----
            float p[NCG][16]; // [8h + v]: token 32h + 8g + v
#pragma unroll
            for (int cg = 0; cg < NCG; cg++) {
                float sc[16];
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int t = 0; t < 2; t++)
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            sc[8 * h + 4 * t + r] = s[cg][h][t][r] * c2s[cg];
                const int lim = qlen[cg];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int tl = 32 * (i / 8) + 8 * g + (i % 8);
                    if (!(base + tl < lim && S.valid[buf][tl]))
                        sc[i] = -INFINITY;
                }
                float mx = sc[0];
#pragma unroll
                for (int i = 1; i < 16; i++)
                    mx = fmaxf(mx, sc[i]);
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                const float mnew = fmaxf(m2[cg], mx);
                const float alpha = mnew == -INFINITY ? 1.0f : exp2f(m2[cg] - mnew);
                m2[cg] = mnew;
                float ps = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    p[cg][i] = mnew == -INFINITY ? 0.0f : exp2f(sc[i] - mnew + 14.0f);
                    ps += p[cg][i];
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
            }

            // ---- P * V, V operand: dimension 16nb + j, tokens 32h + 8g .. +7 ----
#pragma unroll
            for (int h = 0; h < 2; h++) {
                h8 ph[NCG], pl[NCG];
                if (KT == KV_F16) {
#pragma unroll
                    for (int cg = 0; cg < NCG; cg++)
                        split8(&p[cg][8 * h], ph[cg], pl[cg]);
                }
#pragma unroll
                for (int nb = 0; nb < NB; nb++) {
                    if (KT == KV_Q8_0 && (nb & 1) == 0) {
                        const int db = nb / 2;
                        float vs8[8];
#pragma unroll
                        for (int v = 0; v < 8; v++)
                            vs8[v] = S.vsc[buf][db][32 * h + 8 * g + v] * vmul[db];
#pragma unroll
                        for (int cg = 0; cg < NCG; cg++) {
                            float x[8];
#pragma unroll
                            for (int v = 0; v < 8; v++)
                                x[v] = p[cg][8 * h + v] * vs8[v];
                            split8(x, ph[cg], pl[cg]);
                        }
                    }
                    const h8 vb = *reinterpret_cast<const h8 *>(&S.v[buf][16 * nb + j][32 * h + 8 * g]);
#pragma unroll
                    for (int cg = 0; cg < NCG; cg++) {
                        o[cg][nb] = mfma(ph[cg], vb, o[cg][nb]);
                        o[cg][nb] = mfma(pl[cg], vb, o[cg][nb]);
                    }
                }
            }
        }

        if (more)
            stage_store<HD, KT>(a, bt, base + kTB, wg_len, tid, buf ^ 1, R, S);
        __syncthreads();
    }

    if (!wave_active)
        return;
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
}

} // namespace mfma_prefill

bool mfma_prefill_supported(const PoolLayout &L, int num_heads)
{
    if (L.kv_type != KV_F16 && L.kv_type != KV_Q8_0)
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

#ifndef GI_PREFILL_LDS_NCG
#define GI_PREFILL_LDS_NCG 1
#endif

hipError_t launch_prefill_mfma(const PrefillArgs &a, hipStream_t st)
{
    using namespace mfma_prefill;
    const int G = a.num_heads / a.L.num_kv_heads;
    const int64_t cols = (int64_t)a.chunk_len * G;
    const int P = a.L.page_tokens;
    if (64 % P == 0) {
        constexpr int ncg = GI_PREFILL_LDS_NCG;
        const int per_wg = 4 * 16 * ncg;
        dim3 grid((unsigned)((cols + per_wg - 1) / per_wg), a.L.num_kv_heads, a.batch);
#define GI_PFL(HD, KT) hipLaunchKernelGGL((attn_prefill_lds<HD, KT, ncg>), grid, dim3(256), 0, st, a)
        if (a.L.head_dim == 128) {
            if (a.L.kv_type == KV_F16)
                GI_PFL(128, KV_F16);
            else
                GI_PFL(128, KV_Q8_0);
        } else {
            if (a.L.kv_type == KV_F16)
                GI_PFL(64, KV_F16);
            else
                GI_PFL(64, KV_Q8_0);
        }
#undef GI_PFL
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
