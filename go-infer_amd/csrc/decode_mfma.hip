// Paged GQA decode attention on the matrix cores, fp16 pages.
//
// Same semantics as the vector-ALU kernel (pkg/engine/forward.go:242-267
// with the online softmax), arranged for CDNA4's 16x16x32 f16 MFMA:
//
//   S^T[token][head] = K[token][d] * Q^T[d][head]     (A = K rows straight
//                                                       from the page)
//   O[head][d]      += P[head][token] * V[token][d]    (B = V from the
//                                                       dimension-major page)
//
// A wave walks 32-token blocks (two 16-token MFMA row tiles).  The query is
// split into hi + lo halves (q = hi + lo exactly up to 2^-22 |q|) and the
// probabilities likewise, so both products keep float32 accuracy while K/V
// feed the MFMA in their stored fp16 form: no conversion instructions on the
// bandwidth path.  The k-slot -> token assignment of the P*V product is
// chosen to equal the token layout the S tile comes out in, so P never moves
// between lanes.  Each of the 4 waves keeps its own running max/sum and the
// workgroup merges them at the end (and split-K partials are merged by
// merge_splits in decode_attn.hip).
#include "gi_common.h"
#include "gi_kernels.h"

#include <math.h>

namespace gi {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

namespace {

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f4 mfma(h8 a, h8 b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <int HD>
__global__ __launch_bounds__(256) void attn_mfma_f16(DecodeArgs a)
{
    constexpr int KK = HD / 32; // k-steps of the score product
    constexpr int NB = HD / 16; // 16-column blocks of the output
    const PoolLayout &L = a.L;
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int j = lane & 15, q4 = lane >> 4;
    const int H = a.num_heads, KVH = L.num_kv_heads, G = H / KVH, P = L.page_tokens;
    const int h0 = kvh * G;
    int len = a.seq_lens[b];
    if (len > a.max_blocks * P) {
        if (threadIdx.x == 0 && split == 0 && a.status)
            atomicOr(a.status, FLAG_BAD_SLOT);
        len = a.max_blocks * P;
    }
    const int t0 = split * a.split_tokens;
    const int t1 = min(len, t0 + a.split_tokens);
    const int64_t qrow = (int64_t)b * H + h0;

    __shared__ float s_o[4][16][HD];
    __shared__ float s_m[4][16], s_l[4][16];

    float *wsp = nullptr;
    if (a.num_splits > 1)
        wsp = a.ws + (((int64_t)b * KVH + kvh) * a.num_splits + split) * (G * (HD + 2));

    if (t0 >= t1) {
        for (int e = threadIdx.x; e < G * HD; e += 256) {
            if (wsp)
                wsp[e] = 0.0f;
            else
                a.out[qrow * HD + e] = 0.0f;
        }
        if (wsp && threadIdx.x < G) {
            wsp[G * HD + 2 * threadIdx.x] = -INFINITY;
            wsp[G * HD + 2 * threadIdx.x + 1] = 0.0f;
        }
        return;
    }

    // Q^T operand: column j = head h0 + j (zero beyond the group), k-slot
    // (q4, v) of step kk = dimension 32*kk + 8*q4 + v.
    h8 qh[KK], ql[KK];
#pragma unroll
    for (int kk = 0; kk < KK; kk++)
#pragma unroll
        for (int v = 0; v < 8; v++) {
            float x = j < G ? a.q[(qrow + j) * HD + 32 * kk + 8 * q4 + v] : 0.0f;
            _Float16 hi = (_Float16)x;
            qh[kk][v] = hi;
            ql[kk][v] = (_Float16)(x - (float)hi);
        }

    const float c = a.scale * kLog2e;
    float m2 = -INFINITY; // running max of head j, log2 units
    float lsum = 0.0f;    // this lane's share of the running denominator
    f4 o[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
        o[nb] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    const int64_t koff = L.k_off + (int64_t)kvh * P * HD * 2;
    const int64_t voff = L.v_off + (int64_t)kvh * HD * P * 2;
    const int32_t *bt = a.block_tables + (int64_t)b * a.max_blocks;

    for (int base = t0 + 32 * w; base < t1; base += 128) {
        const int tA = base, tB = base + 16;
        int64_t pA = bt[tA / P];
        int64_t pB = tB < t1 ? (int64_t)bt[tB / P] : pA;
        bool okA = pA >= 0 && pA < L.num_pages;
        bool okB = pB >= 0 && pB < L.num_pages;
        if (!(okA && okB)) {
            if (lane == 0 && a.status)
                atomicOr(a.status, FLAG_BAD_PAGE);
            if (!okA)
                pA = 0;
            if (!okB)
                pB = 0;
        }
        const int sA = tA % P, sB = tB % P;
        const uint8_t *gA = a.base + pA * L.page_bytes;
        const uint8_t *gB = a.base + pB * L.page_bytes;

        h8 k0[KK], k1[KK];
#pragma unroll
        for (int kk = 0; kk < KK; kk++) {
            k0[kk] = *reinterpret_cast<const h8 *>(gA + koff + ((int64_t)(sA + j) * HD + 32 * kk + 8 * q4) * 2);
            k1[kk] = *reinterpret_cast<const h8 *>(gB + koff + ((int64_t)(sB + j) * HD + 32 * kk + 8 * q4) * 2);
        }
        h4 v0[NB], v1[NB];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            v0[nb] = *reinterpret_cast<const h4 *>(gA + voff + ((int64_t)(16 * nb + j) * P + sA + 4 * q4) * 2);
            v1[nb] = *reinterpret_cast<const h4 *>(gB + voff + ((int64_t)(16 * nb + j) * P + sB + 4 * q4) * 2);
        }

        f4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < KK; kk++) {
            s0 = mfma(k0[kk], qh[kk], s0);
            s0 = mfma(k0[kk], ql[kk], s0);
            s1 = mfma(k1[kk], qh[kk], s1);
            s1 = mfma(k1[kk], ql[kk], s1);
        }

        // lane holds head j, tokens base + 4*q4 + r (sc[r]) and
        // base + 16 + 4*q4 + r (sc[4 + r])
        float sc[8];
        const bool tail = base + 32 > t1 || !(okA && okB);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            sc[r] = s0[r] * c;
            sc[4 + r] = s1[r] * c;
        }
        if (tail) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int ta = base + 4 * q4 + r, tb = base + 16 + 4 * q4 + r;
                if (!(ta < t1 && okA)) {
                    sc[r] = -INFINITY;
#pragma unroll
                    for (int nb = 0; nb < NB; nb++)
                        v0[nb][r] = (_Float16)0.0f;
                }
                if (!(tb < t1 && okB)) {
                    sc[4 + r] = -INFINITY;
#pragma unroll
                    for (int nb = 0; nb < NB; nb++)
                        v1[nb][r] = (_Float16)0.0f;
                }
            }
        }
        float mx = sc[0];
#pragma unroll
        for (int i = 1; i < 8; i++)
            mx = fmaxf(mx, sc[i]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mnew = fmaxf(m2, mx);
        const float alpha = exp2f(m2 - mnew);
        m2 = mnew;
        float ps = 0.0f;
        h8 ph, pl;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float p = exp2f(sc[i] - mnew);
            ps += p;
            const _Float16 hi = (_Float16)p;
            ph[i] = hi;
            pl[i] = (_Float16)(p - (float)hi);
        }
        lsum = lsum * alpha + ps;
        // output rows of this lane are heads 4*q4 + r; their rescale factor
        // lives in lane 4*q4 + r (any lane whose column is that head)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float ar = __shfl(alpha, 4 * q4 + r);
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
                o[nb][r] *= ar;
        }
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            h8 vv;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                vv[v] = v0[nb][v];
                vv[4 + v] = v1[nb][v];
            }
            o[nb] = mfma(ph, vv, o[nb]);
            o[nb] = mfma(pl, vv, o[nb]);
        }
    }

    // wave totals -> LDS
    float lt = lsum;
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    if (q4 == 0) {
        s_m[w][j] = m2;
        s_l[w][j] = lt;
    }
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            s_o[w][4 * q4 + r][16 * nb + j] = o[nb][r];
    __syncthreads();

    for (int e = threadIdx.x; e < G * HD; e += 256) {
        const int hh = e / HD, d = e - hh * HD;
        float M = s_m[0][hh];
#pragma unroll
        for (int x = 1; x < 4; x++)
            M = fmaxf(M, s_m[x][hh]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int x = 0; x < 4; x++) {
            const float mx2 = s_m[x][hh];
            const float f = mx2 == -INFINITY ? 0.0f : exp2f(mx2 - M);
            num = fmaf(s_o[x][hh][d], f, num);
            den = fmaf(s_l[x][hh], f, den);
        }
        if (wsp) {
            wsp[hh * HD + d] = num;
            if (d == 0) {
                wsp[G * HD + 2 * hh] = M * (1.0f / kLog2e);
                wsp[G * HD + 2 * hh + 1] = den;
            }
        } else {
            a.out[(qrow + hh) * HD + d] = den > 0.0f ? num / den : 0.0f;
        }
    }
}

} // namespace

bool mfma_decode_supported(const PoolLayout &L, int num_heads)
{
    if (L.kv_type != KV_F16 || L.page_tokens % 16 != 0)
        return false;
    if (L.head_dim != 64 && L.head_dim != 128)
        return false;
    if (num_heads % L.num_kv_heads)
        return false;
    const int G = num_heads / L.num_kv_heads;
    return G >= 1 && G <= 16;
}

hipError_t launch_decode_mfma(const DecodeArgs &a, hipStream_t st)
{
    dim3 grid(a.num_splits, a.L.num_kv_heads, a.batch);
    if (a.L.head_dim == 128)
        hipLaunchKernelGGL(attn_mfma_f16<128>, grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(attn_mfma_f16<64>, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

} // namespace gi
