// Paged GQA attention, vector-ALU kernel (all KV types) and the split-K
// merge.
//
// Semantics follow the reference's decode loop (pkg/engine/forward.go:
// 242-267): for q-head h, kv head h / (H/KVH); score[t] = dot(q_h, K[t]) *
// scale; softmax over t < L (pkg/math/kernels.go:48-70); out_h = sum_t
// p[t] V[t].  The softmax is evaluated online (running max / sum per head)
// so a page is read once; the result equals the two-pass form up to float
// rounding.  One workgroup owns one (query, kv head, context split) and
// serves all H/KVH query heads of the group, so each K/V element is read
// from HBM once per decode step.
#include "gi_common.h"
#include "gi_kernels.h"
#include "split_plan.h"

#include <math.h>

namespace gi {

namespace {

constexpr int NT = 256;

// Eight consecutive K elements of (page, kv head, slot) starting at d0,
// widened to float32 exactly as the reference reads them.
template <int KT, int HD>
__device__ __forceinline__ void load8_k(const uint8_t *pg, const PoolLayout &L, int kvh, int s,
                                        int d0, float *o)
{
    const int64_t row = (int64_t)kvh * L.page_tokens + s;
    if (KT == KV_F32) {
        const float4 *p = reinterpret_cast<const float4 *>(pg + L.k_off + (row * HD + d0) * 4);
        float4 a = p[0], b = p[1];
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
        o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    } else if (KT == KV_F16) {
        uint4 w = *reinterpret_cast<const uint4 *>(pg + L.k_off + (row * HD + d0) * 2);
        uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[2 * i] = half_bits_to_float(u[i] & 0xFFFFu);
            o[2 * i + 1] = half_bits_to_float(u[i] >> 16);
        }
    } else if (KT == KV_Q4_0) {
        // dims d0..d0+7 of one block: the low nibbles of bytes j..j+7 when
        // d0 % 32 < 16, else the high nibbles of bytes j-16..j-9
        const int blk = d0 >> 5, j = d0 & 31;
        uint2 w = *reinterpret_cast<const uint2 *>(pg + L.k_off + (row * (HD / 32) + blk) * 16 + (j & 15));
        float sc = half_bits_to_float(reinterpret_cast<const uint16_t *>(pg + L.ks_off)[row * (HD / 32) + blk]);
        const int sh = j & 16 ? 4 : 0;
        uint32_t u[2] = {w.x, w.y};
#pragma unroll
        for (int i = 0; i < 8; i++)
            o[i] = (float)((int)((u[i >> 2] >> (8 * (i & 3) + sh)) & 15) - 8) * sc;
    } else {
        uint2 w = *reinterpret_cast<const uint2 *>(pg + L.k_off + row * HD + d0);
        float sc = half_bits_to_float(
            reinterpret_cast<const uint16_t *>(pg + L.ks_off)[row * (HD / 32) + (d0 >> 5)]);
        uint32_t u[2] = {w.x, w.y};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            int8_t q = (int8_t)((u[i >> 2] >> (8 * (i & 3))) & 0xFF);
            o[i] = (float)q * sc;
        }
    }
}

// One V element (page, kv head, dimension d, slot), widened to float32.
template <int KT, int HD>
__device__ __forceinline__ float load_v(const uint8_t *pg, const PoolLayout &L, int kvh, int d,
                                        int s)
{
    const int64_t idx = ((int64_t)kvh * HD + d) * L.page_tokens + s;
    if (KT == KV_F32)
        return reinterpret_cast<const float *>(pg + L.v_off)[idx];
    if (KT == KV_F16)
        return half_bits_to_float(reinterpret_cast<const uint16_t *>(pg + L.v_off)[idx]);
    if (KT == KV_Q4_0) {
        const int blk = d >> 5, j = d & 31;
        const int64_t bi = (int64_t)kvh * (HD / 32) + blk;
        const uint8_t b = pg[L.v_off + (bi * 16 + (j & 15)) * L.page_tokens + s];
        const float sc = half_bits_to_float(reinterpret_cast<const uint16_t *>(pg + L.vs_off)[bi * L.page_tokens + s]);
        return (float)((int)((j & 16 ? b >> 4 : b) & 15) - 8) * sc;
    }
    float sc = half_bits_to_float(reinterpret_cast<const uint16_t *>(
        pg + L.vs_off)[((int64_t)kvh * (HD / 32) + (d >> 5)) * L.page_tokens + s]);
    return (float)reinterpret_cast<const int8_t *>(pg + L.v_off)[idx] * sc;
}

// Workgroup = 256 threads over one (query, kv head, split).  Tiles of TOK
// tokens: in the score phase TPT = HD/8 threads share a token (8 elements
// each, tree-reduced with lane shuffles); the softmax phase keeps a running
// max / sum per query head in LDS; in the P*V phase thread (d, group) owns
// one output dimension for a slice of the tile's tokens, reading the
// dimension-major V tile.
template <int KT, int HD, int G>
__global__ __launch_bounds__(NT) void attn_valu(DecodeArgs a)
{
    constexpr int TPT = HD / 8;
    constexpr int TOK = NT / TPT;
    constexpr int NG = NT / HD;
    constexpr int TPG = TOK / NG;
    static_assert(G * TOK <= NT, "softmax phase needs one thread per (head, token)");
    static_assert(TOK % NG == 0, "tile tokens split evenly over P*V groups");

    const PoolLayout &L = a.L;
    const int kvh = blockIdx.y;
    const int tid = threadIdx.x;
    const int H = a.num_heads;
    const int h0 = kvh * G;
    const int P = L.page_tokens;

    __shared__ float s_p[G][TOK];
    __shared__ float s_alpha[G];
    __shared__ float s_m[G], s_l[G];
    __shared__ float s_acc[NG][G][HD];

    // decode: the workgroup is a work unit of the plan (split_plan.h) and
    // walks the segments of its block range; prefill: query row blockIdx.z
    // whole, one workgroup per (query, kv head)
    const bool planned = a.plan_units > 0;
    UnitCursor cur{};
    if (planned && !plan_unit<NT>(a, blockIdx.x, kvh, blockIdx.x == 0 && blockIdx.y == 0, cur))
        return;
    for (;;) {
        int b, qi, t0, t1, len;
        Segment seg{};
        if (planned) {
            bool unused = false;
            b = cur.b;
            qi = 0;
            len = plan_len(a, b, (int64_t)a.max_blocks * P, unused);
            seg = plan_segment(cur, len);
            t0 = seg.t0;
            t1 = seg.t1;
        } else {
            b = blockIdx.z / a.n_q;
            qi = blockIdx.z - b * a.n_q;
            len = a.start_pos ? a.start_pos[b] + qi + 1 : a.seq_lens[b];
            if (len > a.max_blocks * P) {
                // More tokens than the block table maps: read what it maps.
                if (tid == 0 && a.status)
                    atomicOr(a.status, FLAG_BAD_SLOT);
                len = a.max_blocks * P;
            }
            t0 = 0;
            t1 = len;
        }
        const int qrow = b * a.n_q + qi;
        const int32_t *bt = a.block_tables + (int64_t)b * a.max_blocks;
        const int64_t qbase = (int64_t)qrow * H;

        // partial slot when the sequence continues outside this unit's range
        float *wsp = planned && seg.split ? plan_slot(a, cur.unit, seg.slot, kvh, G, HD) : nullptr;

        if (t0 >= t1) {
            // Empty range (an empty prefill context): zero output.
            for (int e = tid; e < G * HD; e += NT)
                a.out[(qbase + h0 + e / HD) * HD + e % HD] = 0.0f;
            break;
        }

        const int part = tid % TPT, tok = tid / TPT, d0 = part * 8;
        float qr[G][8];
    #pragma unroll
        for (int g = 0; g < G; g++)
    #pragma unroll
            for (int j = 0; j < 8; j++)
                qr[g][j] = a.q[(qbase + h0 + g) * HD + d0 + j];
        if (tid < G) {
            s_m[tid] = -INFINITY;
            s_l[tid] = 0.0f;
        }
        const int pd = tid % HD, pgp = tid / HD;
        float acc[G];
    #pragma unroll
        for (int g = 0; g < G; g++)
            acc[g] = 0.0f;
        __syncthreads();

        for (int tb = t0; tb < t1; tb += TOK) {
            // ---- scores ----
            const int t = tb + tok;
            bool valid = t < t1;
            float ps[G];
    #pragma unroll
            for (int g = 0; g < G; g++)
                ps[g] = 0.0f;
            if (valid) {
                int64_t page = bt[t / P];
                if (page < 0 || page >= L.num_pages) {
                    if (part == 0 && a.status)
                        atomicOr(a.status, FLAG_BAD_PAGE);
                    valid = false;
                } else {
                    float kf[8];
                    load8_k<KT, HD>(a.base + page * L.page_bytes, L, kvh, t % P, d0, kf);
    #pragma unroll
                    for (int g = 0; g < G; g++)
    #pragma unroll
                        for (int j = 0; j < 8; j++)
                            ps[g] = fmaf(qr[g][j], kf[j], ps[g]);
                }
            }
    #pragma unroll
            for (int g = 0; g < G; g++)
    #pragma unroll
                for (int m = TPT / 2; m >= 1; m >>= 1)
                    ps[g] += __shfl_xor(ps[g], m, TPT);
    #pragma unroll
            for (int g = 0; g < G; g++)
                if (part == g)
                    s_p[g][tok] = valid ? ps[g] * a.scale : -INFINITY;
            __syncthreads();

            // ---- online softmax, one thread per (head, token) ----
            if (tid < G * TOK) {
                const int g = tid / TOK, tt = tid % TOK;
                const float sv = s_p[g][tt];
                float mx = sv;
    #pragma unroll
                for (int m = TOK / 2; m >= 1; m >>= 1)
                    mx = fmaxf(mx, __shfl_xor(mx, m, TOK));
                const float m_old = s_m[g];
                const float m_new = fmaxf(m_old, mx);
                const float p = sv == -INFINITY ? 0.0f : expf(sv - m_new);
                float sum = p;
    #pragma unroll
                for (int m = TOK / 2; m >= 1; m >>= 1)
                    sum += __shfl_xor(sum, m, TOK);
                s_p[g][tt] = p;
                if (tt == 0) {
                    const float al = m_old == -INFINITY ? 0.0f : expf(m_old - m_new);
                    s_alpha[g] = al;
                    s_m[g] = m_new;
                    s_l[g] = s_l[g] * al + sum;
                }
            }
            __syncthreads();

            // ---- P * V ----
    #pragma unroll
            for (int g = 0; g < G; g++)
                acc[g] *= s_alpha[g];
            for (int i = 0; i < TPG; i++) {
                const int tt = pgp * TPG + i;
                const int t2 = tb + tt;
                if (t2 < t1) {
                    int64_t page = bt[t2 / P];
                    if (page >= 0 && page < L.num_pages) {
                        float vv = load_v<KT, HD>(a.base + page * L.page_bytes, L, kvh, pd, t2 % P);
    #pragma unroll
                        for (int g = 0; g < G; g++)
                            acc[g] = fmaf(s_p[g][tt], vv, acc[g]);
                    }
                }
            }
            __syncthreads();
        }

    #pragma unroll
        for (int g = 0; g < G; g++)
            s_acc[pgp][g][pd] = acc[g];
        __syncthreads();
        if (tid < HD) {
    #pragma unroll
            for (int g = 0; g < G; g++) {
                float s = 0.0f;
    #pragma unroll
                for (int grp = 0; grp < NG; grp++)
                    s += s_acc[grp][g][pd];
                if (wsp) {
                    wsp[g * HD + pd] = s;
                } else {
                    const float l = s_l[g];
                    a.out[(qbase + h0 + g) * HD + pd] = l > 0.0f ? s / l : 0.0f;
                }
            }
            if (wsp && tid < G) {
                wsp[G * HD + 2 * tid] = s_m[tid];
                wsp[G * HD + 2 * tid + 1] = s_l[tid];
            }
        }
        if (planned && seg.split && seg.slot == 1 && kvh == 0 && tid == 0) {
            // b starts here and continues: merge_splits combines its units
            plan_desc(a, cur.unit)[0] = b;
            plan_desc(a, cur.unit)[1] = (cur.sblk + plan_nblk(len) - 1) / cur.cb - cur.unit + 1;
        }
        if (!planned || !plan_next(a, cur, plan_nblk(len)))
            break;
        __syncthreads(); // the shared arrays are free for the next segment
    }
}

// Combines the partials of split sequences (split_plan.h):
//   out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M),  M = max_s m_s,
// summed in unit order (so the result does not depend on scheduling).  One
// workgroup per (kv head, unit): unit u's descriptor names the sequence that
// starts in its range and continues (its partials: slot 1 of unit u, then
// slot 0 of the next n - 1 units); other workgroups exit at once.  Thread g
// first takes head g's maximum and denominator; the per-split factors then
// go through LDS, so that every thread issues its partial loads together.
constexpr int kMergePass = 32; // splits per pass
__global__ __launch_bounds__(256) void merge_splits(DecodeArgs a)
{
    const int kvh = blockIdx.x, u0 = blockIdx.y, tid = threadIdx.x;
    const int b = plan_desc(a, u0)[0], n = plan_desc(a, u0)[1];
    if (b < 0 || n <= 1)
        return;
    const int HD = a.L.head_dim, G = a.num_heads / a.L.num_kv_heads;
    float *out = a.out + ((int64_t)b * a.num_heads + kvh * G) * HD;
    // partial s: slot 1 of unit u0, then slot 0 of units u0 + 1 ..
    auto part = [&](int s) -> const float * {
        return s == 0 ? plan_slot(a, u0, 1, kvh, G, HD) : plan_slot(a, u0 + s, 0, kvh, G, HD);
    };
    __shared__ float s_f[kMergePass][16]; // e^(m_s - M) of head g
    __shared__ float s_M[16], s_den[16];
    if (tid < G) {
        float M = -INFINITY;
        for (int s0 = 0; s0 < n; s0 += 8) {
            float m[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                m[i] = s0 + i < n ? part(s0 + i)[G * HD + 2 * tid] : -INFINITY;
#pragma unroll
            for (int i = 0; i < 8; i++)
                M = fmaxf(M, m[i]);
        }
        float den = 0.0f;
        if (M != -INFINITY) {
            for (int s0 = 0; s0 < n; s0 += 8) {
                float m[8], l[8];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    m[i] = s0 + i < n ? part(s0 + i)[G * HD + 2 * tid] : -INFINITY;
                    l[i] = s0 + i < n ? part(s0 + i)[G * HD + 2 * tid + 1] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (m[i] != -INFINITY)
                        den = fmaf(l[i], expf(m[i] - M), den);
            }
        }
        s_M[tid] = M;
        s_den[tid] = den;
    }
    // outputs of this thread: e = tid + 256 i < G * HD (G * HD <= 2048)
    float num[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < n; s0 += kMergePass) {
        const int ns = min(kMergePass, n - s0);
        __syncthreads(); // s_M is set, and s_f is free again
        for (int e = tid; e < ns * G; e += 256) {
            const int s = e / G, g = e - s * G;
            const float M = s_M[g], m = part(s0 + s)[G * HD + 2 * g];
            s_f[s][g] = (M == -INFINITY || m == -INFINITY) ? 0.0f : expf(m - M);
        }
        __syncthreads();
        for (int s1 = 0; s1 < ns; s1 += 8) {
            float v[8][8];
#pragma unroll
            for (int k = 0; k < 8; k++)
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int e = tid + 256 * i;
                    v[k][i] = s1 + k < ns && e < G * HD ? part(s0 + s1 + k)[e] : 0.0f;
                }
#pragma unroll
            for (int k = 0; k < 8; k++)
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int e = tid + 256 * i;
                    if (s1 + k < ns && e < G * HD)
                        num[i] = fmaf(v[k][i], s_f[s1 + k][e / HD], num[i]);
                }
        }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int e = tid + 256 * i;
        if (e < G * HD) {
            const float den = s_den[e / HD];
            out[e] = den > 0.0f ? num[i] / den : 0.0f;
        }
    }
}

template <int KT>
hipError_t launch_valu_kt(const DecodeArgs &a, dim3 grid, hipStream_t st)
{
    const int HD = a.L.head_dim;
    const int G = a.num_heads / a.L.num_kv_heads;
#define GI_VALU(HDv, Gv)                                                                     \
    if (HD == HDv && G == Gv) {                                                              \
        hipLaunchKernelGGL((attn_valu<KT, HDv, Gv>), grid, dim3(NT), 0, st, a);              \
        return hipGetLastError();                                                            \
    }
    GI_VALU(64, 1) GI_VALU(64, 2) GI_VALU(64, 4) GI_VALU(64, 8)
    GI_VALU(128, 1) GI_VALU(128, 2) GI_VALU(128, 4) GI_VALU(128, 8) GI_VALU(128, 16)
#undef GI_VALU
    return hipErrorInvalidValue;
}

} // namespace

void decode_plan(const PoolLayout &L, int num_cus, int max_len, DecodeArgs &a)
{
    // work units (workgroups) per kv head: kDecodeWgPerCu per CU over the kv
    // heads, fewer when max_len (a hint: 0 when unknown) shows a smaller
    // stream, so that no unit is planned below kMinUnitBlocks blocks.  A
    // wrong hint only changes the balance: the kernels size their ranges from
    // the lengths in device memory.
    int wg = (kDecodeWgPerCu * (num_cus > 0 ? num_cus : 256) + L.num_kv_heads - 1) / L.num_kv_heads;
    if (max_len > 0) {
        const int64_t blocks = (int64_t)a.batch * ((max_len + kPlanBlock - 1) / kPlanBlock);
        const int64_t need = (blocks + kMinUnitBlocks - 1) / kMinUnitBlocks;
        if (need < wg)
            wg = (int)(need > 0 ? need : 1);
    }
    a.plan_units = wg;
}

int decode_grid_items(const DecodeArgs &a) { return a.plan_units; }

size_t decode_desc_offset(const PoolLayout &L, int num_heads, int plan_units)
{
    const int G = num_heads / L.num_kv_heads;
    return ((size_t)2 * plan_units * L.num_kv_heads * G * (L.head_dim + 2) * sizeof(float) + 255) / 256 * 256;
}

size_t decode_workspace_bytes(const PoolLayout &L, int num_heads, int plan_units)
{
    return decode_desc_offset(L, num_heads, plan_units) + (size_t)2 * plan_units * sizeof(int);
}

int decode_kernel_kind(const PoolLayout &L, int num_heads, int requested)
{
    const bool mfma = mfma_decode_supported(L, num_heads);
    if (requested == 0 || !mfma)
        return 0;
    return 1;
}

hipError_t launch_decode(const DecodeArgs &a, hipStream_t st)
{
    const PoolLayout &L = a.L;
    if (a.num_heads % L.num_kv_heads)
        return hipErrorInvalidValue;
    const int n_q = a.n_q > 0 ? a.n_q : 1;
    hipError_t e;
    if (a.plan_units > 0 && n_q == 1 && !a.start_pos && decode_kernel_kind(L, a.num_heads, a.kernel) == 1) {
        e = launch_decode_mfma(a, st);
    } else {
        dim3 grid = a.plan_units > 0 ? dim3(decode_grid_items(a), L.num_kv_heads, 1)
                                     : dim3(1, L.num_kv_heads, a.batch * n_q);
        switch (L.kv_type) {
        case KV_F32: e = launch_valu_kt<KV_F32>(a, grid, st); break;
        case KV_F16: e = launch_valu_kt<KV_F16>(a, grid, st); break;
        case KV_Q4_0: e = launch_valu_kt<KV_Q4_0>(a, grid, st); break;
        default: e = launch_valu_kt<KV_Q8_0>(a, grid, st); break;
        }
    }
    // one unit per kv head covers the whole stream: nothing is split
    if (e != hipSuccess || a.plan_units <= 1)
        return e;
    hipLaunchKernelGGL(merge_splits, dim3(L.num_kv_heads, a.plan_units), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs &p, hipStream_t st)
{
    if (p.chunk_len <= 0 || p.batch <= 0)
        return hipSuccess;
    if (p.kernel != 0 && mfma_prefill_supported(p.L, p.num_heads))
        return launch_prefill_mfma(p, st);
    DecodeArgs a{};
    a.L = p.L;
    a.base = p.base;
    a.q = p.q;
    a.out = p.out;
    a.block_tables = p.block_tables;
    a.max_blocks = p.max_blocks;
    a.seq_lens = nullptr;
    a.batch = p.batch;
    a.n_q = p.chunk_len;
    a.start_pos = p.start_pos;
    a.num_heads = p.num_heads;
    a.scale = p.scale;
    a.plan_units = 0; // one workgroup per (query, kv head), no split
    a.ws = nullptr;
    a.plan_desc = nullptr;
    a.status = p.status;
    a.kernel = 0;
    return launch_decode(a, st);
}

} // namespace gi
