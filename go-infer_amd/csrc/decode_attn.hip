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
    const int split = blockIdx.x, kvh = blockIdx.y, qrow = blockIdx.z;
    const int b = qrow / a.n_q, qi = qrow - b * a.n_q;
    const int tid = threadIdx.x;
    const int H = a.num_heads;
    const int h0 = kvh * G;
    const int P = L.page_tokens;
    int len = a.start_pos ? a.start_pos[b] + qi + 1 : a.seq_lens[b];
    if (len > a.max_blocks * P || len < 0) {
        // More tokens than the block table maps (read what it maps), or a
        // negative length (nothing to read).
        if (tid == 0 && split == 0 && a.status)
            atomicOr(a.status, FLAG_BAD_SLOT);
        len = len < 0 ? 0 : a.max_blocks * P;
    }
    // the last split runs to the end of the sequence, so that a length
    // beyond the one the plan was sized for is still attended in full
    const int t0 = split * a.split_tokens;
    const int t1 = split == a.num_splits - 1 ? len : min(len, t0 + a.split_tokens);
    const int32_t *bt = a.block_tables + (int64_t)b * a.max_blocks;
    const int64_t qbase = (int64_t)qrow * H;

    __shared__ float s_p[G][TOK];
    __shared__ float s_alpha[G];
    __shared__ float s_m[G], s_l[G];
    __shared__ float s_acc[NG][G][HD];

    float *wsp = nullptr;
    if (a.num_splits > 1)
        wsp = a.ws + (((int64_t)qrow * L.num_kv_heads + kvh) * a.num_splits + split) * (G * (HD + 2));

    if (t0 >= t1) {
        // Empty split: partial with m = -inf, l = 0 (or zero output when the
        // whole sequence is empty).
        for (int e = tid; e < G * HD; e += NT) {
            if (wsp)
                wsp[e] = 0.0f;
            else
                a.out[(qbase + h0 + e / HD) * HD + e % HD] = 0.0f;
        }
        if (wsp && tid < G) {
            wsp[G * HD + 2 * tid] = -INFINITY;
            wsp[G * HD + 2 * tid + 1] = 0.0f;
        }
        return;
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
}

// Merges split partials: out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M).
// One workgroup per (query row, head), one thread per output dimension.
__global__ __launch_bounds__(256) void merge_splits(float *__restrict__ out,
                                                    const float *__restrict__ ws, int H, int KVH,
                                                    int HD, int splits)
{
    const int h = blockIdx.x, qrow = blockIdx.y;
    const int G = H / KVH;
    const int kvh = h / G, g = h - kvh * G;
    const int64_t stride = (int64_t)G * (HD + 2);
    const float *w0 = ws + ((int64_t)qrow * KVH + kvh) * splits * stride;
    float M = -INFINITY;
    for (int s = 0; s < splits; s++)
        M = fmaxf(M, w0[s * stride + G * HD + 2 * g]);
    for (int d = threadIdx.x; d < HD; d += blockDim.x) {
        float num = 0.0f, den = 0.0f;
        if (M != -INFINITY) {
            for (int s = 0; s < splits; s++) {
                const float *w = w0 + s * stride;
                const float m = w[G * HD + 2 * g];
                if (m == -INFINITY)
                    continue;
                const float f = expf(m - M);
                num = fmaf(w[g * HD + d], f, num);
                den = fmaf(w[G * HD + 2 * g + 1], f, den);
            }
        }
        out[((int64_t)qrow * H + h) * HD + d] = den > 0.0f ? num / den : 0.0f;
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

size_t decode_workspace_bytes(const PoolLayout &L, int batch, int num_heads, int num_splits)
{
    if (num_splits <= 1)
        return 0;
    const int G = num_heads / L.num_kv_heads;
    return (size_t)batch * L.num_kv_heads * num_splits * G * (L.head_dim + 2) * sizeof(float);
}

// Split-K planning: enough (split, kv head, sequence) workgroups for about
// kDecodeWgPerCu per CU, each split at least kDecodeMinSplit tokens.
// Measured on MI355X: 1 and 1024 beat finer splits (2/1024, 4/512, 8/256,
// 16/128) on 32 ragged sequences of 512-4096 tokens (one workgroup per
// (sequence, kv head), no merge: 2.79 against 2.93 ms per step) and match
// 2/1024 on 8 sequences of 32768, since every workgroup pays a fixed cost
// (query load, cross-wave merge, partials) and a split sequence pays the
// merge launch.  A plan that balances equal token ranges over all
// workgroups regardless of sequence boundaries (with partial slots per range
// and a merge per sequence) measured 2-10% slower on long and uniform
// batches and only 5% faster on ragged ones.
constexpr int kDecodeWgPerCu = 1;
constexpr int kDecodeMinSplit = 1024;

void decode_plan(const PoolLayout &L, int batch, int num_heads, int max_len, int num_cus,
                 int *split_tokens, int *num_splits)
{
    (void)num_heads;
    // Split unit: whole page pairs and a multiple of 64 tokens.
    int unit = 2 * L.page_tokens;
    while (unit % 64)
        unit += 2 * L.page_tokens;
    if (max_len < 1)
        max_len = 1;
    const int64_t pairs = (int64_t)batch * L.num_kv_heads;
    const int64_t target = (int64_t)kDecodeWgPerCu * (num_cus > 0 ? num_cus : 256);
    int splits = (int)((target + pairs - 1) / pairs);
    // A minimum of tokens per split keeps the merge negligible.
    int max_splits = (max_len + kDecodeMinSplit - 1) / kDecodeMinSplit;
    if (splits > max_splits)
        splits = max_splits;
    if (splits < 1)
        splits = 1;
    int per = (max_len + splits - 1) / splits;
    per = (per + unit - 1) / unit * unit;
    splits = (max_len + per - 1) / per;
    *split_tokens = per;
    *num_splits = splits;
}

// Whether a decode step stores its token inside the matrix-core decode
// launch (DecodeArgs.new_k) rather than in an append launch before it:
// when the grid fits the CUs at once (two workgroups each).  Measured
// same-box: batch 32 x U[512, 4096] 2.84 against 2.93 ms per step, 8 x
// 32768 (page 32) 14.64-14.69 against 14.93-14.97, batch 1 (TinyLlama,
// one graph) 5,245 against 4,315 tokens/s; but batch 256 x 8192 (four
// rounds) 42.63-42.96 against 42.09-42.42 ms, the fused launch slower by
// more than the append launch it saves.
bool decode_fuses_append(const PoolLayout &L, int batch, int num_splits, int num_cus)
{
    // one round: as many workgroups as the CUs hold at once (two each)
    const int64_t wgs = (int64_t)batch * L.num_kv_heads * (num_splits > 0 ? num_splits : 1);
    return wgs <= (int64_t)2 * (num_cus > 0 ? num_cus : 256);
}

int decode_waves(const PoolLayout &L, int batch, int num_splits, int num_cus)
{
    const int64_t wgs = (int64_t)batch * L.num_kv_heads * (num_splits > 0 ? num_splits : 1);
    const bool one_round = wgs <= (num_cus > 0 ? num_cus : 256);
    // f32 pages stage HD * 256 bytes per wave in LDS: eight waves at head
    // dimension 64 (128 KiB), four at 128
    if (L.kv_type == KV_F32)
        return one_round && L.head_dim == 64 ? 8 : 4;
    return one_round ? 8 : 4;
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
    if (n_q == 1 && !a.start_pos && decode_kernel_kind(L, a.num_heads, a.kernel) == 1) {
        e = launch_decode_mfma(a, st); // stores a decode step's token itself
    } else {
        if (a.new_k) { // the vector path appends in a launch of its own
            e = launch_append_at_len(L, a.append_base, a.batch, a.block_tables, a.max_blocks, a.seq_lens,
                                     a.new_k, a.new_v, a.status, st);
            if (e != hipSuccess)
                return e;
        }
        dim3 grid(a.num_splits, L.num_kv_heads, a.batch * n_q);
        switch (L.kv_type) {
        case KV_F32: e = launch_valu_kt<KV_F32>(a, grid, st); break;
        case KV_F16: e = launch_valu_kt<KV_F16>(a, grid, st); break;
        case KV_Q4_0: e = launch_valu_kt<KV_Q4_0>(a, grid, st); break;
        default: e = launch_valu_kt<KV_Q8_0>(a, grid, st); break;
        }
    }
    if (e != hipSuccess || a.num_splits <= 1)
        return e;
    hipLaunchKernelGGL(merge_splits, dim3(a.num_heads, a.batch * n_q), dim3(min(L.head_dim, 256)),
                       0, st, a.out, a.ws, a.num_heads, L.num_kv_heads, L.head_dim, a.num_splits);
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
    a.split_tokens = 1 << 30;
    a.num_splits = 1;
    a.ws = nullptr;
    a.status = p.status;
    a.kernel = 0;
    if (p.chunk_len <= 0 || p.batch <= 0)
        return hipSuccess;
    return launch_decode(a, st);
}

} // namespace gi
