// Per-token K/V append into pages and block gather back to the reference's
// contiguous layout.
//
// Append restates, on the page layout of gi_common.h, what the reference does
// when it stores one token vector:
//   f32  : copy            (pkg/engine/kvcache.go:173-178, forward.go:236-240)
//   f16  : FP32ToFP16 per element, truncating (pkg/quant/fp16.go:38-69)
//   q8_0 : QuantizeQ8_0 of the whole kv_dim vector (kvcache.go:152-161,
//          pkg/quant/quant.go:407-456), blocks of 32 never straddle a head
//          because head_dim % 32 == 0.
//   q4_0 : QuantizeQ4_0 likewise (kvcache.go:162-171, quant.go:458-521).
// The fused form applies RoPE (pkg/math/kernels.go:22-35) to q and K first,
// as Forward does before its store (forward.go:228-240, 527-545).
// Gather (KVCache.Get / ForkAt, kvcache.go:183-284) rebuilds tokens [0, n)
// of one sequence from its block table: token t lives at
// (block_table[t / page_tokens], t % page_tokens) (paged_kv.go:107-131).
#include "gi_common.h"
#include "gi_kernels.h"
#include "mfma_ops.h"
#include "token_store.h"

#include <algorithm>

namespace gi {

namespace {

constexpr int kThreads = 256;
using mfma_ops::f4;
using mfma_ops::u2;
using mfma_ops::u4;

__device__ __forceinline__ void raise_flag(int *status, int bit)
{
    if (status)
        atomicOr(status, bit);
}

// Resolves token i's destination page and slot.  Explicit mode reads the
// caller's (block id, slot) arrays, as returned by AppendToken; decode mode
// appends at position seq_lens[i]-1 of sequence i through its block table.
struct Dest {
    const int32_t *block_ids;
    const int32_t *slots;
    const int32_t *block_tables;
    const int32_t *seq_lens;
    int max_blocks;
};

__device__ __forceinline__ bool resolve(const Dest &D, const PoolLayout &L, int i,
                                        int64_t *page, int *slot, int *status)
{
    int64_t p;
    int s;
    if (D.block_ids) {
        p = D.block_ids[i];
        s = D.slots[i];
    } else {
        int len = D.seq_lens[i];
        int pos = len - 1;
        int blk = pos >= 0 ? pos / L.page_tokens : -1;
        if (blk < 0 || blk >= D.max_blocks) {
            raise_flag(status, FLAG_BAD_SLOT);
            return false;
        }
        p = D.block_tables[(int64_t)i * D.max_blocks + blk];
        s = pos % L.page_tokens;
    }
    if (p < 0 || p >= L.num_pages) {
        raise_flag(status, FLAG_BAD_PAGE);
        return false;
    }
    if (s < 0 || s >= L.page_tokens) {
        raise_flag(status, FLAG_BAD_SLOT);
        return false;
    }
    *page = p;
    *slot = s;
    return true;
}

// f32 / f16 append: one thread per (token, element); K and V both.
// AT_LEN selects the decode-step form (position from seq_lens); it only
// names the instance so profiles tell the per-step append from bulk writes.
template <int KT, bool AT_LEN>
__global__ __launch_bounds__(kThreads) void append_plain(PoolLayout L, uint8_t *base, int n_tok,
                                                         Dest D, const float *__restrict__ k,
                                                         const float *__restrict__ v, int *status)
{
    const int hd = L.head_dim;
    const int kv_dim = L.num_kv_heads * hd;
    const int64_t total = (int64_t)n_tok * kv_dim;
    for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * kThreads) {
        int i = (int)(e / kv_dim);
        int j = (int)(e - (int64_t)i * kv_dim);
        int64_t page;
        int s;
        // Every thread of a token resolves the same destination; only the
        // token's first element raises a flag so each bad token counts once.
        int *st = j == 0 ? status : nullptr;
        if (!resolve(D, L, i, &page, &s, st))
            continue;
        const int kvh = j / hd;
        store_token_elem<KT>(L, base + page * L.page_bytes, s, kvh, j - kvh * hd, k[e], v[e], true);
    }
}

// q8_0 append: 32 consecutive threads quantise one block of 32 elements.
template <bool AT_LEN>
__global__ __launch_bounds__(kThreads) void append_q8(PoolLayout L, uint8_t *base, int n_tok,
                                                      Dest D, const float *__restrict__ k,
                                                      const float *__restrict__ v, int *status)
{
    const int hd = L.head_dim;
    const int kv_dim = L.num_kv_heads * hd;
    const int64_t total = (int64_t)n_tok * kv_dim; // multiple of 32
    for (int64_t e0 = (int64_t)blockIdx.x * kThreads; e0 < total;
         e0 += (int64_t)gridDim.x * kThreads) {
        int64_t e = e0 + threadIdx.x;
        // total and kThreads are multiples of 32, so a 32-lane group is
        // either wholly in range or wholly out: the shuffles below see only
        // complete groups.
        if (e >= total)
            break;
        int i = (int)(e / kv_dim);
        int j = (int)(e - (int64_t)i * kv_dim);
        int64_t page = 0;
        int s = 0;
        int *st = j == 0 ? status : nullptr;
        const bool ok = resolve(D, L, i, &page, &s, st);
        const int kvh = j / hd;
        store_token_elem<KV_Q8_0>(L, base + page * L.page_bytes, s, kvh, j - kvh * hd, k[e], v[e], ok);
    }
}

// q4_0 append: 32 consecutive threads quantise one block of 32 elements
// (QuantizeQ4_0 of the whole kv_dim vector, kvcache.go:162-171).
template <bool AT_LEN>
__global__ __launch_bounds__(kThreads) void append_q4(PoolLayout L, uint8_t *base, int n_tok,
                                                      Dest D, const float *__restrict__ k,
                                                      const float *__restrict__ v, int *status)
{
    const int kv_dim = L.num_kv_heads * L.head_dim;
    const int64_t total = (int64_t)n_tok * kv_dim; // multiple of 32
    for (int64_t e0 = (int64_t)blockIdx.x * kThreads; e0 < total;
         e0 += (int64_t)gridDim.x * kThreads) {
        int64_t e = e0 + threadIdx.x;
        // whole 32-lane groups are in or out of range (see append_q8)
        if (e >= total)
            break;
        int i = (int)(e / kv_dim);
        int j = (int)(e - (int64_t)i * kv_dim);
        int64_t page = 0;
        int s = 0;
        bool ok = resolve(D, L, i, &page, &s, j == 0 ? status : nullptr);
        quant_store_q4(L, base + page * L.page_bytes, s, j, k[e], v[e], ok);
    }
}

// Bulk append with explicit destinations (gi_paged_append, a prefill chunk):
// a workgroup takes kRowTok consecutive tokens of one kv head.  Each thread
// converts 4 consecutive elements of one token (a 32-element quantisation
// block is 8 consecutive lanes), writes them into the token's K row, and
// stages their V form in LDS transposed to [row][token]: V pages are
// dimension-major, so written element by element each V store would touch
// its own 32-byte sector.  Then each thread writes 8 tokens of one V row (or
// of one V-scale row) with one store when they sit on consecutive slots of
// one page with the store aligned (the usual chunk append), token by token
// otherwise; neighbouring lanes write the two halves of a 16-token row.
// Bytes are identical to append_plain / append_q8 / append_q4 (the same
// conversion and quantisation code).  head_dim is a multiple of 32 and at
// most kRowMaxHd.
constexpr int kRowTok = 16, kRowMaxHd = 256;

template <int KT>
__global__ __launch_bounds__(kThreads) void append_rows(PoolLayout L, uint8_t *base, int n_tok, Dest D,
                                                        const float *__restrict__ k, const float *__restrict__ v,
                                                        int *status)
{
    const int hd = L.head_dim, P = L.page_tokens, nb = hd / 32;
    const int kv_dim = L.num_kv_heads * hd;
    const int h = blockIdx.y, i0 = blockIdx.x * kRowTok, tid = threadIdx.x;
    const int nt = min(kRowTok, n_tok - i0);
    const int gpt = hd / 4; // 4-element groups per token
    const int ngroups = kRowTok * gpt;
    __shared__ int64_t s_page[kRowTok];
    __shared__ int s_slot[kRowTok];              // -1: token not stored
    __shared__ uint32_t s_v[kRowMaxHd * kRowTok]; // V element bits (or codes, q4 bytes) [row][token]
    __shared__ uint16_t s_vs[kRowMaxHd / 32 * kRowTok]; // V block scales [block][token]

    if (tid < kRowTok) {
        int64_t pg = 0;
        int sl = -1;
        // the kv head 0 workgroup reports each bad token once
        if (tid < nt && !resolve(D, L, i0 + tid, &pg, &sl, h == 0 ? status : nullptr))
            sl = -1;
        s_page[tid] = pg;
        s_slot[tid] = sl;
    }
    __syncthreads();

    // ---- K rows, and V converted into LDS ----
    for (int g0 = 0; g0 < ngroups; g0 += kThreads) {
        // whole 8-lane groups (one quantisation block) are in or out of range
        const int g = g0 + tid;
        const int t = g / gpt, a4 = g - t * gpt, d0 = 4 * a4, blk = a4 >> 3, a = a4 & 7;
        const bool in = g < ngroups && t < nt;
        f4 kx = f4{0.0f, 0.0f, 0.0f, 0.0f}, vx = kx;
        if (in) {
            const int64_t e = (int64_t)(i0 + t) * kv_dim + (int64_t)h * hd + d0;
            kx = *reinterpret_cast<const f4 *>(k + e);
            vx = *reinterpret_cast<const f4 *>(v + e);
        }
        const int sl = g < ngroups ? s_slot[t] : -1;
        uint8_t *pg = base + (g < ngroups ? s_page[t] : 0) * L.page_bytes;
        const bool st = in && sl >= 0;
        const int64_t krow = (int64_t)h * P + sl; // K row of the token
        uint32_t vb[4];                            // V element bits / codes for s_v
        if constexpr (KT == KV_F32) {
            if (st)
                *reinterpret_cast<f4 *>(pg + L.k_off + (krow * hd + d0) * 4) = kx;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                // (copied out before the bit cast: hipcc's __builtin_bit_cast
                // of a vector element reads element 0 whatever the index)
                const float x = vx[c];
                vb[c] = __builtin_bit_cast(uint32_t, x);
            }
        } else if constexpr (KT == KV_F16) {
            uint32_t kh[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                kh[c] = float_to_half_bits_rtz(kx[c]);
                vb[c] = float_to_half_bits_rtz(vx[c]);
            }
            if (st)
                *reinterpret_cast<u2 *>(pg + L.k_off + (krow * hd + d0) * 2) =
                    u2{kh[0] | (kh[1] << 16), kh[2] | (kh[3] << 16)};
        } else {
            uint32_t kk = 0, vk = 0;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                kk = max(kk, abs_key(kx[c]));
                vk = max(vk, abs_key(vx[c]));
            }
#pragma unroll
            for (int m = 1; m < 8; m <<= 1) {
                kk = max(kk, (uint32_t)__shfl_xor((int)kk, m, 8));
                vk = max(vk, (uint32_t)__shfl_xor((int)vk, m, 8));
            }
            float kinv, vinv;
            const bool q8 = KT == KV_Q8_0;
            const uint32_t kd = q8 ? q8_scale(__builtin_bit_cast(float, kk), &kinv)
                                   : q4_scale(__builtin_bit_cast(float, kk), &kinv);
            const uint32_t vd = q8 ? q8_scale(__builtin_bit_cast(float, vk), &vinv)
                                   : q4_scale(__builtin_bit_cast(float, vk), &vinv);
            if (q8) {
                uint32_t kw = 0;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    kw |= ((uint32_t)q8_quant(kx[c], kinv) & 0xFFu) << (8 * c);
                    vb[c] = (uint32_t)q8_quant(vx[c], vinv) & 0xFFu;
                }
                if (st)
                    *reinterpret_cast<uint32_t *>(pg + L.k_off + krow * hd + d0) = kw;
                if (st && a == 0)
                    reinterpret_cast<uint16_t *>(pg + L.ks_off)[krow * nb + blk] = (uint16_t)kd;
            } else {
                // byte j of a block holds element j (low nibble) and j + 16
                // (high): lanes a < 4 take the high nibbles of lane a + 4
                uint32_t kn = 0, vn = 0;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    kn |= (uint32_t)q4_quant(kx[c], kinv) << (8 * c);
                    vn |= (uint32_t)q4_quant(vx[c], vinv) << (8 * c);
                }
                const uint32_t kh = (uint32_t)__shfl_down((int)kn, 4, 8);
                const uint32_t vh = (uint32_t)__shfl_down((int)vn, 4, 8);
                const uint32_t kw = kn | (kh << 4), vw = vn | (vh << 4);
                if (st && a < 4)
                    *reinterpret_cast<uint32_t *>(pg + L.k_off + (krow * nb + blk) * 16 + 4 * a) = kw;
                if (st && a == 0)
                    reinterpret_cast<uint16_t *>(pg + L.ks_off)[krow * nb + blk] = (uint16_t)kd;
#pragma unroll
                for (int c = 0; c < 4; c++)
                    vb[c] = (vw >> (8 * c)) & 0xFFu;
            }
            if (g < ngroups && a == 0)
                s_vs[blk * kRowTok + t] = (uint16_t)vd;
        }
        if (g < ngroups) {
            if (KT == KV_Q4_0) {
                if (a < 4) // byte rows 4a .. 4a + 3 of block blk
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        s_v[(blk * 16 + 4 * a + c) * kRowTok + t] = vb[c];
            } else {
#pragma unroll
                for (int c = 0; c < 4; c++)
                    s_v[(d0 + c) * kRowTok + t] = vb[c];
            }
        }
    }
    __syncthreads();

    // ---- V rows and V-scale rows, 8 tokens per task ----
    constexpr int ESZ = KT == KV_F32 ? 4 : KT == KV_F16 ? 2 : 1;
    const int vrows = KT == KV_Q4_0 ? hd / 2 : hd;
    const bool quant = KT == KV_Q8_0 || KT == KV_Q4_0;
    const int ntask = (vrows + (quant ? nb : 0)) * (kRowTok / 8);
    for (int task = tid; task < ntask; task += kThreads) {
        const int row = task / (kRowTok / 8), t0 = 8 * (task % (kRowTok / 8));
        const bool scale_row = row >= vrows; // quantised pages: V-scale row of block row - vrows
        const int64_t off = scale_row ? L.vs_off + (((int64_t)h * nb + (row - vrows)) * P) * 2
                                      : L.v_off + (((int64_t)h * vrows + row) * P) * ESZ;
        const int esz = scale_row ? 2 : ESZ;
        // one store when the 8 tokens are consecutive slots of one page
        const int s0 = s_slot[t0];
        bool run = s0 >= 0;
#pragma unroll
        for (int t = 1; t < 8; t++)
            run = run && s_slot[t0 + t] == s0 + t && s_page[t0 + t] == s_page[t0];
        uint8_t *dst0 = base + s_page[t0] * L.page_bytes + off + (int64_t)s0 * esz;
        run = run && ((uintptr_t)dst0 & (uintptr_t)(8 * esz - 1)) == 0;
        uint32_t x[8];
#pragma unroll
        for (int t = 0; t < 8; t++)
            x[t] = scale_row ? (uint32_t)s_vs[(row - vrows) * kRowTok + t0 + t] : s_v[row * kRowTok + t0 + t];
        if (run) {
            if (esz == 4) {
                reinterpret_cast<u4 *>(dst0)[0] = u4{x[0], x[1], x[2], x[3]};
                reinterpret_cast<u4 *>(dst0)[1] = u4{x[4], x[5], x[6], x[7]};
            } else if (esz == 2) {
                *reinterpret_cast<u4 *>(dst0) =
                    u4{x[0] | (x[1] << 16), x[2] | (x[3] << 16), x[4] | (x[5] << 16), x[6] | (x[7] << 16)};
            } else {
                *reinterpret_cast<u2 *>(dst0) = u2{x[0] | (x[1] << 8) | (x[2] << 16) | (x[3] << 24),
                                                   x[4] | (x[5] << 8) | (x[6] << 16) | (x[7] << 24)};
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int s = s_slot[t0 + t];
                if (s < 0)
                    continue;
                uint8_t *d = base + s_page[t0 + t] * L.page_bytes + off + (int64_t)s * esz;
                if (esz == 4)
                    *reinterpret_cast<uint32_t *>(d) = x[t];
                else if (esz == 2)
                    *reinterpret_cast<uint16_t *>(d) = (uint16_t)x[t];
                else
                    *d = (uint8_t)x[t];
            }
        }
    }
}

// Gather one sequence's tokens [0, n_tok) of one layer.
//   widen == 0: stored format, the reference's bytes per token vector
//               (f32: 4*kv_dim, f16: 2*kv_dim, q8_0: kv_dim/32 blocks of
//               34 bytes = LE fp16 scale + 32 int8, quant.go:38-41).
//   widen == 1: float32 values (FP16ToFP32 / DequantizeQ8_0).
template <int KT, int WIDEN>
__global__ __launch_bounds__(kThreads) void gather_kernel(PoolLayout L, const uint8_t *base,
                                                          const int32_t *__restrict__ table,
                                                          int n_tok, uint8_t *kout, uint8_t *vout,
                                                          int *status)
{
    const int hd = L.head_dim;
    const int kv_dim = L.num_kv_heads * hd;
    const int P = L.page_tokens;
    const int nb = hd / 32;
    // Units per token: one per element, except raw q8_0 / q4_0: one per byte.
    const int per_tok = (KT == KV_Q8_0 && !WIDEN) ? (kv_dim / 32) * 34
                        : (KT == KV_Q4_0 && !WIDEN) ? (kv_dim / 32) * 18
                                                    : kv_dim;
    const int64_t total = (int64_t)n_tok * per_tok;
    for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * kThreads) {
        int t = (int)(e / per_tok);
        int u = (int)(e - (int64_t)t * per_tok);
        int64_t page = table[t / P];
        int s = t % P;
        if (page < 0 || page >= L.num_pages) {
            if (u == 0)
                raise_flag(status, FLAG_BAD_PAGE);
            continue;
        }
        const uint8_t *pg = base + page * L.page_bytes;
        if (KT == KV_Q4_0) {
            // 18-byte blocks: LE fp16 scale, then byte j = dim j | dim j+16 << 4
            int b, r;
            if (WIDEN) {
                b = u >> 5;
                r = 2 + (u & 15); // the byte holding dim u & 31
            } else {
                b = u / 18;
                r = u - b * 18;
            }
            const int kvh = b / nb, blk = b - kvh * nb;
            const uint16_t ks = reinterpret_cast<const uint16_t *>(pg + L.ks_off)[((int64_t)kvh * P + s) * nb + blk];
            const uint16_t vs = reinterpret_cast<const uint16_t *>(pg + L.vs_off)[((int64_t)kvh * nb + blk) * P + s];
            uint8_t kb = 0, vb = 0;
            if (r >= 2) {
                kb = pg[L.k_off + (((int64_t)kvh * P + s) * nb + blk) * 16 + (r - 2)];
                vb = pg[L.v_off + (((int64_t)kvh * nb + blk) * 16 + (r - 2)) * P + s];
            }
            if (WIDEN) { // (nibble - 8) * d (quant.go:103-110)
                const int sh = (u & 16) ? 4 : 0;
                reinterpret_cast<float *>(kout)[e] = (float)(((kb >> sh) & 15) - 8) * half_bits_to_float(ks);
                reinterpret_cast<float *>(vout)[e] = (float)(((vb >> sh) & 15) - 8) * half_bits_to_float(vs);
            } else {
                kout[e] = r == 0 ? (uint8_t)(ks & 0xFF) : r == 1 ? (uint8_t)(ks >> 8) : kb;
                vout[e] = r == 0 ? (uint8_t)(vs & 0xFF) : r == 1 ? (uint8_t)(vs >> 8) : vb;
            }
            continue;
        }
        if (KT == KV_Q8_0 && !WIDEN) {
            int b = u / 34, r = u - b * 34; // global 32-block index and byte
            int kvh = b / nb, blk = b - kvh * nb;
            uint8_t kb, vb;
            if (r < 2) {
                uint16_t ks = reinterpret_cast<const uint16_t *>(pg + L.ks_off)
                    [((int64_t)kvh * P + s) * nb + blk];
                uint16_t vs = reinterpret_cast<const uint16_t *>(pg + L.vs_off)
                    [((int64_t)kvh * nb + blk) * P + s];
                kb = (uint8_t)(r == 0 ? ks & 0xFF : ks >> 8);
                vb = (uint8_t)(r == 0 ? vs & 0xFF : vs >> 8);
            } else {
                int d = blk * 32 + (r - 2);
                kb = (pg + L.k_off)[((int64_t)kvh * P + s) * hd + d];
                vb = (pg + L.v_off)[((int64_t)kvh * hd + d) * P + s];
            }
            kout[e] = kb;
            vout[e] = vb;
            continue;
        }
        int kvh = u / hd;
        int d = u - kvh * hd;
        int64_t ki = ((int64_t)kvh * P + s) * hd + d;
        int64_t vi = ((int64_t)kvh * hd + d) * P + s;
        if (KT == KV_F32) {
            reinterpret_cast<float *>(kout)[e] = reinterpret_cast<const float *>(pg + L.k_off)[ki];
            reinterpret_cast<float *>(vout)[e] = reinterpret_cast<const float *>(pg + L.v_off)[vi];
        } else if (KT == KV_F16) {
            uint16_t kh = reinterpret_cast<const uint16_t *>(pg + L.k_off)[ki];
            uint16_t vh = reinterpret_cast<const uint16_t *>(pg + L.v_off)[vi];
            if (WIDEN) {
                reinterpret_cast<float *>(kout)[e] = half_bits_to_float(kh);
                reinterpret_cast<float *>(vout)[e] = half_bits_to_float(vh);
            } else {
                reinterpret_cast<uint16_t *>(kout)[e] = kh;
                reinterpret_cast<uint16_t *>(vout)[e] = vh;
            }
        } else { // q8_0 widened: float32(int8 q) * FP16ToFP32(d) (quant.go:207)
            int blk = d >> 5;
            float ks = half_bits_to_float(reinterpret_cast<const uint16_t *>(pg + L.ks_off)
                                              [((int64_t)kvh * P + s) * nb + blk]);
            float vs = half_bits_to_float(reinterpret_cast<const uint16_t *>(pg + L.vs_off)
                                              [((int64_t)kvh * nb + blk) * P + s]);
            int8_t kq = reinterpret_cast<const int8_t *>(pg + L.k_off)[ki];
            int8_t vq = reinterpret_cast<const int8_t *>(pg + L.v_off)[vi];
            reinterpret_cast<float *>(kout)[e] = (float)kq * ks;
            reinterpret_cast<float *>(vout)[e] = (float)vq * vs;
        }
    }
}

int grid_for(int64_t units)
{
    int64_t g = (units + kThreads - 1) / kThreads;
    if (g > 65536)
        g = 65536;
    return g < 1 ? 1 : (int)g;
}

hipError_t append_any(const PoolLayout &L, uint8_t *base, int n_tok, const Dest &D,
                      const float *k, const float *v, int *status, hipStream_t st)
{
    if (n_tok <= 0)
        return hipSuccess;
    const bool at_len = D.block_ids == nullptr;
    // the row kernel reads K/V 16 bytes at a time: inputs of any other
    // alignment (a caller's float pointer) take the per-element kernels
    const bool aligned16 = ((uintptr_t)k % 16 == 0) && ((uintptr_t)v % 16 == 0);
    if (!at_len && aligned16 && L.head_dim % 32 == 0 && L.head_dim <= kRowMaxHd) {
        dim3 rgrid((unsigned)((n_tok + kRowTok - 1) / kRowTok), (unsigned)L.num_kv_heads);
#define GI_ROWS(KT) hipLaunchKernelGGL((append_rows<KT>), rgrid, dim3(kThreads), 0, st, L, base, n_tok, D, k, v, status)
        switch (L.kv_type) {
        case KV_F32:
            GI_ROWS(KV_F32);
            break;
        case KV_F16:
            GI_ROWS(KV_F16);
            break;
        case KV_Q4_0:
            GI_ROWS(KV_Q4_0);
            break;
        default:
            GI_ROWS(KV_Q8_0);
            break;
        }
#undef GI_ROWS
        return hipGetLastError();
    }
    int64_t units = (int64_t)n_tok * L.num_kv_heads * L.head_dim;
    dim3 grid(grid_for(units)), block(kThreads);
#define GI_APPEND(KERNEL)                                                                    \
    hipLaunchKernelGGL(KERNEL, grid, block, 0, st, L, base, n_tok, D, k, v, status)
    switch (L.kv_type) {
    case KV_F32:
        if (at_len)
            GI_APPEND((append_plain<KV_F32, true>));
        else
            GI_APPEND((append_plain<KV_F32, false>));
        break;
    case KV_F16:
        if (at_len)
            GI_APPEND((append_plain<KV_F16, true>));
        else
            GI_APPEND((append_plain<KV_F16, false>));
        break;
    case KV_Q4_0:
        if (at_len)
            GI_APPEND(append_q4<true>);
        else
            GI_APPEND(append_q4<false>);
        break;
    default:
        if (at_len)
            GI_APPEND(append_q8<true>);
        else
            GI_APPEND(append_q8<false>);
        break;
    }
#undef GI_APPEND
    return hipGetLastError();
}

// One rotated pair of ApplyRoPE (kernels.go:31-33): each product is rounded
// before the sum or difference, as Go's amd64 code evaluates it, so no
// multiply-add may be contracted here.
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float *y0, float *y1)
{
#pragma clang fp contract(off)
    float a = x0 * c;
    float b = x1 * s;
    float e = x0 * s;
    float f = x1 * c;
    *y0 = a - b;
    *y1 = e + f;
}

// Rotates the first 2*rh dims of each of n_heads heads of x (head stride hd)
// into y; the dims past 2*rh are copied.  Pair p = (head, j) is (j, j + rh)
// of that head.  Pairs [p0, p0 + step * k) go to the threads of the
// workgroup in turn, and y may alias x: every element is read and written
// by the one thread that owns its pair.
__device__ __forceinline__ void rope_rows(const float *x, float *y, int n_heads, int hd, int rh,
                                          const float2 *cs, int p0, int step)
{
    for (int p = p0 + threadIdx.x; p < n_heads * rh; p += step) {
        int h = p / rh, j = p - h * rh;
        const float *xh = x + (int64_t)h * hd;
        float *yh = y + (int64_t)h * hd;
        float2 t = cs[j];
        float y0, y1;
        rope_pair(xh[j], xh[j + rh], t.x, t.y, &y0, &y1);
        yh[j] = y0;
        yh[j + rh] = y1;
    }
    const int rest = hd - 2 * rh;
    if (rest > 0) {
        for (int p = p0 + threadIdx.x; p < n_heads * rest; p += step) {
            int h = p / rest, j = 2 * rh + (p - h * rest);
            y[(int64_t)h * hd + j] = x[(int64_t)h * hd + j];
        }
    }
}

// Fused RoPE + append.  Grid (n_tok, 1 + q_blocks): block (i, 0) turns
// token i's K into LDS and stores K (in the pool's format: f32 copy,
// truncated fp16, or Q8_0 blocks of the rotated vector) and V; block
// (i, 1 + b) turns kThreads pairs of token i's q into q_out, one pair per
// thread, so no thread waits on a chain of dependent loads.  A token whose
// position is outside the table is skipped whole (its q_out row is not
// written); one whose page or slot is bad has its q turned but nothing
// stored.
template <int KT, bool AT_LEN>
__global__ __launch_bounds__(kThreads) void rope_append(PoolLayout L, uint8_t *base, Dest D, RopeArgs R,
                                                        const float *__restrict__ k,
                                                        const float *__restrict__ v, int *status)
{
    extern __shared__ float sk[]; // kv_dim rotated K values
    const int i = blockIdx.x;
    const int hd = L.head_dim;
    const int kv_dim = L.num_kv_heads * hd;
    const int pos = AT_LEN ? D.seq_lens[i] - 1 : R.positions[i];
    if (pos < 0 || pos >= R.max_pos) {
        if (threadIdx.x == 0 && blockIdx.y == 0)
            raise_flag(status, FLAG_BAD_POS);
        return;
    }
    const float2 *cs = R.table + (int64_t)pos * R.rope_half;
    if (blockIdx.y > 0) {
        const int64_t qo = (int64_t)i * R.num_heads * hd;
        const int nqb = gridDim.y - 1;
        rope_rows(R.q + qo, R.q_out + qo, R.num_heads, hd, R.rope_half, cs,
                  (int)(blockIdx.y - 1) * kThreads, nqb * kThreads);
        return;
    }
    const float *kx = k + (int64_t)i * kv_dim;
    const float *vx = v + (int64_t)i * kv_dim;
    rope_rows(kx, sk, L.num_kv_heads, hd, R.rope_half, cs, 0, kThreads);
    __syncthreads();
    int64_t page;
    int s;
    // every thread resolves the same destination; thread 0 reports
    if (!resolve(D, L, i, &page, &s, threadIdx.x == 0 ? status : nullptr))
        return;
    uint8_t *pg = base + page * L.page_bytes;
    const int P = L.page_tokens;
    if (KT == KV_Q4_0) {
        // 32-lane groups are whole blocks in every iteration (see below)
        for (int e = threadIdx.x; e < kv_dim; e += kThreads)
            quant_store_q4(L, pg, s, e, sk[e], vx[e], true);
        return;
    }
    if (KT == KV_Q8_0) {
        const int nb = hd / 32;
        // kv_dim and kThreads are multiples of 32: a 32-lane group (one
        // Q8_0 block) is wholly in or out of range in every iteration.
        for (int e = threadIdx.x; e < kv_dim; e += kThreads) {
            float kv0 = sk[e], vv0 = vx[e];
            float kinv, vinv;
            uint32_t kd = q8_scale(__builtin_bit_cast(float, max32(abs_key(kv0))), &kinv);
            uint32_t vd = q8_scale(__builtin_bit_cast(float, max32(abs_key(vv0))), &vinv);
            int kvh = e / hd, d = e - kvh * hd, blk = d >> 5;
            reinterpret_cast<int8_t *>(pg + L.k_off)[((int64_t)kvh * P + s) * hd + d] = (int8_t)q8_quant(kv0, kinv);
            reinterpret_cast<int8_t *>(pg + L.v_off)[((int64_t)kvh * hd + d) * P + s] = (int8_t)q8_quant(vv0, vinv);
            if ((d & 31) == 0) {
                reinterpret_cast<uint16_t *>(pg + L.ks_off)[((int64_t)kvh * P + s) * nb + blk] = (uint16_t)kd;
                reinterpret_cast<uint16_t *>(pg + L.vs_off)[((int64_t)kvh * nb + blk) * P + s] = (uint16_t)vd;
            }
        }
        return;
    }
    for (int e = threadIdx.x; e < kv_dim; e += kThreads) {
        int kvh = e / hd, d = e - kvh * hd;
        int64_t ki = ((int64_t)kvh * P + s) * hd + d;
        int64_t vi = ((int64_t)kvh * hd + d) * P + s;
        if (KT == KV_F32) {
            reinterpret_cast<float *>(pg + L.k_off)[ki] = sk[e];
            reinterpret_cast<float *>(pg + L.v_off)[vi] = vx[e];
        } else {
            reinterpret_cast<uint16_t *>(pg + L.k_off)[ki] = (uint16_t)float_to_half_bits_rtz(sk[e]);
            reinterpret_cast<uint16_t *>(pg + L.v_off)[vi] = (uint16_t)float_to_half_bits_rtz(vx[e]);
        }
    }
}

} // namespace

hipError_t launch_append(const PoolLayout &L, uint8_t *base, int n_tok, const int32_t *block_ids,
                         const int32_t *slots, const float *k, const float *v, int *status,
                         hipStream_t st)
{
    Dest D{block_ids, slots, nullptr, nullptr, 0};
    return append_any(L, base, n_tok, D, k, v, status, st);
}

hipError_t launch_append_at_len(const PoolLayout &L, uint8_t *base, int batch,
                                const int32_t *block_tables, int max_blocks,
                                const int32_t *seq_lens, const float *k, const float *v,
                                int *status, hipStream_t st)
{
    Dest D{nullptr, nullptr, block_tables, seq_lens, max_blocks};
    return append_any(L, base, batch, D, k, v, status, st);
}

hipError_t launch_rope_append(const PoolLayout &L, uint8_t *base, int n_tok, const int32_t *block_ids,
                              const int32_t *slots, const int32_t *block_tables, int max_blocks,
                              const int32_t *seq_lens, const RopeArgs &R, const float *k,
                              const float *v, int *status, hipStream_t st)
{
    if (n_tok <= 0)
        return hipSuccess;
    Dest D{block_ids, slots, block_tables, seq_lens, max_blocks};
    const bool at_len = block_ids == nullptr;
    const size_t lds = sizeof(float) * (size_t)L.num_kv_heads * L.head_dim;
    // q blocks: one rotated pair (or copied dim past rope_dim) per thread
    const int64_t q_units = (int64_t)R.num_heads *
                            std::max(R.rope_half, L.head_dim - 2 * R.rope_half);
    const int nqb = (int)((q_units + kThreads - 1) / kThreads);
    dim3 grid((unsigned)n_tok, (unsigned)(1 + nqb)), block(kThreads);
#define GI_ROPE(KT)                                                                                \
    do {                                                                                           \
        if (at_len)                                                                                \
            hipLaunchKernelGGL((rope_append<KT, true>), grid, block, lds, st, L, base, D, R, k, v, \
                               status);                                                            \
        else                                                                                       \
            hipLaunchKernelGGL((rope_append<KT, false>), grid, block, lds, st, L, base, D, R, k,   \
                               v, status);                                                         \
    } while (0)
    switch (L.kv_type) {
    case KV_F32:
        GI_ROPE(KV_F32);
        break;
    case KV_F16:
        GI_ROPE(KV_F16);
        break;
    case KV_Q4_0:
        GI_ROPE(KV_Q4_0);
        break;
    default:
        GI_ROPE(KV_Q8_0);
        break;
    }
#undef GI_ROPE
    return hipGetLastError();
}

hipError_t launch_gather(const PoolLayout &L, const uint8_t *base, const int32_t *table, int n_tok,
                         void *k_out, void *v_out, int widen, int *status, hipStream_t st)
{
    if (n_tok <= 0)
        return hipSuccess;
    int kv_dim = L.num_kv_heads * L.head_dim;
    int64_t per_tok = (L.kv_type == KV_Q8_0 && !widen) ? (kv_dim / 32) * 34
                      : (L.kv_type == KV_Q4_0 && !widen) ? (kv_dim / 32) * 18
                                                         : kv_dim;
    dim3 grid(grid_for((int64_t)n_tok * per_tok)), block(kThreads);
    uint8_t *ko = (uint8_t *)k_out, *vo = (uint8_t *)v_out;
#define GI_GATHER(KT, W) \
    hipLaunchKernelGGL((gather_kernel<KT, W>), grid, block, 0, st, L, base, table, n_tok, ko, vo, status)
    if (L.kv_type == KV_F32) {
        GI_GATHER(KV_F32, 0);
    } else if (L.kv_type == KV_F16) {
        if (widen)
            GI_GATHER(KV_F16, 1);
        else
            GI_GATHER(KV_F16, 0);
    } else if (L.kv_type == KV_Q4_0) {
        if (widen)
            GI_GATHER(KV_Q4_0, 1);
        else
            GI_GATHER(KV_Q4_0, 0);
    } else {
        if (widen)
            GI_GATHER(KV_Q8_0, 1);
        else
            GI_GATHER(KV_Q8_0, 0);
    }
#undef GI_GATHER
    return hipGetLastError();
}

namespace {

// Page copy: grid (chunks, pairs, layers), 16 bytes per thread and step.
// Pairs with an id outside the pool are skipped and flagged.
__global__ __launch_bounds__(kThreads) void copy_pages_kernel(uint8_t *const *layer_base, int64_t page_bytes,
                                                              int64_t num_pages, const int32_t *src,
                                                              const int32_t *dst, int *status)
{
    const int pair = blockIdx.y, layer = blockIdx.z;
    const int64_t s = src[pair], d = dst[pair];
    if (s < 0 || s >= num_pages || d < 0 || d >= num_pages) {
        if (blockIdx.x == 0 && threadIdx.x == 0 && status)
            atomicOr(status, FLAG_BAD_PAGE);
        return;
    }
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    uint8_t *base = layer_base[layer];
    const u4 *sp = reinterpret_cast<const u4 *>(base + s * page_bytes);
    u4 *dp = reinterpret_cast<u4 *>(base + d * page_bytes);
    const int64_t n16 = page_bytes / 16;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n16; i += (int64_t)gridDim.x * kThreads)
        dp[i] = sp[i];
}

} // namespace

hipError_t launch_copy_pages(const PoolLayout &L, uint8_t *const *layer_base, int n, const int32_t *src,
                             const int32_t *dst, int *status, hipStream_t st)
{
    if (n <= 0)
        return hipSuccess;
    const int64_t n16 = L.page_bytes / 16;
    const unsigned gx = (unsigned)std::min<int64_t>((n16 + kThreads - 1) / kThreads, 64);
    for (int i0 = 0; i0 < n; i0 += 65535) { // grid y limit
        const int cnt = std::min(n - i0, 65535);
        hipLaunchKernelGGL(copy_pages_kernel, dim3(gx, (unsigned)cnt, (unsigned)L.num_layers), dim3(kThreads),
                           0, st, layer_base, L.page_bytes, L.num_pages, src + i0, dst + i0, status);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            return e;
    }
    return hipSuccess;
}

} // namespace gi
