// Weight matrix times a batch of activations on the matrix cores: the
// O-projection that follows attention (pkg/engine/forward.go:270 and 580,
// Weights.MatMul / MatMulBatch, pkg/engine/weights.go:237-350), for weights
// of GGML type F32, F16, Q8_0 or Q4_0.
//
//   y[b][r] = sum_c W[r][c] * x[b][c]      (pkg/math/gemv.go, metal.MatMulBatch,
//                                            pkg/metal/metal_darwin.go:849-880)
//
// Weights are converted once (gi_weights_upload) from their GGUF layout into
// operand order, and activations are split into it on every call, so that
// each 16-byte operand load of a wave reads one contiguous 1 KiB run (a
// row-major load would send every quarter-wave to 16 rows, and the L1 tag
// rate -- one line per lane -- bounds that form):
//   16-bit weight matrices (F16, the F32 halves): the 16 x 32 tile (rows
//   16t.., columns 32kk..) is 512 elements in lane order, lane
//   16 * ((c / 8) % 4) + r % 16 holding columns 8 ((c / 8) % 4) .. +7 of its
//   row (op_index);
//   activation halves: the same tiles, each row-major (x_index), which the
//   direct loads permute into lane order;
//   Q8_0  int8 codes in the same order (512 bytes per tile), fp16 block
//         scales [cols/32][rows_pad];
//   Q4_0  per tile and block, the 16 nibble bytes of each of the 16 rows
//         (byte j holds elements j and j+16, quant.go:504), 256 bytes;
//         scales as Q8_0;
//   F32   two fp16 halves, hi and lo, of W * 2^e[r] (e[r] from the row's
//         largest |w|, so both halves stay normal), and 2^-e[r] per row.
// Rows of weights are padded with zeros to multiples of 128 and those of
// activations to multiples of 64, so the product loops need no bounds checks.
//
// Activations are split per batch row into fp16 hi + lo of x * 2^e[b], so the
// products keep float32 accuracy.  The matrix cores then compute W * x^T on
// 16x16x32 f16 tiles: quantised codes are exact fp16 values, and one 32-wide
// k-step is exactly one quantisation block, so each k-step's partial product
// is scaled by its block scale in float32 (DotVecQ8_0 / DotVecQ4_0 sum a
// block, then multiply by d).  F32 weights take three products (hi*hi, hi*lo,
// lo*hi).
//
// Two forms of the product:
//   * matmul_lds (quantised weights, and batches under 128): a workgroup owns
//     a 64 x 64 (rows x batch) output tile.  Its four waves take every fourth
//     k-step each, and each wave streams its k-steps through its own LDS
//     stages by direct global->LDS loads, two steps ahead (one for F32, whose
//     stages are twice as large).  Waves 1-3 then leave their partial tiles
//     in LDS and wave 0 adds them to its own, so one launch covers the
//     product with no global reduction.
//   * matmul_sk (F16 and F32 weights, batches of 128 and more): 128 x 128
//     tiles over slices of the k-steps, the slices' partial tiles added by
//     reduce_splits (described at the kernel).
#include "../../include/goinfer_paged.h"
#include "gi_common.h"
#include "devbuf.h"
#include "mfma_ops.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <new>
#include <string>
#include <type_traits>
#include <utility>

namespace gi {
namespace {

using mfma_ops::f4;
using mfma_ops::h8;
using mfma_ops::i8x8_to_h8;
using mfma_ops::mfma16;
using mfma_ops::u2;
using mfma_ops::u4x8_to_h8;

enum : int { W_F32 = 0, W_F16 = 1, W_Q4_0 = 2, W_Q8_0 = 8 }; // GGML type ids



// Activation rows are padded to multiples of 64, the batch side of the
// 64 x 64 output tile; weight rows to multiples of 128, the row side of the
// split-K tile (and so of 64 too).
__host__ __device__ __forceinline__ int64_t round_pad(int64_t n) { return (n + 63) / 64 * 64; }
__host__ __device__ __forceinline__ int64_t weight_rows_pad(int64_t n) { return (n + 127) / 128 * 128; }

// Element (r, c) of a 16-bit matrix (or an int8 code matrix) with KS
// k-steps of 32 columns, in operand order.
__host__ __device__ __forceinline__ int64_t op_index(int64_t r, int c, int KS)
{
    return (((r >> 4) * KS + (c >> 5)) * 64 + 16 * ((c >> 3) & 3) + (r & 15)) * 8 + (c & 7);
}

// Element (b, c) of the activation halves: each 16 x 32 tile row-major
// (16 rows of 64 bytes), so that one batch row's k-step is one 64-byte run
// when it is written.  The direct loads read a tile's 1 KiB whole and permute
// it into lane order (operand order) on the way into LDS.
__host__ __device__ __forceinline__ int64_t x_index(int64_t b, int c, int KS)
{
    return (((b >> 4) * KS + (c >> 5)) * 16 + (b & 15)) * 32 + (c & 31);
}

// Byte i of row r's Q4_0 block kk.
__host__ __device__ __forceinline__ int64_t q4_index(int64_t r, int kk, int i, int KS)
{
    return (((r >> 4) * KS + kk) * 16 + (r & 15)) * 16 + i;
}

// ---- conversion of GGUF weights into the operand layout ------------------

// Q8_0 / Q4_0: one thread per (row, block) of the padded rows; raw blocks
// are byte-addressed.
__global__ __launch_bounds__(256) void convert_quant(const uint8_t *__restrict__ raw, int type, int rows,
                                                    int rows_pad, int cols, uint8_t *__restrict__ codes,
                                                    uint16_t *__restrict__ scales)
{
    const int nb = cols / 32;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows_pad * nb)
        return;
    const int r = (int)(i / nb), kb = (int)(i - (int64_t)r * nb);
    const bool live = r < rows;
    const int bb = type == W_Q8_0 ? 34 : 18;
    const uint8_t *blk = raw + (live ? i : 0) * bb;
    scales[(int64_t)kb * rows_pad + r] = live ? (uint16_t)(blk[0] | (blk[1] << 8)) : 0;
    if (type == W_Q8_0) {
        for (int j = 0; j < 32; j++)
            codes[op_index(r, 32 * kb + j, nb)] = live ? blk[2 + j] : 0;
    } else {
        for (int j = 0; j < 16; j++)
            codes[q4_index(r, kb, j, nb)] = live ? blk[2 + j] : 0x88; // padded rows: codes 8 (zero)
    }
}

// F16: one thread per 8 consecutive elements of the padded rows.
__global__ __launch_bounds__(256) void convert_f16(const uint16_t *__restrict__ raw, int rows, int rows_pad, int cols,
                                                  uint16_t *__restrict__ dst)
{
    const int per = cols / 8;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows_pad * per)
        return;
    const int r = (int)(i / per), c = 8 * (int)(i - (int64_t)r * per);
    uint4 v = {0u, 0u, 0u, 0u};
    if (r < rows)
        v = *reinterpret_cast<const uint4 *>(raw + (int64_t)r * cols + c);
    *reinterpret_cast<uint4 *>(dst + op_index(r, c, cols / 32)) = v;
}

// F32: one workgroup per padded row; W * 2^e split into hi + lo fp16.
__global__ __launch_bounds__(256) void convert_f32(const float *__restrict__ raw, int rows, int cols,
                                                  _Float16 *__restrict__ hi, _Float16 *__restrict__ lo,
                                                  float *__restrict__ row_scale)
{
    __shared__ float s_max[256];
    const int r = blockIdx.x, KS = cols / 32;
    if (r >= rows) {
        for (int c = threadIdx.x; c < cols; c += 256) {
            hi[op_index(r, c, KS)] = (_Float16)0.0f;
            lo[op_index(r, c, KS)] = (_Float16)0.0f;
        }
        if (threadIdx.x == 0)
            row_scale[r] = 0.0f;
        return;
    }
    const float *w = raw + (int64_t)r * cols;
    float m = 0.0f;
    for (int c = threadIdx.x; c < cols; c += 256)
        m = fmaxf(m, fabsf(w[c]));
    s_max[threadIdx.x] = m;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s)
            s_max[threadIdx.x] = fmaxf(s_max[threadIdx.x], s_max[threadIdx.x + s]);
        __syncthreads();
    }
    const int e = pow2_exponent_for(s_max[0]);
    const float up = ldexpf(1.0f, e);
    for (int c = threadIdx.x; c < cols; c += 256) {
        const float x = w[c] * up; // exact: a power of two
        const _Float16 h = (_Float16)x;
        hi[op_index(r, c, KS)] = h;
        lo[op_index(r, c, KS)] = (_Float16)(x - (float)h);
    }
    if (threadIdx.x == 0)
        row_scale[r] = ldexpf(1.0f, -e);
}

// ---- activations: x * 2^e split into hi + lo per batch row ---------------

// One workgroup per padded batch row (rows past the batch are zeros); each
// thread takes runs of 8 columns, so the halves go out as 16-byte stores,
// four of them one 64-byte run of a tile (x_index).
__global__ __launch_bounds__(256) void split_rows(const float *__restrict__ x, int batch, int cols,
                                                 _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
                                                 float *__restrict__ xscale)
{
    __shared__ float s_max[4];
    const int b = blockIdx.x, KS = cols / 32, runs = cols / 8;
    if (b >= batch) {
        for (int q = threadIdx.x; q < runs; q += 256) {
            *reinterpret_cast<uint4 *>(xh + x_index(b, 8 * q, KS)) = uint4{0u, 0u, 0u, 0u};
            *reinterpret_cast<uint4 *>(xl + x_index(b, 8 * q, KS)) = uint4{0u, 0u, 0u, 0u};
        }
        return;
    }
    const float *xr = x + (int64_t)b * cols;
    // a thread's first KEEP runs stay in registers between the two passes
    // (all of them for rows up to 8192 columns)
    constexpr int KEEP = 4;
    f4 ku[KEEP], kv[KEEP];
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < KEEP; k++) {
        const int q = threadIdx.x + 256 * k;
        ku[k] = kv[k] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if (q < runs) {
            ku[k] = *reinterpret_cast<const f4 *>(xr + 8 * q);
            kv[k] = *reinterpret_cast<const f4 *>(xr + 8 * q + 4);
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
            m = fmaxf(m, fmaxf(fabsf(ku[k][i]), fabsf(kv[k][i])));
    }
    for (int q = threadIdx.x + 256 * KEEP; q < runs; q += 256) {
        const f4 u = *reinterpret_cast<const f4 *>(xr + 8 * q), v = *reinterpret_cast<const f4 *>(xr + 8 * q + 4);
#pragma unroll
        for (int i = 0; i < 4; i++)
            m = fmaxf(m, fmaxf(fabsf(u[i]), fabsf(v[i])));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0)
        s_max[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    const int e = pow2_exponent_for(m);
    const float up = ldexpf(1.0f, e);
    auto emit = [&](int q, const f4 &u, const f4 &v) {
        h8 hi, lo;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float t = (k < 4 ? u[k] : v[k - 4]) * up; // exact: a power of two
            const _Float16 h = (_Float16)t;
            hi[k] = h;
            lo[k] = (_Float16)(t - (float)h);
        }
        *reinterpret_cast<h8 *>(xh + x_index(b, 8 * q, KS)) = hi;
        *reinterpret_cast<h8 *>(xl + x_index(b, 8 * q, KS)) = lo;
    };
#pragma unroll
    for (int k = 0; k < KEEP; k++) {
        const int q = threadIdx.x + 256 * k;
        if (q < runs)
            emit(q, ku[k], kv[k]);
    }
    for (int q = threadIdx.x + 256 * KEEP; q < runs; q += 256)
        emit(q, *reinterpret_cast<const f4 *>(xr + 8 * q), *reinterpret_cast<const f4 *>(xr + 8 * q + 4));
    if (threadIdx.x == 0)
        xscale[b] = ldexpf(1.0f, -e);
}

// ---- the product -----------------------------------------------------------

struct MatArgs {
    int type;
    int rows, cols, batch;
    int rows_pad;           // rows padded to a multiple of 128
    const uint8_t *a;      // F16 / F32-hi / Q8 codes / Q4 nibble bytes
    const uint8_t *a_lo;   // F32 lo
    const uint16_t *scales; // Q8 / Q4 block scales [cols/32][rows_pad]
    const float *row_scale; // F32
    const _Float16 *xh, *xl;
    const float *xscale;
    float *y;
};

// One wave's operands of one k-step, as the direct loads lay them down: the
// four batch tiles' hi and lo halves (1 KiB each), the four weight tiles
// (F16 1 KiB, F32 hi then lo, Q8_0 512 B, Q4_0 256 B), and for Q8_0 / Q4_0
// the 64 rows' block scales.
template <int WT>
struct MStage {
    static constexpr int XB = 8 * 1024;
    static constexpr int WB = WT == W_F32 ? 8192 : WT == W_F16 ? 4096 : WT == W_Q8_0 ? 2048 : 1024;
    static constexpr int SB = (WT == W_Q8_0 || WT == W_Q4_0) ? 128 : 0;
    static constexpr int BYTES = XB + WB + SB;
    // direct loads per k-step: 8 activation tiles, the weight tiles, the scales
    static constexpr int NL = 8 + (WT == W_F32 ? 8 : 4) + (SB ? 1 : 0);
};

typedef __attribute__((address_space(3))) void *lds_void;

template <int WT, int NST>
__global__ __launch_bounds__(256) void matmul_lds(MatArgs a)
{
    typedef MStage<WT> M;
    constexpr int STAGE_ALL = 4 * NST * M::BYTES, ACC = 3 * 64 * 65 * 4;
    __shared__ __attribute__((aligned(16))) uint8_t smem[STAGE_ALL > ACC ? STAGE_ALL : ACC];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int b0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
    const int C = a.cols, R = a.rows, KS = C / 32;
    const int64_t rt0 = r0 / 16, bt0 = b0 / 16;
    f4 acc[4][4];
#pragma unroll
    for (int rs = 0; rs < 4; rs++)
#pragma unroll
        for (int bs = 0; bs < 4; bs++)
            acc[rs][bs] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    uint8_t *mine = smem + w * NST * M::BYTES;
    // This wave's k-steps are w, w + 4, ...: nk of them.
    const int nk = w < KS ? (KS - w + 3) / 4 : 0;
    // The NL direct loads of this wave's i-th k-step (clamped to its last,
    // so every call issues the same number of loads) into stage st.
    auto issue = [&](int i, int st) {
        const int kk = w + 4 * min(i, nk - 1);
        uint8_t *d = mine + st * M::BYTES;
#pragma unroll
        for (int bs = 0; bs < 4; bs++) {
            // lane (j, g) fetches row j's k-elements 8g .. 8g+7 of the tile
            const int64_t o = ((bt0 + bs) * KS + kk) * 512 + 32 * j + 8 * g;
            __builtin_amdgcn_global_load_lds(a.xh + o, (lds_void)(d + 2048 * bs), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(a.xl + o, (lds_void)(d + 2048 * bs + 1024), 16, 0, 0);
        }
        d += M::XB;
#pragma unroll
        for (int rs = 0; rs < 4; rs++) {
            const int64_t t = (rt0 + rs) * KS + kk;
            if (WT == W_F16 || WT == W_F32) {
                __builtin_amdgcn_global_load_lds(a.a + t * 1024 + 16 * lane, (lds_void)(d + 1024 * rs), 16, 0, 0);
                if (WT == W_F32)
                    __builtin_amdgcn_global_load_lds(a.a_lo + t * 1024 + 16 * lane, (lds_void)(d + 4096 + 1024 * rs),
                                                     16, 0, 0);
            } else {
                constexpr int TB = WT == W_Q8_0 ? 512 : 256; // bytes of one weight tile
                if (lane < TB / 16)
                    __builtin_amdgcn_global_load_lds(a.a + t * TB + 16 * lane, (lds_void)(d + TB * rs), 16, 0, 0);
            }
        }
        if (M::SB && lane < 8)
            __builtin_amdgcn_global_load_lds(a.scales + (int64_t)kk * a.rows_pad + r0 + 8 * lane,
                                             (lds_void)(d + M::WB), 16, 0, 0);
    };
    if (nk > 0) {
#pragma unroll
        for (int i = 0; i < NST - 1; i++)
            issue(i, i);
        for (int i = 0; i < nk; i++) {
            issue(i + NST - 1, (i + NST - 1) % NST);
            // this k-step's loads are done once no more than the later
            // stages' remain in flight
            constexpr int VM = (NST - 1) * M::NL;
            __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (15 << 8));
            const uint8_t *sp = mine + (i % NST) * M::BYTES;
            h8 bh[4], bl[4];
#pragma unroll
            for (int bs = 0; bs < 4; bs++) {
                bh[bs] = *reinterpret_cast<const h8 *>(sp + 2048 * bs + 16 * lane);
                bl[bs] = *reinterpret_cast<const h8 *>(sp + 2048 * bs + 1024 + 16 * lane);
            }
            const uint8_t *wp = sp + M::XB;
#pragma unroll
            for (int rs = 0; rs < 4; rs++) {
                if (WT == W_F16 || WT == W_F32) {
                    const h8 ah = *reinterpret_cast<const h8 *>(wp + 1024 * rs + 16 * lane);
                    h8 al = {};
                    if (WT == W_F32)
                        al = *reinterpret_cast<const h8 *>(wp + 4096 + 1024 * rs + 16 * lane);
#pragma unroll
                    for (int bs = 0; bs < 4; bs++) {
                        acc[rs][bs] = mfma16(ah, bh[bs], acc[rs][bs]);
                        acc[rs][bs] = mfma16(ah, bl[bs], acc[rs][bs]);
                        if (WT == W_F32)
                            acc[rs][bs] = mfma16(al, bh[bs], acc[rs][bs]);
                    }
                } else {
                    const h8 aq = WT == W_Q8_0
                                      ? i8x8_to_h8(*reinterpret_cast<const u2 *>(wp + 512 * rs + 8 * lane))
                                      : u4x8_to_h8(*reinterpret_cast<const u2 *>(wp + 256 * rs + 16 * j + 8 * (g & 1)),
                                                   (g & 2) ? 4 : 0);
                    const u2 sw = *reinterpret_cast<const u2 *>(wp + M::WB + (16 * rs + 4 * g) * 2);
                    const uint32_t s01 = sw.x, s23 = sw.y;
                    float d[4];
                    d[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(s01 & 0xFFFFu));
                    d[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(s01 >> 16));
                    d[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(s23 & 0xFFFFu));
                    d[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(s23 >> 16));
#pragma unroll
                    for (int bs = 0; bs < 4; bs++) {
                        f4 z = mfma16(aq, bh[bs], f4{0.0f, 0.0f, 0.0f, 0.0f});
                        z = mfma16(aq, bl[bs], z);
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            acc[rs][bs][r] = fmaf(z[r], d[r], acc[rs][bs][r]);
                    }
                }
            }
        }
    }
    // the trailing (unused) loads land before the staging area becomes the
    // reduction buffer
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    float(*s_acc)[64][65] = reinterpret_cast<float(*)[64][65]>(smem);
    if (w > 0) {
#pragma unroll
        for (int rs = 0; rs < 4; rs++)
#pragma unroll
            for (int bs = 0; bs < 4; bs++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    s_acc[w - 1][16 * rs + 4 * g + i][16 * bs + j] = acc[rs][bs][i];
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
        for (int rs = 0; rs < 4; rs++)
#pragma unroll
            for (int bs = 0; bs < 4; bs++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int rl = 16 * rs + 4 * g + i, bl = 16 * bs + j;
                    s_acc[0][rl][bl] = acc[rs][bs][i] + s_acc[0][rl][bl] + s_acc[1][rl][bl] + s_acc[2][rl][bl];
                }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * 64; e += 256) {
        const int bl = e >> 6, rl = e & 63; // rows fastest: coalesced stores
        const int b = b0 + bl, r = r0 + rl;
        if (b >= a.batch || r >= R)
            continue;
        float v = s_acc[0][rl][bl];
        v *= a.xscale[b];
        if (WT == W_F32)
            v *= a.row_scale[r];
        a.y[(int64_t)b * R + r] = v;
    }
}

// ---- 16-bit weights, batches of 128 and more: split-K ------------------------
//
// A workgroup of four waves owns a 128 x 128 (rows x batch) output tile over
// one of S slices of the k-steps, and two workgroups share a CU.  Wave w
// takes batch rows 32w .. 32w + 31 of the tile and all 128 rows, so each
// weight fragment read from LDS feeds four products (two batch tiles, hi and
// lo) and each activation fragment eight (the row tiles).  Per k-step the
// eight weight tiles (shared by the waves, each loading two) and every wave's
// activation halves arrive by direct global->LDS loads two k-steps ahead,
// through three stages; one barrier per k-step hands a stage from the loads
// to the products.  The per-CU load volume is 24 KiB per 128 products against
// 12 KiB per 32 in the 64 x 64 form.  With S > 1 the partial tiles go to a
// workspace and reduce_splits adds them.  Quantised weights keep the 64 x 64
// form: their per-block scale multiply-adds need 272 registers here (one
// wave per SIMD), and measured slower (Q8_0 50.5 against 41.8 us per call
// at 256 x 4096 x 4096).

struct SKArgs {
    MatArgs m;
    int splits;   // S: slices of the k-steps
    int ks_per;   // k-steps per slice (the last may have fewer)
    float *part;  // S > 1: partial tiles [S][batch_pad][rows_pad]
    int batch_pad;
};

// The split-K form serves batches of at least kSplitKMinBatch rows; its
// k-step slices give about kSplitKWorkgroups workgroups, none shorter than
// kMinSliceSteps k-steps.
constexpr int kSplitKMinBatch = 128, kSplitKWorkgroups = 256, kMinSliceSteps = 4;

template <int N>
using ic = std::integral_constant<int, N>;

template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>)
{
    (f(ic<I>{}), ...);
}
// f(ic<0>{}), ..., f(ic<N - 1>{}): an unrolled loop whose index is a
// constant expression
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f)
{
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int WT>
__global__ __launch_bounds__(256) void matmul_sk(SKArgs s)
{
    static_assert(WT == W_F16 || WT == W_F32, "16-bit weight tiles (F32 as hi + lo)");
    // (device pass only: the host pass, which emits the launch stub, cannot
    // instantiate the target builtins inside the generic lambdas below)
#if __HIP_DEVICE_COMPILE__
    constexpr int NST = 3;                 // stages (k-steps in flight); the loop is unrolled by NST
    constexpr int NWV = 4;                 // waves
    constexpr int BS = 2;                  // batch tiles of 16 per wave
    constexpr int BT = 16 * BS * NWV;      // batch rows per workgroup
    constexpr int XB = 1024 * 2 * BS;      // a wave's activation halves of one k-step
    constexpr int WB = (WT == W_F32 ? 16 : 8) * 1024; // the 128 rows' weight tiles of one k-step
    // weight tiles per wave, and its direct loads of them per k-step
    constexpr int TPW = 8 / NWV, DW = (WT == W_F32 ? 2 : 1) * TPW;
    const MatArgs &a = s.m;
    // Every load in flight is a direct global->LDS load: with register loads
    // in flight beside them the compiler assumes the two kinds complete out
    // of order and waits for all of them.  Each stage is an array of its own,
    // named at compile time where it is used, so that before an LDS read the
    // compiler waits only for the loads into that array (it does not tell
    // apart offsets into one array).
    __shared__ __attribute__((aligned(16))) uint8_t w0[WB], w1[WB], w2[WB];
    __shared__ __attribute__((aligned(16))) uint8_t x0[NWV * XB], x1[NWV * XB], x2[NWV * XB];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int sl = blockIdx.x, r0 = blockIdx.y * 128;
    const int bw0 = blockIdx.z * BT + 16 * BS * w; // this wave's first batch row
    const bool active = bw0 < s.batch_pad;          // uniform: the activations are padded to 64
    const int KS = a.cols / 32;
    const int k0 = sl * s.ks_per, nk = min(s.ks_per, KS - k0);
    const int64_t rt0 = r0 / 16, bt0 = bw0 / 16;
    f4 acc[8][BS];
#pragma unroll
    for (int rs = 0; rs < 8; rs++)
#pragma unroll
        for (int bs = 0; bs < BS; bs++)
            acc[rs][bs] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    auto wstage = [&](auto u) __attribute__((always_inline)) -> uint8_t * {
        constexpr int U = decltype(u)::value % NST;
        return U == 0 ? w0 : U == 1 ? w1 : w2;
    };
    auto xstage = [&](auto u) __attribute__((always_inline)) -> uint8_t * {
        constexpr int U = decltype(u)::value % NST;
        return (U == 0 ? x0 : U == 1 ? x1 : x2) + XB * w;
    };
    // This wave's direct loads of k-step i of the slice (clamped to the last,
    // so every call issues the same number) into stage u: its share of the
    // weight tiles, then (ACT) its activation halves, each permuted into
    // lane order on the way (lane (j, g) fetches row j's k-elements
    // 8g .. 8g + 7, x_index).
    auto issue = [&](int i, auto u, auto act) __attribute__((always_inline)) {
        const int kk = k0 + min(i, nk - 1);
        uint8_t *d = wstage(u);
        // 1 KiB tiles TPW w .. TPW w + TPW - 1 (F32: their lo tiles too, 8 KiB
        // later)
#pragma unroll
        for (int q = 0; q < DW; q++) {
            const uint8_t *src = q >= TPW ? a.a_lo : a.a;
            const int tile = TPW * w + q % TPW;
            const int64_t t = (rt0 + tile) * KS + kk;
            __builtin_amdgcn_global_load_lds(src + t * 1024 + 16 * lane, (lds_void)(d + 1024 * (8 * (q / TPW) + tile)),
                                             16, 0, 0);
        }
        if (decltype(act)::value) {
            uint8_t *xd = xstage(u);
#pragma unroll
            for (int bs = 0; bs < BS; bs++) {
                const int64_t o = ((bt0 + bs) * KS + kk) * 512 + 32 * j + 8 * g;
                __builtin_amdgcn_global_load_lds(a.xh + o, (lds_void)(xd + 2048 * bs), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(a.xl + o, (lds_void)(xd + 2048 * bs + 1024), 16, 0, 0);
            }
        }
    };
    // Loads per k-step and wave; before the barrier of k-step i a wave waits
    // until only the next stage's are in flight (its own of stage i have
    // landed).
    constexpr int VMA = (NST - 2) * (DW + 2 * BS), VMI = (NST - 2) * DW;
    // One k-step: ACT, a wave inside the batch (loads and products), else one
    // that only loads its share of the weights.
    auto body = [&](int i, auto u, auto act) __attribute__((always_inline)) {
        constexpr bool ACT = decltype(act)::value;
        if (ACT)
            __builtin_amdgcn_s_waitcnt((VMA & 15) | ((VMA >> 4) << 14) | 0x0F70);
        else
            __builtin_amdgcn_s_waitcnt((VMI & 15) | ((VMI >> 4) << 14) | 0x0F70);
        // every wave's loads of stage i have landed, and every wave is done
        // with stage i - 1, which the loads below refill.  A bare barrier:
        // __syncthreads' release fence would wait for every load in flight.
        asm volatile("s_barrier" ::: "memory");
        issue(i + NST - 1, ic<decltype(u)::value + NST - 1>{}, act);
        if (!ACT)
            return;
        const uint8_t *sp = wstage(u);
        const uint8_t *xp = xstage(u);
        h8 xh[BS], xl[BS];
#pragma unroll
        for (int bs = 0; bs < BS; bs++) {
            xh[bs] = *reinterpret_cast<const h8 *>(xp + 2048 * bs + 16 * lane);
            xl[bs] = *reinterpret_cast<const h8 *>(xp + 2048 * bs + 1024 + 16 * lane);
        }
#pragma unroll
        for (int rs = 0; rs < 8; rs++) {
            const h8 ah = *reinterpret_cast<const h8 *>(sp + 1024 * rs + 16 * lane);
            h8 al = {};
            if (WT == W_F32)
                al = *reinterpret_cast<const h8 *>(sp + 8192 + 1024 * rs + 16 * lane);
#pragma unroll
            for (int bs = 0; bs < BS; bs++) {
                acc[rs][bs] = mfma16(ah, xh[bs], acc[rs][bs]);
                acc[rs][bs] = mfma16(ah, xl[bs], acc[rs][bs]);
                if (WT == W_F32)
                    acc[rs][bs] = mfma16(al, xh[bs], acc[rs][bs]);
            }
        }
    };
    // whole rounds of NST k-steps, then the remainder
    auto run = [&](auto act) __attribute__((always_inline)) {
        static_for<NST - 1>([&](auto u) __attribute__((always_inline)) { issue(decltype(u)::value, u, act); });
        const int nfull = nk / NST * NST;
        for (int i = 0; i < nfull; i += NST)
            static_for<NST>([&](auto u) __attribute__((always_inline)) { body(i + decltype(u)::value, u, act); });
        static_for<NST - 1>([&](auto u) __attribute__((always_inline)) {
            if (nfull + decltype(u)::value < nk)
                body(nfull + decltype(u)::value, u, act);
        });
    };
    if (nk > 0) {
        if (active)
            run(std::true_type{});
        else
            run(std::false_type{});
    }
    // the trailing (unused) loads land before the workgroup ends
    __builtin_amdgcn_s_waitcnt(0x0F70);
    if (!active)
        return;
    // lane (j, g) holds rows 16 rs + 4g + i of batch row 16 bs + j
#pragma unroll
    for (int bs = 0; bs < BS; bs++) {
        const int b = bw0 + 16 * bs + j;
        if (s.splits > 1) {
            float *pp = s.part + ((int64_t)sl * s.batch_pad + b) * a.rows_pad + r0 + 4 * g;
#pragma unroll
            for (int rs = 0; rs < 8; rs++)
                *reinterpret_cast<f4 *>(pp + 16 * rs) = acc[rs][bs];
        } else if (b < a.batch) {
            const float xs = a.xscale[b];
#pragma unroll
            for (int rs = 0; rs < 8; rs++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = r0 + 16 * rs + 4 * g + i;
                    if (r < a.rows)
                        a.y[(int64_t)b * a.rows + r] =
                            acc[rs][bs][i] * xs * (WT == W_F32 ? a.row_scale[r] : 1.0f);
                }
        }
    }
#endif
}

// y[b][r] = (sum over the S slices of the partial tiles) * xscale[b]
// (* row_scale[r] for F32 weights): four consecutive rows per thread.
__global__ __launch_bounds__(256) void reduce_splits(const float *__restrict__ part, int splits, int batch,
                                                    int batch_pad, int rows, int rows_pad,
                                                    const float *__restrict__ xscale,
                                                    const float *__restrict__ row_scale, float *__restrict__ y)
{
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; // index of 4 rows
    const int per = rows_pad / 4;
    const int b = (int)(q / per), r = 4 * (int)(q - (int64_t)b * per);
    if (b >= batch)
        return;
    f4 v = *reinterpret_cast<const f4 *>(part + (int64_t)b * rows_pad + r);
#pragma unroll 4
    for (int sl = 1; sl < splits; sl++)
        v += *reinterpret_cast<const f4 *>(part + ((int64_t)sl * batch_pad + b) * rows_pad + r);
    const float xs = xscale[b];
    f4 o;
#pragma unroll
    for (int i = 0; i < 4; i++)
        o[i] = v[i] * xs * (row_scale ? row_scale[min(r + i, rows - 1)] : 1.0f);
    float *yp = y + (int64_t)b * rows + r;
    if ((rows & 3) == 0 && r + 4 <= rows) {
        *reinterpret_cast<f4 *>(yp) = o; // 16-byte aligned: rows and r are multiples of 4
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (r + i < rows)
                yp[i] = o[i];
    }
}

int hip_fail(hipError_t e, const char *what)
{
    return set_error(GI_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

} // namespace
} // namespace gi

struct gi_weights {
    gi_paged *h = nullptr; // stream and allocation of the products
    int device = 0;        // frees need only this, so destroy does not use h
    int type = 0, rows = 0, cols = 0;
    uint8_t *a = nullptr, *a_lo = nullptr;
    uint16_t *scales = nullptr;
    float *row_scale = nullptr;
    // activation split (hi, lo halves, row scales), grown on demand
    gi::DevBuffer xsplit;
};

extern "C" {

int gi_weights_upload(gi_paged *h, int ggml_type, int rows, int cols, const void *raw, gi_weights **out)
{
    using namespace gi;
    if (!out)
        return set_error(GI_ERR_BAD_ARG, "gi_weights_upload: out is NULL");
    *out = nullptr;
    if (!h || !raw || rows <= 0 || cols <= 0 || cols % 32)
        return set_error(GI_ERR_BAD_ARG, "gi_weights_upload: need a pool handle, weights, rows > 0 and cols % 32 == 0");
    if (ggml_type != W_F32 && ggml_type != W_F16 && ggml_type != W_Q8_0 && ggml_type != W_Q4_0)
        return set_error(GI_ERR_BAD_ARG, "gi_weights_upload: GGML type " + std::to_string(ggml_type) +
                                             " has no device kernel (F32, F16, Q4_0, Q8_0 do)");
    const int64_t nb = cols / 32;
    const int64_t raw_bytes = (int64_t)rows * (ggml_type == W_F32   ? (int64_t)cols * 4
                                               : ggml_type == W_F16 ? (int64_t)cols * 2
                                               : ggml_type == W_Q8_0 ? nb * 34
                                                                     : nb * 18);
    gi_weights *wt = new (std::nothrow) gi_weights();
    if (!wt)
        return set_error(GI_ERR_OOM, "gi_weights_upload: out of host memory");
    wt->h = h;
    wt->type = ggml_type;
    wt->rows = rows;
    wt->cols = cols;
    hipStream_t st = (hipStream_t)gi_paged_stream(h);
    void *tmp = nullptr, *p = nullptr;
    int rc = GI_OK;
    auto alloc = [&](size_t n, void **dst) {
        if (rc == GI_OK)
            rc = gi_dev_alloc(h, n, dst);
    };
    const int64_t rows_pad = weight_rows_pad(rows);
    {
        alloc((size_t)raw_bytes, &tmp);
        if (rc == GI_OK)
            rc = gi_memcpy_h2d(h, tmp, raw, (size_t)raw_bytes);
        hipError_t e = hipSuccess;
        if (ggml_type == W_F16) {
            alloc((size_t)rows_pad * cols * 2, &p);
            wt->a = (uint8_t *)p;
            if (rc == GI_OK) {
                const int64_t n = rows_pad * (cols / 8);
                hipLaunchKernelGGL(convert_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                                   (const uint16_t *)tmp, rows, (int)rows_pad, cols, (uint16_t *)wt->a);
                e = hipGetLastError();
            }
        } else if (ggml_type == W_F32) {
            alloc((size_t)rows_pad * cols * 2, &p);
            wt->a = (uint8_t *)p;
            alloc((size_t)rows_pad * cols * 2, &p);
            wt->a_lo = (uint8_t *)p;
            alloc((size_t)rows_pad * 4, &p);
            wt->row_scale = (float *)p;
            if (rc == GI_OK) {
                hipLaunchKernelGGL(convert_f32, dim3((unsigned)rows_pad), dim3(256), 0, st, (const float *)tmp, rows,
                                   cols, (_Float16 *)wt->a, (_Float16 *)wt->a_lo, wt->row_scale);
                e = hipGetLastError();
            }
        } else {
            alloc((size_t)rows_pad * (ggml_type == W_Q8_0 ? cols : cols / 2), &p);
            wt->a = (uint8_t *)p;
            alloc((size_t)rows_pad * nb * 2, &p);
            wt->scales = (uint16_t *)p;
            if (rc == GI_OK) {
                const int64_t n = rows_pad * nb;
                hipLaunchKernelGGL(convert_quant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                                   (const uint8_t *)tmp, ggml_type, rows, (int)rows_pad, cols, wt->a, wt->scales);
                e = hipGetLastError();
            }
        }
        if (e != hipSuccess && rc == GI_OK)
            rc = hip_fail(e, "gi_weights_upload");
        if (tmp) {
            const int rc2 = gi_dev_free(h, tmp); // waits for the conversion
            if (rc == GI_OK)
                rc = rc2;
        }
    }
    // the pool's device, which every gi_dev_alloc above made current
    (void)hipGetDevice(&wt->device);
    if (rc != GI_OK) {
        gi_weights_destroy(wt);
        return rc;
    }
    *out = wt;
    return GI_OK;
}

void gi_weights_destroy(gi_weights *w)
{
    if (!w)
        return;
    // Does not touch the pool handle, which may be gone already; waits for
    // the device's queued work (which may still read these buffers) first.
    if (hipSetDevice(w->device) == hipSuccess)
        (void)hipDeviceSynchronize();
    for (void *p : {(void *)w->a, (void *)w->a_lo, (void *)w->scales, (void *)w->row_scale})
        if (p)
            (void)hipFree(p);
    gi::devbuf_release(w->xsplit);
    delete w;
}

int gi_matmul_batch(gi_weights *w, int batch, const float *x, float *y)
{
    using namespace gi;
    if (!w || batch < 0 || (batch > 0 && (!x || !y)))
        return set_error(GI_ERR_BAD_ARG, "gi_matmul_batch: bad argument");
    if (batch == 0)
        return GI_OK;
    gi_paged *h = w->h;
    const int batch_pad = (int)round_pad(batch); // activation rows, zero-padded
    const int rows_pad = (int)weight_rows_pad(w->rows);
    hipStream_t st = (hipStream_t)gi_paged_stream(h);
    // the split-K form from two batch tiles of 64 up; its slices: enough for
    // one workgroup per CU, each at least kMinSliceSteps k-steps long
    const int KS = w->cols / 32;
    const bool sk = batch_pad >= kSplitKMinBatch && (w->type == W_F16 || w->type == W_F32);
    int splits = 1, ks_per = KS;
    if (sk) {
        const int tiles = (rows_pad / 128) * ((batch_pad + 127) / 128);
        splits = std::max(1, std::min((kSplitKWorkgroups + tiles - 1) / tiles, KS / kMinSliceSteps));
        ks_per = (KS + splits - 1) / splits;
        splits = (KS + ks_per - 1) / ks_per;
    }
    // hi and lo halves [batch_pad][cols], the row scales, then the partial
    // tiles [splits][batch_pad][rows_pad]
    const size_t nx = (size_t)batch_pad * w->cols * 2;
    const size_t part_off = (2 * nx + (size_t)batch_pad * 4 + 255) / 256 * 256;
    const size_t need = part_off + (splits > 1 ? (size_t)splits * batch_pad * rows_pad * 4 : 0);
    hipError_t e = hipSetDevice(w->device);
    if (e != hipSuccess)
        return hip_fail(e, "gi_matmul_batch");
    const int rc = devbuf_reserve(w->xsplit, need, st, "gi_matmul_batch");
    if (rc != GI_OK)
        return rc;
    _Float16 *xh = (_Float16 *)w->xsplit.ptr;
    _Float16 *xl = (_Float16 *)((uint8_t *)w->xsplit.ptr + nx);
    float *xscale = (float *)((uint8_t *)w->xsplit.ptr + 2 * nx);
    hipLaunchKernelGGL(split_rows, dim3((unsigned)batch_pad), dim3(256), 0, st, x, batch, w->cols, xh, xl, xscale);
    MatArgs a{};
    a.type = w->type;
    a.rows = w->rows;
    a.rows_pad = rows_pad;
    a.cols = w->cols;
    a.batch = batch;
    a.a = w->a;
    a.a_lo = w->a_lo;
    a.scales = w->scales;
    a.row_scale = w->row_scale;
    a.xh = xh;
    a.xl = xl;
    a.xscale = xscale;
    a.y = y;
    if (sk) {
        SKArgs k{};
        k.m = a;
        k.splits = splits;
        k.ks_per = ks_per;
        k.part = (float *)((uint8_t *)w->xsplit.ptr + part_off);
        k.batch_pad = batch_pad;
        dim3 grid((unsigned)splits, (unsigned)(rows_pad / 128), (unsigned)((batch_pad + 127) / 128));
        if (w->type == W_F32)
            hipLaunchKernelGGL((matmul_sk<W_F32>), grid, dim3(256), 0, st, k);
        else
            hipLaunchKernelGGL((matmul_sk<W_F16>), grid, dim3(256), 0, st, k);
        if (splits > 1) {
            const int64_t n = (int64_t)batch * (rows_pad / 4);
            hipLaunchKernelGGL(reduce_splits, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, k.part, splits,
                               batch, batch_pad, w->rows, rows_pad, xscale,
                               w->type == W_F32 ? (const float *)w->row_scale : nullptr, y);
        }
    } else {
        dim3 grid((unsigned)(batch_pad / 64), (unsigned)(a.rows_pad / 64));
        switch (w->type) {
        case W_F32: hipLaunchKernelGGL((matmul_lds<W_F32, 2>), grid, dim3(256), 0, st, a); break;
        case W_F16: hipLaunchKernelGGL((matmul_lds<W_F16, 3>), grid, dim3(256), 0, st, a); break;
        case W_Q8_0: hipLaunchKernelGGL((matmul_lds<W_Q8_0, 3>), grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL((matmul_lds<W_Q4_0, 3>), grid, dim3(256), 0, st, a); break;
        }
    }
    e = hipGetLastError();
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_matmul_batch");
}

} // extern "C"
