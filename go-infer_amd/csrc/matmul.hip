// Weight matrix times a batch of activations on the matrix cores: the
// O-projection that follows attention (pkg/engine/forward.go:270 and 580,
// Weights.MatMul / MatMulBatch, pkg/engine/weights.go:237-350), for weights
// of GGML type F32, F16, Q8_0 or Q4_0.
//
//   y[b][r] = sum_c W[r][c] * x[b][c]      (pkg/math/gemv.go, metal.MatMulBatch,
//                                            pkg/metal/metal_darwin.go:849-880)
//
// Weights are converted once (gi_weights_upload) from their GGUF layout into
// one laid out for 16-byte operand loads:
//   F16   fp16 [rows][cols] as stored;
//   F32   two fp16 arrays, hi and lo, of W * 2^e[r] (e[r] from the row's
//         largest |w|, so both halves stay normal), and 2^-e[r] per row;
//   Q8_0  int8 codes [rows][cols] and fp16 block scales [cols/32][rows];
//   Q4_0  the 16 nibble bytes of each block [rows][cols/32][16] (byte j holds
//         elements j and j+16, quant.go:504) and the scales as Q8_0.
// (GGUF's 34- and 18-byte blocks are not 16-byte aligned.)
//
// Activations are split per batch row into fp16 hi + lo of x * 2^e[b], so the
// products keep float32 accuracy.  The matrix cores then compute W * x^T on
// 16x16x32 f16 tiles: quantised codes are exact fp16 values, and one 32-wide
// k-step is exactly one quantisation block, so each k-step's partial product
// is scaled by its block scale in float32 (DotVecQ8_0 / DotVecQ4_0 sum a
// block, then multiply by d).  F32 weights take three products (hi*hi, hi*lo,
// lo*hi).
//
// A workgroup owns a 64 x 64 (rows x batch) output tile.  Its four waves take
// every fourth k-step each; waves 1-3 leave their partial tiles in LDS and
// wave 0 adds them to its own, so one launch of (batch/64) x (rows/64)
// workgroups covers the product with no global reduction.
#include "../../include/goinfer_paged.h"
#include "gi_common.h"
#include "gi_host.h"
#include "mfma_ops.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <new>
#include <string>

namespace gi {
namespace {

using mfma_ops::f4;
using mfma_ops::h8;
using mfma_ops::i8x8_to_h8;
using mfma_ops::mfma16;
using mfma_ops::u2;
using mfma_ops::u4x8_to_h8;

enum : int { W_F32 = 0, W_F16 = 1, W_Q4_0 = 2, W_Q8_0 = 8 }; // GGML type ids

// ---- conversion of GGUF weights into the operand layout ------------------

// Q8_0 / Q4_0: one thread per (row, block); raw blocks are byte-addressed.
__global__ __launch_bounds__(256) void convert_quant(const uint8_t *__restrict__ raw, int type, int rows,
                                                    int cols, uint8_t *__restrict__ codes,
                                                    uint16_t *__restrict__ scales)
{
    const int nb = cols / 32;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows * nb)
        return;
    const int r = (int)(i / nb), kb = (int)(i - (int64_t)r * nb);
    const int bb = type == W_Q8_0 ? 34 : 18;
    const uint8_t *blk = raw + i * bb;
    scales[(int64_t)kb * rows + r] = (uint16_t)(blk[0] | (blk[1] << 8));
    const int n = type == W_Q8_0 ? 32 : 16;
    uint8_t *dst = codes + i * n; // [rows][cols] int8, or [rows][nb][16]
    for (int j = 0; j < n; j++)
        dst[j] = blk[2 + j];
}

// F32: one workgroup per row; W * 2^e split into hi + lo fp16.
__global__ __launch_bounds__(256) void convert_f32(const float *__restrict__ raw, int cols,
                                                  _Float16 *__restrict__ hi, _Float16 *__restrict__ lo,
                                                  float *__restrict__ row_scale)
{
    __shared__ float s_max[256];
    const int r = blockIdx.x;
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
        hi[(int64_t)r * cols + c] = h;
        lo[(int64_t)r * cols + c] = (_Float16)(x - (float)h);
    }
    if (threadIdx.x == 0)
        row_scale[r] = ldexpf(1.0f, -e);
}

// ---- activations: x * 2^e split into hi + lo per batch row ---------------

__global__ __launch_bounds__(256) void split_rows(const float *__restrict__ x, int cols, _Float16 *__restrict__ xh,
                                                 _Float16 *__restrict__ xl, float *__restrict__ xscale)
{
    __shared__ float s_max[256];
    const int b = blockIdx.x;
    const float *xr = x + (int64_t)b * cols;
    float m = 0.0f;
    for (int c = threadIdx.x; c < cols; c += 256)
        m = fmaxf(m, fabsf(xr[c]));
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
        const float v = xr[c] * up; // exact: a power of two
        const _Float16 h = (_Float16)v;
        xh[(int64_t)b * cols + c] = h;
        xl[(int64_t)b * cols + c] = (_Float16)(v - (float)h);
    }
    if (threadIdx.x == 0)
        xscale[b] = ldexpf(1.0f, -e);
}

// ---- the product -----------------------------------------------------------

struct MatArgs {
    int type;
    int rows, cols, batch;
    const uint8_t *a;      // F16 / F32-hi / Q8 codes / Q4 nibble bytes
    const uint8_t *a_lo;   // F32 lo
    const uint16_t *scales; // Q8 / Q4 block scales [cols/32][rows]
    const float *row_scale; // F32
    const _Float16 *xh, *xl;
    const float *xscale;
    float *y;
};

template <bool NT>
__device__ __forceinline__ h8 ld_h8(const void *p)
{
    if (NT)
        return __builtin_nontemporal_load(reinterpret_cast<const h8 *>(p));
    return *reinterpret_cast<const h8 *>(p);
}

// Workgroup: 4 waves, output tile rows [r0, r0+64) x batch [b0, b0+64).
// Wave w takes k-steps w, w+4, ...; lane (j, g) of row tile rs holds output
// rows 16*rs + 4g + i (i < 4), batch column 16*bs + j.
template <int WT>
__global__ __launch_bounds__(256) void matmul_tile(MatArgs a)
{
    __shared__ float s_acc[3][64][65]; // waves 1..3; wave 0 folds them in
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int b0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
    const int C = a.cols, R = a.rows, KS = C / 32;
    f4 acc[4][4];
#pragma unroll
    for (int rs = 0; rs < 4; rs++)
#pragma unroll
        for (int bs = 0; bs < 4; bs++)
            acc[rs][bs] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    // A rows of this lane (clamped: rows past the end are computed and not stored)
    int64_t arow[4];
#pragma unroll
    for (int rs = 0; rs < 4; rs++)
        arow[rs] = min(r0 + 16 * rs + j, R - 1);
    // B columns: batch rows (past the end: zero operands)
    bool bvalid[4];
    int64_t brow[4];
#pragma unroll
    for (int bs = 0; bs < 4; bs++) {
        const int b = b0 + 16 * bs + j;
        bvalid[bs] = b < a.batch;
        brow[bs] = bvalid[bs] ? b : 0;
    }
    const h8 zero8 = {};
    for (int kk = w; kk < KS; kk += 4) {
        const int c0 = 32 * kk + 8 * g;
        h8 bh[4], bl[4];
#pragma unroll
        for (int bs = 0; bs < 4; bs++) {
            bh[bs] = bvalid[bs] ? ld_h8<false>(a.xh + brow[bs] * C + c0) : zero8;
            bl[bs] = bvalid[bs] ? ld_h8<false>(a.xl + brow[bs] * C + c0) : zero8;
        }
#pragma unroll
        for (int rs = 0; rs < 4; rs++) {
            if (WT == W_F16 || WT == W_F32) {
                const h8 ah = ld_h8<true>(a.a + (arow[rs] * C + c0) * 2);
                h8 al = {};
                if (WT == W_F32)
                    al = ld_h8<true>(a.a_lo + (arow[rs] * C + c0) * 2);
#pragma unroll
                for (int bs = 0; bs < 4; bs++) {
                    acc[rs][bs] = mfma16(ah, bh[bs], acc[rs][bs]);
                    acc[rs][bs] = mfma16(ah, bl[bs], acc[rs][bs]);
                    if (WT == W_F32)
                        acc[rs][bs] = mfma16(al, bh[bs], acc[rs][bs]);
                }
            } else {
                h8 aq;
                if (WT == W_Q8_0) {
                    aq = i8x8_to_h8(*reinterpret_cast<const u2 *>(a.a + arow[rs] * C + c0));
                } else {
                    // dims 8g..8g+7 of the block: low (g < 2) or high nibbles
                    // of bytes 8*(g%2) .. +7
                    const u2 wq = *reinterpret_cast<const u2 *>(a.a + (arow[rs] * KS + kk) * 16 + 8 * (g & 1));
                    aq = u4x8_to_h8(wq, (g & 2) ? 4 : 0);
                }
                // scales of output rows 16rs + 4g + i, i < 4 (rows past the
                // end read row R-1's)
                float d[4];
                const int rb = r0 + 16 * rs + 4 * g;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint16_t hb = a.scales[(int64_t)kk * R + min(rb + i, R - 1)];
                    d[i] = (float)__builtin_bit_cast(_Float16, hb);
                }
#pragma unroll
                for (int bs = 0; bs < 4; bs++) {
                    f4 z = mfma16(aq, bh[bs], f4{0.0f, 0.0f, 0.0f, 0.0f});
                    z = mfma16(aq, bl[bs], z);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[rs][bs][i] = fmaf(z[i], d[i], acc[rs][bs][i]);
                }
            }
        }
    }
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
    // activation split, grown on demand
    _Float16 *xh = nullptr, *xl = nullptr;
    float *xscale = nullptr;
    int x_cap = 0; // batch rows the split buffers hold
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
    if (ggml_type == W_F16) {
        alloc((size_t)raw_bytes, &p);
        wt->a = (uint8_t *)p;
        if (rc == GI_OK)
            rc = gi_memcpy_h2d(h, wt->a, raw, (size_t)raw_bytes);
    } else {
        alloc((size_t)raw_bytes, &tmp);
        if (rc == GI_OK)
            rc = gi_memcpy_h2d(h, tmp, raw, (size_t)raw_bytes);
        if (ggml_type == W_F32) {
            alloc((size_t)rows * cols * 2, &p);
            wt->a = (uint8_t *)p;
            alloc((size_t)rows * cols * 2, &p);
            wt->a_lo = (uint8_t *)p;
            alloc((size_t)rows * 4, &p);
            wt->row_scale = (float *)p;
            if (rc == GI_OK) {
                hipLaunchKernelGGL(convert_f32, dim3((unsigned)rows), dim3(256), 0, st, (const float *)tmp, cols,
                                   (_Float16 *)wt->a, (_Float16 *)wt->a_lo, wt->row_scale);
                hipError_t e = hipGetLastError();
                if (e != hipSuccess)
                    rc = hip_fail(e, "gi_weights_upload");
            }
        } else {
            alloc((size_t)rows * (ggml_type == W_Q8_0 ? cols : cols / 2), &p);
            wt->a = (uint8_t *)p;
            alloc((size_t)rows * nb * 2, &p);
            wt->scales = (uint16_t *)p;
            if (rc == GI_OK) {
                const int64_t n = (int64_t)rows * nb;
                hipLaunchKernelGGL(convert_quant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                                   (const uint8_t *)tmp, ggml_type, rows, cols, wt->a, wt->scales);
                hipError_t e = hipGetLastError();
                if (e != hipSuccess)
                    rc = hip_fail(e, "gi_weights_upload");
            }
        }
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
    for (void *p : {(void *)w->a, (void *)w->a_lo, (void *)w->scales, (void *)w->row_scale, (void *)w->xh,
                    (void *)w->xl, (void *)w->xscale})
        if (p)
            (void)hipFree(p);
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
    if (batch > w->x_cap) {
        for (void *p : {(void *)w->xh, (void *)w->xl, (void *)w->xscale})
            if (p)
                (void)gi_dev_free(h, p); // waits for queued work that reads them
        w->xh = w->xl = nullptr;
        w->xscale = nullptr;
        w->x_cap = 0;
        void *p = nullptr;
        const size_t nx = (size_t)batch * w->cols * 2;
        int rc = gi_dev_alloc(h, nx, &p);
        w->xh = (_Float16 *)p;
        if (rc == GI_OK && (rc = gi_dev_alloc(h, nx, &p)) == GI_OK)
            w->xl = (_Float16 *)p;
        if (rc == GI_OK && (rc = gi_dev_alloc(h, (size_t)batch * 4, &p)) == GI_OK)
            w->xscale = (float *)p;
        if (rc != GI_OK)
            return rc;
        w->x_cap = batch;
    }
    hipStream_t st = (hipStream_t)gi_paged_stream(h);
    hipLaunchKernelGGL(split_rows, dim3((unsigned)batch), dim3(256), 0, st, x, w->cols, w->xh, w->xl, w->xscale);
    MatArgs a{};
    a.type = w->type;
    a.rows = w->rows;
    a.cols = w->cols;
    a.batch = batch;
    a.a = w->a;
    a.a_lo = w->a_lo;
    a.scales = w->scales;
    a.row_scale = w->row_scale;
    a.xh = w->xh;
    a.xl = w->xl;
    a.xscale = w->xscale;
    a.y = y;
    dim3 grid((unsigned)((batch + 63) / 64), (unsigned)((w->rows + 63) / 64));
    switch (w->type) {
    case W_F32: hipLaunchKernelGGL(matmul_tile<W_F32>, grid, dim3(256), 0, st, a); break;
    case W_F16: hipLaunchKernelGGL(matmul_tile<W_F16>, grid, dim3(256), 0, st, a); break;
    case W_Q8_0: hipLaunchKernelGGL(matmul_tile<W_Q8_0>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(matmul_tile<W_Q4_0>, grid, dim3(256), 0, st, a); break;
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_matmul_batch");
}

} // extern "C"
