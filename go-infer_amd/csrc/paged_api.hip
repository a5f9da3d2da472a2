// C ABI of the paged KV-cache library: device pool handle, stream, errors,
// argument checks, and dispatch to the kernels.  Declarations and the
// reference interfaces each entry point replaces are in
// include/goinfer_paged.h.
#include "../../include/goinfer_paged.h"
#include "devbuf.h"
#include "gi_kernels.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

namespace gi {

static thread_local std::string g_last_error;

int set_error(int code, const std::string &msg)
{
    g_last_error = msg;
    return code;
}

void clear_error() { g_last_error.clear(); }

int devbuf_reserve(DevBuffer &b, size_t need, hipStream_t st, const char *what)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess)
        return set_error(GI_ERR_HIP, std::string(what) + ": hipStreamIsCapturing: " + hipGetErrorString(e));
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (capturing)
        b.captured = true;
    if (need <= b.bytes)
        return GI_OK;
    if (capturing)
        return set_error(GI_ERR_BAD_ARG,
                         std::string(what) + ": needs " + std::to_string(need) + " bytes of workspace (holds " +
                             std::to_string(b.bytes) +
                             ") while the stream is capturing a graph; make one eager call of this shape "
                             "(or a larger batch) before capturing");
    if (b.ptr) {
        if (b.captured) {
            // a captured graph may still address it: keep it until release
            b.retired.push_back(b.ptr);
        } else {
            // work already queued may still read it
            e = hipStreamSynchronize(st);
            if (e != hipSuccess)
                return set_error(GI_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
            (void)hipFree(b.ptr);
        }
        b.ptr = nullptr;
        b.bytes = 0;
    }
    const size_t want = need + need / 4;
    void *p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess)
        return set_error(GI_ERR_OOM, std::string(what) + ": hipMalloc(" + std::to_string(want) + ") failed");
    b.ptr = p;
    b.bytes = want;
    return GI_OK;
}

void devbuf_release(DevBuffer &b)
{
    if (b.ptr)
        (void)hipFree(b.ptr);
    for (void *p : b.retired)
        (void)hipFree(p);
    b.retired.clear();
    b.ptr = nullptr;
    b.bytes = 0;
}

} // namespace gi

struct gi_paged {
    std::mutex mu;
    gi::PoolLayout L{};
    int device = 0;
    int num_cus = 256;
    std::vector<uint8_t *> layer_base;
    uint8_t **d_layer_base = nullptr; // the same pointers in device memory
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    int *d_status = nullptr;
    gi::DevBuffer plan_ws; // decode: partials of split sequences
    void *scratch = nullptr; // this device's address of `scratch` (allocate-nothing decode)
    struct ScratchOrder *scratch_order = nullptr; // and the ordering of its users
    int decode_kernel = -1; // -1 automatic, 0 vector ALU, 1 matrix core
    float2 *d_rope = nullptr; // (cos, sin) [rope_max_pos][rope_half]
    int rope_half = 0;
    int rope_max_pos = 0;
};

namespace {

int hip_fail(hipError_t e, const char *what)
{
    return gi::set_error(GI_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Makes the handle's device current for this thread.
int enter(gi_paged *h, const char *what)
{
    if (!h)
        return gi::set_error(GI_ERR_BAD_ARG, std::string(what) + ": NULL handle");
    hipError_t e = hipSetDevice(h->device);
    if (e != hipSuccess)
        return hip_fail(e, what);
    return GI_OK;
}

int check_layer(const gi_paged *h, int layer, const char *what)
{
    if (layer < 0 || layer >= h->L.num_layers)
        return gi::set_error(GI_ERR_BAD_ARG, std::string(what) + ": layer " + std::to_string(layer) +
                                                 " out of range");
    return GI_OK;
}

// Scratch of gi_paged_decode_attention_noalloc: the split partials live in
// this fixed array of the code object (one per device, held until the
// process ends) instead of the handle's growable workspace.  Its name is a
// host-side stand-in for the array, not a device address: host code uses the
// address hipGetSymbolAddress gives on each device (scratch_address).
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

} // namespace

// Every handle on a device shares that device's array, whatever its stream.
// Successive users are ordered on the device: each call's launches are
// followed by a record of `done` on its stream, and a call from another
// stream first waits for it.  The event is created once per device, with the
// address; no call allocates.  (A stream that is capturing a graph neither
// waits nor records: the replays of such a graph are ordered against other
// users of the array by the caller.)
struct ScratchOrder {
    void *addr = nullptr;
    hipEvent_t done = nullptr;  // recorded after the last eager user's launches
    hipStream_t last = nullptr; // that user's stream
    bool recorded = false;
    std::mutex mu; // held from the wait to the record
};

namespace {

std::mutex g_scratch_mu;
std::vector<std::unique_ptr<ScratchOrder>> g_scratch; // by device id

// With `device` current: the device address of `scratch` there and its
// ordering state, set up once per device.
int scratch_address(int device, void **addr, ScratchOrder **order)
{
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if ((size_t)device < g_scratch.size() && g_scratch[(size_t)device]) {
        *addr = g_scratch[(size_t)device]->addr;
        *order = g_scratch[(size_t)device].get();
        return GI_OK;
    }
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "scratch: hipGetSymbolAddress");
    std::unique_ptr<ScratchOrder> so(new ScratchOrder);
    so->addr = p;
    e = hipEventCreateWithFlags(&so->done, hipEventDisableTiming);
    if (e != hipSuccess)
        return hip_fail(e, "scratch: hipEventCreateWithFlags");
    if (g_scratch.size() <= (size_t)device)
        g_scratch.resize((size_t)device + 1);
    *addr = p;
    *order = so.get();
    g_scratch[(size_t)device] = std::move(so);
    return GI_OK;
}

bool supported_heads(const gi::PoolLayout &L, int num_heads)
{
    if (num_heads <= 0 || num_heads % L.num_kv_heads)
        return false;
    int G = num_heads / L.num_kv_heads;
    if (L.head_dim == 128 && G == 16)
        return true;
    return (L.head_dim == 64 || L.head_dim == 128) && (G == 1 || G == 2 || G == 4 || G == 8);
}

} // namespace

extern "C" {

const char *gi_last_error(void) { return gi::g_last_error.c_str(); }

int gi_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess)
        return 0;
    return n;
}

int gi_device_name(char *buf, int cap)
{
    if (!buf || cap <= 0)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_device_name: bad buffer");
    buf[0] = 0;
    int dev = 0;
    if (gi_device_count() <= 0 || hipGetDevice(&dev) != hipSuccess)
        return gi::set_error(GI_ERR_NO_DEVICE, "no HIP device");
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess)
        return hip_fail(e, "gi_device_name");
    snprintf(buf, (size_t)cap, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return GI_OK;
}

int gi_paged_create(int num_layers, int num_kv_heads, int head_dim, int page_tokens,
                    int64_t num_pages, int kv_type, gi_paged **out)
{
    if (!out)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_create: out is NULL");
    *out = nullptr;
    gi::PoolLayout L;
    if (gi::make_layout(kv_type, num_layers, num_kv_heads, head_dim, page_tokens, num_pages, &L))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_create: unsupported shape or kv type");
    if (gi_device_count() <= 0)
        return gi::set_error(GI_ERR_NO_DEVICE, "gi_paged_create: no HIP device");
    gi_paged *h = new (std::nothrow) gi_paged();
    if (!h)
        return gi::set_error(GI_ERR_OOM, "gi_paged_create: out of host memory");
    h->L = L;
    hipError_t e = hipGetDevice(&h->device);
    if (e == hipSuccess) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, h->device) == hipSuccess)
            h->num_cus = p.multiProcessorCount;
        e = hipStreamCreateWithFlags(&h->own_stream, hipStreamNonBlocking);
    }
    if (e != hipSuccess) {
        int rc = hip_fail(e, "gi_paged_create");
        delete h;
        return rc;
    }
    h->stream = h->own_stream;
    int rc = scratch_address(h->device, &h->scratch, &h->scratch_order);
    if (rc == GI_OK && hipMalloc((void **)&h->d_status, sizeof(int)) != hipSuccess) {
        h->d_status = nullptr;
        rc = gi::set_error(GI_ERR_OOM, "gi_paged_create: status word");
    }
    const size_t layer_bytes = (size_t)(L.page_bytes * L.num_pages);
    for (int l = 0; rc == GI_OK && l < num_layers; l++) {
        void *p = nullptr;
        if (hipMalloc(&p, layer_bytes) != hipSuccess) {
            rc = gi::set_error(GI_ERR_OOM, "gi_paged_create: cannot allocate layer " + std::to_string(l) +
                                               " (" + std::to_string(layer_bytes) + " bytes)");
            break;
        }
        h->layer_base.push_back((uint8_t *)p);
        e = hipMemsetAsync(p, 0, layer_bytes, h->stream);
        if (e != hipSuccess)
            rc = hip_fail(e, "gi_paged_create: clear");
    }
    if (rc == GI_OK) {
        const size_t pb = sizeof(uint8_t *) * (size_t)num_layers;
        if (hipMalloc((void **)&h->d_layer_base, pb) != hipSuccess) {
            h->d_layer_base = nullptr;
            rc = gi::set_error(GI_ERR_OOM, "gi_paged_create: layer table");
        } else if ((e = hipMemcpy(h->d_layer_base, h->layer_base.data(), pb, hipMemcpyHostToDevice)) !=
                   hipSuccess) {
            rc = hip_fail(e, "gi_paged_create: layer table");
        }
    }
    if (rc == GI_OK) {
        e = hipMemsetAsync(h->d_status, 0, sizeof(int), h->stream);
        if (e == hipSuccess)
            e = hipStreamSynchronize(h->stream);
        if (e != hipSuccess)
            rc = hip_fail(e, "gi_paged_create: clear");
    }
    if (rc != GI_OK) {
        gi_paged_destroy(h);
        return rc;
    }
    *out = h;
    gi::clear_error();
    return GI_OK;
}

void gi_paged_destroy(gi_paged *h)
{
    if (!h)
        return;
    (void)hipSetDevice(h->device);
    if (h->own_stream)
        (void)hipStreamSynchronize(h->own_stream);
    if (h->stream && h->stream != h->own_stream)
        (void)hipStreamSynchronize(h->stream);
    for (uint8_t *p : h->layer_base)
        (void)hipFree(p);
    if (h->d_status)
        (void)hipFree(h->d_status);
    if (h->d_layer_base)
        (void)hipFree(h->d_layer_base);
    gi::devbuf_release(h->plan_ws);
    if (h->d_rope)
        (void)hipFree(h->d_rope);
    if (h->own_stream)
        (void)hipStreamDestroy(h->own_stream);
    delete h;
}

int gi_paged_page_bytes(const gi_paged *h, int64_t *page_bytes, int64_t *pool_bytes)
{
    if (!h)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_page_bytes: NULL handle");
    if (page_bytes)
        *page_bytes = h->L.page_bytes;
    if (pool_bytes)
        *pool_bytes = h->L.page_bytes * h->L.num_pages * h->L.num_layers;
    return GI_OK;
}

int gi_paged_set_stream(gi_paged *h, void *stream)
{
    int rc = enter(h, "gi_paged_set_stream");
    if (rc)
        return rc;
    std::lock_guard<std::mutex> g(h->mu);
    hipStream_t next = (hipStream_t)stream;
    if (next != h->stream) {
        // Work queued on the old stream finishes before the new one runs.
        hipError_t e = hipStreamSynchronize(h->stream);
        if (e != hipSuccess)
            return hip_fail(e, "gi_paged_set_stream");
    }
    h->stream = next;
    return GI_OK;
}

void *gi_paged_stream(gi_paged *h) { return h ? (void *)h->stream : nullptr; }

int gi_synchronize(gi_paged *h)
{
    int rc = enter(h, "gi_synchronize");
    if (rc)
        return rc;
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess)
        return hip_fail(e, "gi_synchronize");
    int flags = 0;
    e = hipMemcpy(&flags, h->d_status, sizeof(int), hipMemcpyDeviceToHost);
    if (e != hipSuccess)
        return hip_fail(e, "gi_synchronize: status");
    if (flags) {
        const int zero = 0;
        e = hipMemcpy(h->d_status, &zero, sizeof(int), hipMemcpyHostToDevice);
        if (e != hipSuccess)
            return hip_fail(e, "gi_synchronize: status reset");
        std::string why;
        if (flags & gi::FLAG_BAD_PAGE)
            why += " page id outside the pool;";
        if (flags & gi::FLAG_BAD_SLOT)
            why += " slot or position outside the block table;";
        if (flags & gi::FLAG_BAD_POS)
            why += " position outside the RoPE table;";
        return gi::set_error(GI_ERR_BAD_PAGE, "kernel saw:" + why + " affected tokens were skipped");
    }
    return GI_OK;
}

int gi_dev_alloc(gi_paged *h, size_t bytes, void **dptr)
{
    int rc = enter(h, "gi_dev_alloc");
    if (rc)
        return rc;
    if (!dptr)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_dev_alloc: dptr is NULL");
    *dptr = nullptr;
    if (hipMalloc(dptr, bytes ? bytes : 1) != hipSuccess) {
        *dptr = nullptr;
        return gi::set_error(GI_ERR_OOM, "gi_dev_alloc: hipMalloc(" + std::to_string(bytes) + ") failed");
    }
    return GI_OK;
}

int gi_dev_free(gi_paged *h, void *dptr)
{
    int rc = enter(h, "gi_dev_free");
    if (rc)
        return rc;
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = hipStreamSynchronize(h->stream);
    if (e == hipSuccess && dptr)
        e = hipFree(dptr);
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_dev_free");
}

int gi_memcpy_h2d(gi_paged *h, void *dst, const void *src, size_t bytes)
{
    int rc = enter(h, "gi_memcpy_h2d");
    if (rc)
        return rc;
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, h->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(h->stream);
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_memcpy_h2d");
}

int gi_memcpy_d2h(gi_paged *h, void *dst, const void *src, size_t bytes)
{
    int rc = enter(h, "gi_memcpy_d2h");
    if (rc)
        return rc;
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, h->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(h->stream);
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_memcpy_d2h");
}

int gi_paged_append(gi_paged *h, int layer, int n_tok, const int32_t *block_ids,
                    const int32_t *slots, const float *k, const float *v)
{
    int rc = enter(h, "gi_paged_append");
    if (rc || (rc = check_layer(h, layer, "gi_paged_append")))
        return rc;
    if (n_tok < 0 || (n_tok > 0 && (!block_ids || !slots || !k || !v)))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_append: bad argument");
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = gi::launch_append(h->L, h->layer_base[(size_t)layer], n_tok, block_ids, slots, k, v,
                                     h->d_status, h->stream);
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_paged_append");
}

int gi_paged_append_at_len(gi_paged *h, int layer, int batch, const int32_t *block_tables,
                           int max_blocks, const int32_t *seq_lens, const float *k, const float *v)
{
    int rc = enter(h, "gi_paged_append_at_len");
    if (rc || (rc = check_layer(h, layer, "gi_paged_append_at_len")))
        return rc;
    if (batch < 0 || (batch > 0 && (!block_tables || !seq_lens || !k || !v || max_blocks <= 0)))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_append_at_len: bad argument");
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = gi::launch_append_at_len(h->L, h->layer_base[(size_t)layer], batch, block_tables,
                                            max_blocks, seq_lens, k, v, h->d_status, h->stream);
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_paged_append_at_len");
}

int gi_paged_set_rope(gi_paged *h, float theta, int rope_dim, int max_positions)
{
    int rc = enter(h, "gi_paged_set_rope");
    if (rc)
        return rc;
    const int hd = h->L.head_dim;
    if (rope_dim <= 0)
        rope_dim = hd;
    if (!std::isfinite(theta) || !(theta > 0.0f) || rope_dim > hd || rope_dim % 2 ||
        max_positions <= 0)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_set_rope: need theta > 0, an even rope_dim "
                                             "<= head_dim and max_positions > 0");
    const int rh = rope_dim / 2;
    const size_t n = (size_t)max_positions * (size_t)rh;
    // ApplyRoPE's angles (pkg/math/kernels.go:24-28): freq = 1/theta^(2j/d)
    // and pos*freq in float64, cos and sin rounded to float32.
    std::vector<float2> tab;
    try {
        tab.resize(n);
    } catch (const std::bad_alloc &) {
        return gi::set_error(GI_ERR_OOM, "gi_paged_set_rope: out of host memory");
    }
    std::vector<double> freq((size_t)rh);
    for (int j = 0; j < rh; j++)
        freq[(size_t)j] = 1.0 / std::pow((double)theta, (double)(2 * j) / (double)rope_dim);
    for (int p = 0; p < max_positions; p++) {
        for (int j = 0; j < rh; j++) {
            double val = (double)p * freq[(size_t)j];
            tab[(size_t)p * rh + j] = make_float2((float)std::cos(val), (float)std::sin(val));
        }
    }
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = hipStreamSynchronize(h->stream); // queued work may read the old table
    if (e != hipSuccess)
        return hip_fail(e, "gi_paged_set_rope");
    if (h->d_rope) {
        (void)hipFree(h->d_rope);
        h->d_rope = nullptr;
        h->rope_half = h->rope_max_pos = 0;
    }
    float2 *d = nullptr;
    if (hipMalloc((void **)&d, n * sizeof(float2)) != hipSuccess)
        return gi::set_error(GI_ERR_OOM, "gi_paged_set_rope: hipMalloc of the table failed");
    e = hipMemcpy(d, tab.data(), n * sizeof(float2), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return hip_fail(e, "gi_paged_set_rope: upload");
    }
    h->d_rope = d;
    h->rope_half = rh;
    h->rope_max_pos = max_positions;
    return GI_OK;
}

static int check_rope(gi_paged *h, int layer, int n_tok, int num_heads, const float *q, const float *q_out,
                      const float *k, const float *v, const char *what)
{
    int rc = check_layer(h, layer, what);
    if (rc)
        return rc;
    if (!h->d_rope)
        return gi::set_error(GI_ERR_BAD_ARG, std::string(what) + ": no RoPE table (gi_paged_set_rope)");
    if (n_tok < 0 || num_heads < 0)
        return gi::set_error(GI_ERR_BAD_ARG, std::string(what) + ": bad argument");
    if (n_tok > 0 && (!k || !v || (num_heads > 0 && (!q || !q_out))))
        return gi::set_error(GI_ERR_BAD_ARG, std::string(what) + ": NULL buffer");
    if ((size_t)h->L.num_kv_heads * h->L.head_dim * sizeof(float) > 65536)
        return gi::set_error(GI_ERR_BAD_ARG, std::string(what) + ": kv_dim above 16384");
    return GI_OK;
}

static gi::RopeArgs rope_args(const gi_paged *h, int num_heads, const int32_t *positions, const float *q,
                              float *q_out)
{
    gi::RopeArgs R{};
    R.table = h->d_rope;
    R.rope_half = h->rope_half;
    R.max_pos = h->rope_max_pos;
    R.num_heads = num_heads;
    R.positions = positions;
    R.q = q;
    R.q_out = q_out;
    return R;
}

int gi_paged_rope_append(gi_paged *h, int layer, int n_tok, int num_heads, const int32_t *positions,
                         const int32_t *block_ids, const int32_t *slots, const float *q, float *q_out,
                         const float *k, const float *v)
{
    int rc = enter(h, "gi_paged_rope_append");
    if (rc || (rc = check_rope(h, layer, n_tok, num_heads, q, q_out, k, v, "gi_paged_rope_append")))
        return rc;
    if (n_tok > 0 && (!positions || !block_ids || !slots))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_rope_append: NULL positions, block_ids or slots");
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = gi::launch_rope_append(h->L, h->layer_base[(size_t)layer], n_tok, block_ids, slots, nullptr,
                                          0, nullptr, rope_args(h, num_heads, positions, q, q_out), k, v,
                                          h->d_status, h->stream);
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_paged_rope_append");
}

int gi_paged_rope_append_at_len(gi_paged *h, int layer, int batch, int num_heads,
                                const int32_t *block_tables, int max_blocks, const int32_t *seq_lens,
                                const float *q, float *q_out, const float *k, const float *v)
{
    int rc = enter(h, "gi_paged_rope_append_at_len");
    if (rc || (rc = check_rope(h, layer, batch, num_heads, q, q_out, k, v, "gi_paged_rope_append_at_len")))
        return rc;
    if (batch > 0 && (!block_tables || !seq_lens || max_blocks <= 0))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_rope_append_at_len: bad block tables");
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = gi::launch_rope_append(h->L, h->layer_base[(size_t)layer], batch, nullptr, nullptr,
                                          block_tables, max_blocks, seq_lens,
                                          rope_args(h, num_heads, nullptr, q, q_out), k, v, h->d_status,
                                          h->stream);
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_paged_rope_append_at_len");
}

int gi_paged_copy_pages(gi_paged *h, int n, const int32_t *src_ids, const int32_t *dst_ids)
{
    int rc = enter(h, "gi_paged_copy_pages");
    if (rc)
        return rc;
    if (n < 0 || (n > 0 && (!src_ids || !dst_ids)))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_copy_pages: bad argument");
    if (n == 0)
        return GI_OK;
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = gi::launch_copy_pages(h->L, h->d_layer_base, n, src_ids, dst_ids, h->d_status, h->stream);
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_paged_copy_pages");
}

int gi_paged_gather(gi_paged *h, int layer, const int32_t *block_table, int n_tok, void *k_out,
                    void *v_out, int widen)
{
    int rc = enter(h, "gi_paged_gather");
    if (rc || (rc = check_layer(h, layer, "gi_paged_gather")))
        return rc;
    if (n_tok < 0 || (n_tok > 0 && (!block_table || !k_out || !v_out)))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_gather: bad argument");
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = gi::launch_gather(h->L, h->layer_base[(size_t)layer], block_table, n_tok, k_out,
                                     v_out, widen ? 1 : 0, h->d_status, h->stream);
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_paged_gather");
}

// fixed_ws: the allocate-nothing form's scratch (fixed_cap bytes) in place
// of the handle's growable workspace.
static int decode_locked(gi_paged *h, int layer, int batch, int num_heads, const float *q,
                         float *out, const int32_t *block_tables, int max_blocks,
                         const int32_t *seq_lens, int max_seq_len, float scale, void *fixed_ws = nullptr,
                         size_t fixed_cap = 0, const float *new_k = nullptr, const float *new_v = nullptr)
{
    gi::DecodeArgs a{};
    a.L = h->L;
    a.base = h->layer_base[(size_t)layer];
    a.q = q;
    a.out = out;
    a.block_tables = block_tables;
    a.max_blocks = max_blocks;
    a.seq_lens = seq_lens;
    a.batch = batch;
    a.n_q = 1;
    a.start_pos = nullptr;
    a.num_heads = num_heads;
    a.scale = scale;
    a.status = h->d_status;
    a.kernel = h->decode_kernel;
    a.append_base = h->layer_base[(size_t)layer];
    // max_seq_len sizes the split plan only (0: the longest sequence the
    // block tables map); the kernels read the lengths on the device and the
    // last split of each sequence runs to its end
    const int64_t mapped = (int64_t)max_blocks * h->L.page_tokens;
    const int max_len = (int)(max_seq_len > 0 && max_seq_len < mapped ? max_seq_len
                              : mapped < INT32_MAX ? mapped : INT32_MAX);
    gi::decode_plan(h->L, batch, num_heads, max_len, h->num_cus, &a.split_tokens, &a.num_splits);
    a.waves = gi::decode_waves(h->L, batch, a.num_splits, h->num_cus);
    // the workspace first: a call refused here has queued nothing
    const size_t need = gi::decode_workspace_bytes(h->L, batch, num_heads, a.num_splits);
    std::unique_lock<std::mutex> order; // the shared scratch's users, in turn
    bool eager = false;
    if (fixed_ws) {
        if (need > fixed_cap)
            return gi::set_error(GI_ERR_BAD_ARG,
                                 "gi_paged_decode_attention_noalloc: this shape needs " + std::to_string(need) +
                                     " bytes of scratch; the fixed maximum is " + std::to_string(fixed_cap) +
                                     " (use gi_paged_decode_attention)");
        a.ws = (float *)fixed_ws;
        ScratchOrder *so = h->scratch_order;
        order = std::unique_lock<std::mutex>(so->mu);
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        hipError_t e = hipStreamIsCapturing(h->stream, &cs);
        if (e != hipSuccess)
            return hip_fail(e, "gi_paged_decode_attention_noalloc: hipStreamIsCapturing");
        eager = cs == hipStreamCaptureStatusNone;
        if (eager && so->recorded && so->last != h->stream) {
            // the previous user's launches (another stream) finish first
            e = hipStreamWaitEvent(h->stream, so->done, 0);
            if (e != hipSuccess)
                return hip_fail(e, "gi_paged_decode_attention_noalloc: hipStreamWaitEvent");
        }
    } else {
        const int rc = gi::devbuf_reserve(h->plan_ws, need, h->stream, "decode attention");
        if (rc)
            return rc;
        a.ws = (float *)h->plan_ws.ptr;
    }
    if (new_k) {
        // a decode step: the token goes into the decode launch where that
        // pays (one round of workgroups), else into an append launch first
        if (gi::decode_fuses_append(h->L, batch, a.num_splits, h->num_cus)) {
            a.new_k = new_k;
            a.new_v = new_v;
        } else {
            const hipError_t e = gi::launch_append_at_len(h->L, a.append_base, batch, block_tables, max_blocks,
                                                          seq_lens, new_k, new_v, h->d_status, h->stream);
            if (e != hipSuccess)
                return hip_fail(e, "decode step: append");
        }
    }
    hipError_t e = gi::launch_decode(a, h->stream);
    if (e != hipSuccess)
        return hip_fail(e, "decode attention");
    if (eager) {
        ScratchOrder *so = h->scratch_order;
        e = hipEventRecord(so->done, h->stream);
        if (e != hipSuccess)
            return hip_fail(e, "gi_paged_decode_attention_noalloc: hipEventRecord");
        so->last = h->stream;
        so->recorded = true;
    }
    return GI_OK;
}

static int check_decode_args(gi_paged *h, int layer, int batch, int num_heads, const void *q,
                             const void *out, const int32_t *block_tables, int max_blocks,
                             const int32_t *seq_lens, int max_seq_len, float scale,
                             const char *what)
{
    int rc = check_layer(h, layer, what);
    if (rc)
        return rc;
    if (batch < 0 || max_seq_len < 0 || !std::isfinite(scale))
        return gi::set_error(GI_ERR_BAD_ARG, std::string(what) + ": bad argument");
    if (batch > 0 && (!q || !out || !block_tables || !seq_lens || max_blocks <= 0))
        return gi::set_error(GI_ERR_BAD_ARG, std::string(what) + ": NULL buffer or max_blocks <= 0");
    if (!supported_heads(h->L, num_heads))
        return gi::set_error(GI_ERR_BAD_ARG, std::string(what) +
                                                 ": unsupported head layout (head_dim 64/128, "
                                                 "num_heads/num_kv_heads in {1,2,4,8}, or 16 "
                                                 "with head_dim 128)");
    return GI_OK;
}

int gi_paged_decode_attention(gi_paged *h, int layer, int batch, int num_heads, const float *q,
                              float *out, const int32_t *block_tables, int max_blocks,
                              const int32_t *seq_lens, int max_seq_len, float scale)
{
    int rc = enter(h, "gi_paged_decode_attention");
    if (rc || (rc = check_decode_args(h, layer, batch, num_heads, q, out, block_tables, max_blocks,
                                      seq_lens, max_seq_len, scale, "gi_paged_decode_attention")))
        return rc;
    if (batch == 0)
        return GI_OK;
    std::lock_guard<std::mutex> g(h->mu);
    return decode_locked(h, layer, batch, num_heads, q, out, block_tables, max_blocks, seq_lens, max_seq_len, scale);
}

int gi_paged_decode_attention_noalloc(gi_paged *h, int layer, int batch, int num_heads, const float *q,
                                      float *out, const int32_t *block_tables, int max_blocks,
                                      const int32_t *seq_lens, int max_seq_len, float scale)
{
    int rc = enter(h, "gi_paged_decode_attention_noalloc");
    if (rc || (rc = check_decode_args(h, layer, batch, num_heads, q, out, block_tables, max_blocks, seq_lens,
                                      max_seq_len, scale, "gi_paged_decode_attention_noalloc")))
        return rc;
    if (batch == 0)
        return GI_OK;
    std::lock_guard<std::mutex> g(h->mu);
    return decode_locked(h, layer, batch, num_heads, q, out, block_tables, max_blocks, seq_lens, max_seq_len, scale,
                         h->scratch, kNoAllocScratchBytes);
}

int gi_paged_decode_step(gi_paged *h, int layer, int batch, int num_heads, const float *q,
                         const float *k, const float *v, float *out, const int32_t *block_tables,
                         int max_blocks, const int32_t *seq_lens, int max_seq_len, float scale)
{
    int rc = enter(h, "gi_paged_decode_step");
    if (rc || (rc = check_decode_args(h, layer, batch, num_heads, q, out, block_tables, max_blocks,
                                      seq_lens, max_seq_len, scale, "gi_paged_decode_step")))
        return rc;
    if (batch == 0)
        return GI_OK;
    if (!k || !v)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_decode_step: NULL k or v");
    std::lock_guard<std::mutex> g(h->mu);
    // the token is stored inside the decode launch, or by an append launch
    // before it (decode_fuses_append)
    return decode_locked(h, layer, batch, num_heads, q, out, block_tables, max_blocks, seq_lens, max_seq_len, scale,
                         nullptr, 0, k, v);
}

int gi_paged_rope_decode_step(gi_paged *h, int layer, int batch, int num_heads, float *q, const float *k,
                              const float *v, float *out, const int32_t *block_tables, int max_blocks,
                              const int32_t *seq_lens, int max_seq_len, float scale)
{
    int rc = enter(h, "gi_paged_rope_decode_step");
    if (rc || (rc = check_decode_args(h, layer, batch, num_heads, q, out, block_tables, max_blocks,
                                      seq_lens, max_seq_len, scale, "gi_paged_rope_decode_step")) ||
        (rc = check_rope(h, layer, batch, num_heads, q, q, k, v, "gi_paged_rope_decode_step")))
        return rc;
    if (batch == 0)
        return GI_OK;
    std::lock_guard<std::mutex> g(h->mu);
    hipError_t e = gi::launch_rope_append(h->L, h->layer_base[(size_t)layer], batch, nullptr, nullptr,
                                          block_tables, max_blocks, seq_lens,
                                          rope_args(h, num_heads, nullptr, q, q), k, v, h->d_status,
                                          h->stream);
    if (e != hipSuccess)
        return hip_fail(e, "gi_paged_rope_decode_step: rope + append");
    return decode_locked(h, layer, batch, num_heads, q, out, block_tables, max_blocks, seq_lens, max_seq_len, scale);
}

int gi_paged_prefill_attention(gi_paged *h, int layer, int batch, int chunk_len, int num_heads,
                               const float *q, float *out, const int32_t *block_tables,
                               int max_blocks, const int32_t *start_pos, float scale)
{
    int rc = enter(h, "gi_paged_prefill_attention");
    if (rc || (rc = check_decode_args(h, layer, batch, num_heads, q, out, block_tables, max_blocks,
                                      start_pos, 0, scale, "gi_paged_prefill_attention")))
        return rc;
    if (chunk_len < 0)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_prefill_attention: chunk_len < 0");
    if (batch == 0 || chunk_len == 0)
        return GI_OK;
    std::lock_guard<std::mutex> g(h->mu);
    gi::PrefillArgs p{};
    p.L = h->L;
    p.base = h->layer_base[(size_t)layer];
    p.q = q;
    p.out = out;
    p.block_tables = block_tables;
    p.max_blocks = max_blocks;
    p.start_pos = start_pos;
    p.batch = batch;
    p.chunk_len = chunk_len;
    p.num_heads = num_heads;
    p.scale = scale;
    p.status = h->d_status;
    p.kernel = h->decode_kernel;
    hipError_t e = gi::launch_prefill(p, h->stream);
    return e == hipSuccess ? GI_OK : hip_fail(e, "gi_paged_prefill_attention");
}

int gi_paged_decode_kernel(const gi_paged *h, int num_heads)
{
    if (!h)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_decode_kernel: NULL handle");
    return gi::decode_kernel_kind(h->L, num_heads, h->decode_kernel);
}

int gi_paged_attention_plan(const gi_paged *h, int batch, int num_heads, int max_seq_len,
                            gi_attention_plan *plan)
{
    if (!h || !plan || batch < 0 || max_seq_len < 0)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_attention_plan: bad argument");
    if (!supported_heads(h->L, num_heads))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_attention_plan: unsupported head layout");
    gi_attention_plan r{};
    const bool mfma_req = h->decode_kernel != 0;
    r.decode_kernel = gi::decode_kernel_kind(h->L, num_heads, h->decode_kernel);
    r.decode_fallback = mfma_req && r.decode_kernel == 0;
    gi::decode_plan(h->L, batch, num_heads, max_seq_len > 0 ? max_seq_len : 1, h->num_cus,
                    &r.decode_split_tokens, &r.decode_splits);
    r.decode_waves = r.decode_kernel == 1 ? gi::decode_waves(h->L, batch, r.decode_splits, h->num_cus) : 0;
    r.decode_step_fused = r.decode_kernel == 1 && gi::decode_fuses_append(h->L, batch, r.decode_splits, h->num_cus);
    r.prefill_kernel = mfma_req && gi::mfma_prefill_supported(h->L, num_heads) ? 1 : 0;
    r.prefill_fallback = mfma_req && r.prefill_kernel == 0;
    *plan = r;
    return GI_OK;
}

int gi_paged_set_decode_kernel(gi_paged *h, int kind)
{
    if (!h || kind < -1 || kind > 1)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_paged_set_decode_kernel: bad argument");
    std::lock_guard<std::mutex> g(h->mu);
    h->decode_kernel = kind;
    return GI_OK;
}

} // extern "C"
