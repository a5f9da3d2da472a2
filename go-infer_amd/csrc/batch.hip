// Continuous-batching decode driver over one block allocator and one page
// pool (the C ABI is include/goinfer_paged.h, gi_batch_*).
//
// The reference decodes one sequence at a time under Engine.mu
// (pkg/engine/engine.go:417): each token runs Forward for that sequence
// alone, and PagedKVManager (pkg/engine/paged_kv.go:49-148) is never used by
// it.  Here a running set of sequences steps together: one AppendToken per
// sequence per step (all or nothing, gi_kvmgr_append_batch), then every
// layer's RoPE + append + paged attention runs once for the whole set.
//
// The block tables and lengths of the running set stay resident on the
// device as a dense [max_batch][max_blocks] int32 table.  A step changes at
// most one entry per sequence (a new block at a block boundary, or the fresh
// copy that replaces a shared last block), so it uploads only those entries
// and the lengths, and a small kernel scatters the entries into the table.
// Removing a sequence moves the last row into its place, so rows 0..n-1
// stay dense.  Page copies of copy-on-write appends are queued on the pool's
// stream before the layers that read the pages.
#include "../../include/goinfer_paged.h"
#include "gi_host.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <new>
#include <string>
#include <vector>

namespace {

// dst[pairs[2i]] = pairs[2i+1] for i < n (indices checked on the host).
__global__ __launch_bounds__(256) void scatter_entries(int32_t *__restrict__ dst,
                                                      const int32_t *__restrict__ pairs, int n)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n)
        dst[pairs[2 * i]] = pairs[2 * i + 1];
}

} // namespace

struct gi_batch {
    std::mutex mu;
    gi_kvmgr *m = nullptr;
    gi_paged *h = nullptr; // NULL: host bookkeeping only
    int device = 0;        // frees need only this, so destroy does not use h
    int max_batch = 0;
    int max_blocks = 0;
    int page_tokens = 16;
    std::vector<int> seqs;                  // row -> sequence id
    std::vector<std::vector<int32_t>> rows; // row -> block ids (host mirror)
    std::vector<int32_t> lens;              // row -> tokens
    // device
    int32_t *d_tables = nullptr; // [max_batch][max_blocks]
    int32_t *d_lens = nullptr;   // [max_batch]
    int32_t *d_pairs = nullptr;  // [2 * max_batch] (index, value) updates
    int32_t *d_copy = nullptr;   // [2 * max_batch] copy sources, then destinations
    // pinned staging: a ring of slots, each reused once the event of its
    // last upload has passed, so the host may run a few steps ahead of the
    // device.  A slot holds 2*max_batch pairs + max_batch lengths +
    // 2*max_batch copies, or one table row + the lengths.
    static constexpr int kSlots = 4;
    int32_t *h_stage = nullptr;
    size_t slot_ints = 0;
    int slot = 0;
    hipEvent_t staged[kSlots] = {};
    bool staged_pending[kSlots] = {};
};

namespace {

int fail(int code, const std::string &m) { return gi::set_error(code, m); }

int hip_check(hipError_t e, const char *what)
{
    return e == hipSuccess ? GI_OK : fail(GI_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

hipStream_t stream_of(gi_batch *b) { return (hipStream_t)gi_paged_stream(b->h); }

// Takes the next staging slot, waiting if it still feeds an earlier upload.
int stage_ready(gi_batch *b, int32_t **buf)
{
    b->slot = (b->slot + 1) % gi_batch::kSlots;
    *buf = b->h_stage + (size_t)b->slot * b->slot_ints;
    if (!b->staged_pending[b->slot])
        return GI_OK;
    b->staged_pending[b->slot] = false;
    return hip_check(hipEventSynchronize(b->staged[b->slot]), "gi_batch: staging");
}

// Marks the current slot busy until the uploads queued so far are done.
int stage_done(gi_batch *b)
{
    int rc = hip_check(hipEventRecord(b->staged[b->slot], stream_of(b)), "gi_batch: staging");
    if (rc == GI_OK)
        b->staged_pending[b->slot] = true;
    return rc;
}

// Uploads one whole table row and every length.
int upload_row(gi_batch *b, int r)
{
    if (!b->h)
        return GI_OK;
    int32_t *row;
    int rc = stage_ready(b, &row);
    if (rc)
        return rc;
    const std::vector<int32_t> &ids = b->rows[(size_t)r];
    for (int c = 0; c < b->max_blocks; c++)
        row[c] = c < (int)ids.size() ? ids[(size_t)c] : 0;
    hipStream_t st = stream_of(b);
    hipError_t e = hipMemcpyAsync(b->d_tables + (size_t)r * b->max_blocks, row,
                                  sizeof(int32_t) * (size_t)b->max_blocks, hipMemcpyHostToDevice, st);
    if (e == hipSuccess && !b->lens.empty()) {
        std::copy(b->lens.begin(), b->lens.end(), row + b->max_blocks);
        e = hipMemcpyAsync(b->d_lens, row + b->max_blocks, sizeof(int32_t) * b->lens.size(),
                           hipMemcpyHostToDevice, st);
    }
    if ((rc = hip_check(e, "gi_batch: upload")))
        return rc;
    return stage_done(b);
}

int find_row(const gi_batch *b, int seq_id)
{
    for (size_t r = 0; r < b->seqs.size(); r++)
        if (b->seqs[r] == seq_id)
            return (int)r;
    return -1;
}

} // namespace

extern "C" {

int gi_batch_create(gi_kvmgr *m, gi_paged *h, int max_batch, int max_blocks, gi_batch **out)
{
    if (!out)
        return fail(GI_ERR_BAD_ARG, "gi_batch_create: out is NULL");
    *out = nullptr;
    if (!m || max_batch <= 0 || max_blocks <= 0)
        return fail(GI_ERR_BAD_ARG, "gi_batch_create: need a manager, max_batch > 0, max_blocks > 0");
    gi_batch *b = new (std::nothrow) gi_batch();
    if (!b)
        return fail(GI_ERR_OOM, "gi_batch_create: out of host memory");
    b->m = m;
    b->h = h;
    b->max_batch = max_batch;
    b->max_blocks = max_blocks;
    b->page_tokens = gi_kvmgr_block_size(m);
    int rc = GI_OK;
    if (h) {
        const size_t tb = sizeof(int32_t) * (size_t)max_batch * (size_t)max_blocks;
        b->slot_ints = (size_t)max_batch * 5 + (size_t)max_blocks;
        const size_t stage = sizeof(int32_t) * b->slot_ints * gi_batch::kSlots;
        void *p = nullptr;
        if ((rc = gi_dev_alloc(h, tb, &p)) == GI_OK) {
            b->d_tables = (int32_t *)p;
            (void)hipGetDevice(&b->device); // the pool's, made current by gi_dev_alloc
            if ((rc = gi_dev_alloc(h, sizeof(int32_t) * (size_t)max_batch, &p)) == GI_OK)
                b->d_lens = (int32_t *)p;
        }
        if (rc == GI_OK && (rc = gi_dev_alloc(h, sizeof(int32_t) * 2 * (size_t)max_batch, &p)) == GI_OK)
            b->d_pairs = (int32_t *)p;
        if (rc == GI_OK && (rc = gi_dev_alloc(h, sizeof(int32_t) * 2 * (size_t)max_batch, &p)) == GI_OK)
            b->d_copy = (int32_t *)p;
        if (rc == GI_OK && hipHostMalloc((void **)&b->h_stage, stage, hipHostMallocDefault) != hipSuccess) {
            b->h_stage = nullptr;
            rc = fail(GI_ERR_OOM, "gi_batch_create: pinned staging");
        }
        for (int i = 0; rc == GI_OK && i < gi_batch::kSlots; i++)
            rc = hip_check(hipEventCreateWithFlags(&b->staged[i], hipEventDisableTiming), "gi_batch_create");
        if (rc == GI_OK)
            rc = hip_check(hipMemsetAsync(b->d_tables, 0, tb, stream_of(b)), "gi_batch_create");
        if (rc == GI_OK)
            rc = hip_check(hipMemsetAsync(b->d_lens, 0, sizeof(int32_t) * (size_t)max_batch, stream_of(b)),
                           "gi_batch_create");
    }
    if (rc != GI_OK) {
        gi_batch_destroy(b);
        return rc;
    }
    *out = b;
    return GI_OK;
}

void gi_batch_destroy(gi_batch *b)
{
    if (!b)
        return;
    if (b->h) {
        // Does not touch the pool handle, which may be gone already; waits
        // for the device's queued work (uploads, kernels reading the tables).
        if (hipSetDevice(b->device) == hipSuccess)
            (void)hipDeviceSynchronize();
        for (int32_t *p : {b->d_tables, b->d_lens, b->d_pairs, b->d_copy})
            if (p)
                (void)hipFree(p);
        if (b->h_stage)
            (void)hipHostFree(b->h_stage);
        for (hipEvent_t e : b->staged)
            if (e)
                (void)hipEventDestroy(e);
    }
    delete b;
}

int gi_batch_add(gi_batch *b, int seq_id, int *row)
{
    if (!b)
        return fail(GI_ERR_BAD_ARG, "gi_batch_add: NULL handle");
    std::lock_guard<std::mutex> g(b->mu);
    if (find_row(b, seq_id) >= 0)
        return fail(GI_ERR_BAD_ARG, "gi_batch_add: sequence " + std::to_string(seq_id) + " is already running");
    if ((int)b->seqs.size() >= b->max_batch)
        return fail(GI_ERR_BAD_ARG, "gi_batch_add: the batch is full (" + std::to_string(b->max_batch) + ")");
    int nb = 0, nt = 0;
    int rc = gi_kvmgr_block_table(b->m, seq_id, nullptr, 0, &nb, &nt);
    if (rc)
        return rc;
    if (nb > b->max_blocks)
        return fail(GI_ERR_BAD_ARG, "gi_batch_add: sequence " + std::to_string(seq_id) + " holds " +
                                        std::to_string(nb) + " blocks, more than max_blocks");
    std::vector<int32_t> ids((size_t)nb);
    if (nb > 0 && (rc = gi_kvmgr_block_table(b->m, seq_id, ids.data(), nb, &nb, &nt)))
        return rc;
    b->seqs.push_back(seq_id);
    b->rows.push_back(std::move(ids));
    b->lens.push_back(nt);
    const int r = (int)b->seqs.size() - 1;
    if (row)
        *row = r;
    return upload_row(b, r);
}

int gi_batch_remove(gi_batch *b, int seq_id)
{
    if (!b)
        return fail(GI_ERR_BAD_ARG, "gi_batch_remove: NULL handle");
    std::lock_guard<std::mutex> g(b->mu);
    const int r = find_row(b, seq_id);
    if (r < 0)
        return fail(GI_ERR_UNKNOWN_SEQ, "gi_batch_remove: sequence " + std::to_string(seq_id) + " is not running");
    const int last = (int)b->seqs.size() - 1;
    if (r != last) {
        b->seqs[(size_t)r] = b->seqs[(size_t)last];
        b->rows[(size_t)r] = std::move(b->rows[(size_t)last]);
        b->lens[(size_t)r] = b->lens[(size_t)last];
    }
    b->seqs.pop_back();
    b->rows.pop_back();
    b->lens.pop_back();
    if (r != last)
        return upload_row(b, r);
    if (!b->h || b->lens.empty())
        return GI_OK;
    int32_t *buf;
    int rc = stage_ready(b, &buf);
    if (rc)
        return rc;
    std::copy(b->lens.begin(), b->lens.end(), buf);
    rc = hip_check(hipMemcpyAsync(b->d_lens, buf, sizeof(int32_t) * b->lens.size(),
                                  hipMemcpyHostToDevice, stream_of(b)),
                   "gi_batch_remove: upload");
    return rc ? rc : stage_done(b);
}

int gi_batch_step(gi_batch *b, int *n_rows)
{
    if (n_rows)
        *n_rows = 0;
    if (!b)
        return fail(GI_ERR_BAD_ARG, "gi_batch_step: NULL handle");
    std::lock_guard<std::mutex> g(b->mu);
    const int n = (int)b->seqs.size();
    if (n == 0)
        return GI_OK;
    for (int r = 0; r < n; r++)
        if ((int64_t)b->lens[(size_t)r] + 1 > (int64_t)b->max_blocks * b->page_tokens)
            return fail(GI_ERR_BAD_ARG, "gi_batch_step: sequence " + std::to_string(b->seqs[(size_t)r]) +
                                            " would outgrow max_blocks");
    std::vector<int32_t> ids((size_t)n), slots((size_t)n), from((size_t)n);
    int rc = gi_kvmgr_append_batch(b->m, n, b->seqs.data(), ids.data(), slots.data(), from.data());
    if (rc)
        return rc;
    // host mirror, and the table entries that changed
    std::vector<int32_t> pairs, csrc, cdst;
    for (int r = 0; r < n; r++) {
        std::vector<int32_t> &row = b->rows[(size_t)r];
        if (slots[(size_t)r] == 0 && (int)row.size() * b->page_tokens == b->lens[(size_t)r]) {
            row.push_back(ids[(size_t)r]); // a new block
        } else if (from[(size_t)r] >= 0) {
            row.back() = ids[(size_t)r]; // the fresh copy of a shared block
            csrc.push_back(from[(size_t)r]);
            cdst.push_back(ids[(size_t)r]);
        } else {
            b->lens[(size_t)r]++;
            continue;
        }
        b->lens[(size_t)r]++;
        pairs.push_back(r * b->max_blocks + (int)row.size() - 1);
        pairs.push_back(ids[(size_t)r]);
    }
    if (n_rows)
        *n_rows = n;
    if (!b->h)
        return GI_OK;
    int32_t *sp;
    if ((rc = stage_ready(b, &sp)))
        return rc;
    hipStream_t st = stream_of(b);
    int32_t *sl = sp + 2 * b->max_batch, *sc = sl + b->max_batch;
    std::copy(pairs.begin(), pairs.end(), sp);
    std::copy(b->lens.begin(), b->lens.end(), sl);
    const int np = (int)pairs.size() / 2, nc = (int)csrc.size();
    std::copy(csrc.begin(), csrc.end(), sc);
    std::copy(cdst.begin(), cdst.end(), sc + b->max_batch);
    hipError_t e = hipSuccess;
    if (np > 0) {
        e = hipMemcpyAsync(b->d_pairs, sp, sizeof(int32_t) * 2 * (size_t)np, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) {
            hipLaunchKernelGGL(scatter_entries, dim3((unsigned)((np + 255) / 256)), dim3(256), 0, st, b->d_tables,
                               b->d_pairs, np);
            e = hipGetLastError();
        }
    }
    if (e == hipSuccess)
        e = hipMemcpyAsync(b->d_lens, sl, sizeof(int32_t) * (size_t)n, hipMemcpyHostToDevice, st);
    if (e == hipSuccess && nc > 0)
        e = hipMemcpyAsync(b->d_copy, sc, sizeof(int32_t) * 2 * (size_t)b->max_batch, hipMemcpyHostToDevice, st);
    if ((rc = hip_check(e, "gi_batch_step: upload")))
        return rc;
    if ((rc = stage_done(b)))
        return rc;
    if (nc > 0 && (rc = gi_paged_copy_pages(b->h, nc, b->d_copy, b->d_copy + b->max_batch)))
        return rc;
    return GI_OK;
}

int gi_batch_rows(gi_batch *b, int32_t *seq_ids, int32_t *seq_lens, int cap, int *n)
{
    if (!b || !n)
        return fail(GI_ERR_BAD_ARG, "gi_batch_rows: NULL argument");
    std::lock_guard<std::mutex> g(b->mu);
    *n = (int)b->seqs.size();
    for (int r = 0; r < *n && r < cap; r++) {
        if (seq_ids)
            seq_ids[r] = b->seqs[(size_t)r];
        if (seq_lens)
            seq_lens[r] = b->lens[(size_t)r];
    }
    return GI_OK;
}

int gi_batch_row_table(gi_batch *b, int row, int32_t *ids, int cap, int *n_blocks)
{
    if (!b || !n_blocks)
        return fail(GI_ERR_BAD_ARG, "gi_batch_row_table: NULL argument");
    std::lock_guard<std::mutex> g(b->mu);
    if (row < 0 || row >= (int)b->seqs.size())
        return fail(GI_ERR_BAD_ARG, "gi_batch_row_table: row out of range");
    const std::vector<int32_t> &v = b->rows[(size_t)row];
    *n_blocks = (int)v.size();
    for (int c = 0; c < (int)v.size() && c < cap; c++)
        ids[c] = v[(size_t)c];
    return GI_OK;
}

int gi_batch_device_tables(gi_batch *b, int32_t **block_tables, int32_t **seq_lens, int *max_blocks)
{
    if (!b || !b->h)
        return fail(GI_ERR_BAD_ARG, "gi_batch_device_tables: no device pool");
    if (block_tables)
        *block_tables = b->d_tables;
    if (seq_lens)
        *seq_lens = b->d_lens;
    if (max_blocks)
        *max_blocks = b->max_blocks;
    return GI_OK;
}

int gi_batch_decode_layer(gi_batch *b, int layer, int num_heads, float *q, const float *k, const float *v,
                          float *out, float scale, int rope)
{
    if (!b || !b->h)
        return fail(GI_ERR_BAD_ARG, "gi_batch_decode_layer: no device pool");
    int n, max_len = 0;
    {
        std::lock_guard<std::mutex> g(b->mu);
        n = (int)b->seqs.size();
        for (int32_t l : b->lens)
            max_len = std::max(max_len, (int)l);
    }
    if (n == 0)
        return GI_OK;
    if (rope)
        return gi_paged_rope_decode_step(b->h, layer, n, num_heads, q, k, v, out, b->d_tables, b->max_blocks,
                                         b->d_lens, max_len, scale);
    return gi_paged_decode_step(b->h, layer, n, num_heads, q, k, v, out, b->d_tables, b->max_blocks, b->d_lens,
                                max_len, scale);
}

} // extern "C"
