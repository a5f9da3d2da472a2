// Host block allocator: the C++ form of go-infer's PagedKVManager
// (pkg/engine/paged_kv.go:49-148).  It stays on the host, as in the
// reference; the device path consumes the int32 block tables it produces.
//
//   FreeBlocks starts as [0..N) (paged_kv.go:70-74) and is a stack: a
//   sequence that needs a block pops the tail (122-123), FreeSequence pushes
//   a table's ids back in table order (144-146).  Sequence ids start at 1
//   (85).  A sequence needs NumTokens/BlockSize + 1 blocks before a token is
//   placed (116-117) and the token goes to (last block, NumTokens %
//   BlockSize) (127-131).  One mutex guards the manager (paged_kv.go:50).
#include "../../include/goinfer_paged.h"
#include "gi_host.h"

#include <mutex>
#include <new>
#include <unordered_map>
#include <vector>

struct gi_kvmgr {
    std::mutex mu;
    int num_layers = 0;
    int kv_dim = 0;
    int block_size = 16;
    int total_blocks = 256;
    std::vector<int32_t> free_blocks;
    struct Table {
        std::vector<int32_t> ids;
        int num_tokens = 0;
    };
    std::unordered_map<int, Table> tables;
    int next_seq = 1;
};

namespace {

// AppendToken body; caller holds the lock.
int append_locked(gi_kvmgr *m, gi_kvmgr::Table &t, int seq_id, int32_t *block_id, int32_t *slot)
{
    (void)seq_id;
    size_t needed = (size_t)(t.num_tokens / m->block_size) + 1;
    if (t.ids.size() < needed) {
        if (m->free_blocks.empty())
            return gi::set_error(GI_ERR_POOL_EXHAUSTED,
                                 "out of paged KV memory (no free blocks available)");
        t.ids.push_back(m->free_blocks.back());
        m->free_blocks.pop_back();
    }
    *block_id = t.ids.back();
    *slot = t.num_tokens % m->block_size;
    t.num_tokens++;
    return GI_OK;
}

} // namespace

extern "C" {

int gi_kvmgr_create(int num_layers, int kv_dim, int total_blocks, int block_size, gi_kvmgr **out)
{
    if (!out)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_create: out is NULL");
    *out = nullptr;
    if (block_size <= 0)
        block_size = 16; // DefaultBlockTokens (paged_kv.go:8-10, 63-65)
    if (total_blocks <= 0)
        total_blocks = 256; // paged_kv.go:66-68
    gi_kvmgr *m = new (std::nothrow) gi_kvmgr();
    if (!m)
        return gi::set_error(GI_ERR_OOM, "gi_kvmgr_create: out of host memory");
    m->num_layers = num_layers;
    m->kv_dim = kv_dim;
    m->block_size = block_size;
    m->total_blocks = total_blocks;
    try {
        m->free_blocks.resize((size_t)total_blocks);
    } catch (...) {
        delete m;
        return gi::set_error(GI_ERR_OOM, "gi_kvmgr_create: out of host memory");
    }
    for (int i = 0; i < total_blocks; i++)
        m->free_blocks[(size_t)i] = i;
    *out = m;
    gi::clear_error();
    return GI_OK;
}

void gi_kvmgr_destroy(gi_kvmgr *m) { delete m; }

int gi_kvmgr_allocate_sequence(gi_kvmgr *m, int *seq_id)
{
    if (!m || !seq_id)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_allocate_sequence: NULL argument");
    std::lock_guard<std::mutex> g(m->mu);
    int id = m->next_seq++;
    m->tables[id] = gi_kvmgr::Table{};
    m->tables[id].ids.reserve(8);
    *seq_id = id;
    return GI_OK;
}

int gi_kvmgr_append_token(gi_kvmgr *m, int seq_id, int32_t *block_id, int32_t *slot)
{
    if (!m || !block_id || !slot)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_append_token: NULL argument");
    std::lock_guard<std::mutex> g(m->mu);
    auto it = m->tables.find(seq_id);
    if (it == m->tables.end())
        return gi::set_error(GI_ERR_UNKNOWN_SEQ, "sequence " + std::to_string(seq_id) + " not found");
    return append_locked(m, it->second, seq_id, block_id, slot);
}

int gi_kvmgr_append_tokens(gi_kvmgr *m, int seq_id, int n, int32_t *block_ids, int32_t *slots,
                           int *done)
{
    if (done)
        *done = 0;
    if (!m || n < 0 || (n > 0 && (!block_ids || !slots)))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_append_tokens: bad argument");
    std::lock_guard<std::mutex> g(m->mu);
    auto it = m->tables.find(seq_id);
    if (it == m->tables.end())
        return gi::set_error(GI_ERR_UNKNOWN_SEQ, "sequence " + std::to_string(seq_id) + " not found");
    for (int i = 0; i < n; i++) {
        int rc = append_locked(m, it->second, seq_id, block_ids + i, slots + i);
        if (rc != GI_OK)
            return rc;
        if (done)
            *done = i + 1;
    }
    return GI_OK;
}

int gi_kvmgr_free_sequence(gi_kvmgr *m, int seq_id)
{
    if (!m)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_free_sequence: NULL manager");
    std::lock_guard<std::mutex> g(m->mu);
    auto it = m->tables.find(seq_id);
    if (it == m->tables.end())
        return GI_OK; // paged_kv.go:139-142: unknown ids are ignored
    for (int32_t id : it->second.ids)
        m->free_blocks.push_back(id);
    m->tables.erase(it);
    return GI_OK;
}

int gi_kvmgr_block_table(gi_kvmgr *m, int seq_id, int32_t *ids, int cap, int *n_blocks,
                         int *n_tokens)
{
    if (!m || (cap > 0 && !ids))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_block_table: bad argument");
    std::lock_guard<std::mutex> g(m->mu);
    auto it = m->tables.find(seq_id);
    if (it == m->tables.end())
        return gi::set_error(GI_ERR_UNKNOWN_SEQ, "sequence " + std::to_string(seq_id) + " not found");
    const auto &t = it->second;
    int n = (int)t.ids.size();
    for (int i = 0; i < n && i < cap; i++)
        ids[i] = t.ids[(size_t)i];
    if (n_blocks)
        *n_blocks = n;
    if (n_tokens)
        *n_tokens = t.num_tokens;
    return GI_OK;
}

int gi_kvmgr_free_list(gi_kvmgr *m, int32_t *ids, int cap, int *n)
{
    if (!m || (cap > 0 && !ids))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_free_list: bad argument");
    std::lock_guard<std::mutex> g(m->mu);
    int k = (int)m->free_blocks.size();
    for (int i = 0; i < k && i < cap; i++)
        ids[i] = m->free_blocks[(size_t)i];
    if (n)
        *n = k;
    return GI_OK;
}

int gi_kvmgr_set_free_list(gi_kvmgr *m, const int32_t *ids, int n)
{
    if (!m || n < 0 || (n > 0 && !ids))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_set_free_list: bad argument");
    std::lock_guard<std::mutex> g(m->mu);
    std::vector<char> used((size_t)m->total_blocks, 0);
    for (const auto &kv : m->tables)
        for (int32_t id : kv.second.ids)
            used[(size_t)id] = 1;
    for (int i = 0; i < n; i++) {
        int32_t id = ids[i];
        if (id < 0 || id >= m->total_blocks || used[(size_t)id])
            return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_set_free_list: id " + std::to_string(id) +
                                                     " out of range, repeated or in use");
        used[(size_t)id] = 1;
    }
    m->free_blocks.assign(ids, ids + n);
    return GI_OK;
}

} // extern "C"
