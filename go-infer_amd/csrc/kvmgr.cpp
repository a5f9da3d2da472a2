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
//
// Beyond the reference, blocks carry reference counts so that sequences can
// share the pages of a common prefix (fork / prefix cache) instead of deep
// copying them (kvcache.go:217-284, prefix_cache.go:122-150); a block goes
// back to the free list when its last reference is dropped, and an append
// into a block that is still shared first moves the sequence to a fresh copy.
#include "../../include/goinfer_paged.h"
#include "gi_host.h"

#include <algorithm>
#include <deque>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

struct gi_kvmgr {
    std::mutex mu;
    int num_layers = 0;
    int kv_dim = 0;
    int block_size = 16;
    int total_blocks = 256;
    std::vector<int32_t> free_blocks;
    std::vector<uint32_t> refs; // references per block (sequences holding it)
    struct Table {
        std::vector<int32_t> ids;
        int num_tokens = 0;
    };
    std::unordered_map<int, Table> tables;
    int next_seq = 1;
};

namespace {

int pop_free(gi_kvmgr *m, int32_t *id)
{
    if (m->free_blocks.empty())
        return gi::set_error(GI_ERR_POOL_EXHAUSTED, "out of paged KV memory (no free blocks available)");
    *id = m->free_blocks.back();
    m->free_blocks.pop_back();
    m->refs[(size_t)*id] = 1;
    return GI_OK;
}

// AppendToken body; caller holds the lock.  The token goes to slot
// num_tokens % block_size of the last block, which is new when the sequence
// needs one.  An existing last block with other references is copied first
// when copy_from is given (*copy_from = the shared block), and refused with
// GI_ERR_SHARED_PAGE when it is not.
int append_locked(gi_kvmgr *m, gi_kvmgr::Table &t, int seq_id, int32_t *block_id, int32_t *slot,
                  int32_t *copy_from)
{
    if (copy_from)
        *copy_from = -1;
    size_t needed = (size_t)(t.num_tokens / m->block_size) + 1;
    if (t.ids.size() < needed) {
        int32_t id;
        int rc = pop_free(m, &id);
        if (rc)
            return rc;
        t.ids.push_back(id);
    } else if (m->refs[(size_t)t.ids.back()] > 1) {
        if (!copy_from)
            return gi::set_error(GI_ERR_SHARED_PAGE,
                                 "sequence " + std::to_string(seq_id) +
                                     ": the block to append into is shared; use the copy-on-write append");
        int32_t id;
        int rc = pop_free(m, &id);
        if (rc)
            return rc;
        *copy_from = t.ids.back();
        m->refs[(size_t)t.ids.back()]--;
        t.ids.back() = id;
    }
    *block_id = t.ids.back();
    *slot = t.num_tokens % m->block_size;
    t.num_tokens++;
    return GI_OK;
}

// Drops one reference on each block of a table, returning the blocks that
// reach zero to the free list in table order (paged_kv.go:144-146).
void release_locked(gi_kvmgr *m, const gi_kvmgr::Table &t)
{
    for (int32_t id : t.ids)
        if (--m->refs[(size_t)id] == 0)
            m->free_blocks.push_back(id);
}

int fork_locked(gi_kvmgr *m, int src_seq, int n_tokens, int *new_seq)
{
    auto it = m->tables.find(src_seq);
    if (it == m->tables.end())
        return gi::set_error(GI_ERR_UNKNOWN_SEQ, "sequence " + std::to_string(src_seq) + " not found");
    const gi_kvmgr::Table &src = it->second;
    if (n_tokens > src.num_tokens)
        n_tokens = src.num_tokens;
    if (n_tokens < 0)
        n_tokens = 0;
    gi_kvmgr::Table t;
    const size_t nb = (size_t)((n_tokens + m->block_size - 1) / m->block_size);
    t.ids.assign(src.ids.begin(), src.ids.begin() + (ptrdiff_t)nb);
    t.num_tokens = n_tokens;
    for (int32_t id : t.ids)
        m->refs[(size_t)id]++;
    const int id = m->next_seq++;
    m->tables[id] = std::move(t);
    *new_seq = id;
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
        m->refs.assign((size_t)total_blocks, 0u);
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
    return append_locked(m, it->second, seq_id, block_id, slot, nullptr);
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
        int rc = append_locked(m, it->second, seq_id, block_ids + i, slots + i, nullptr);
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
    release_locked(m, it->second);
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
    for (int i = 0; i < m->total_blocks; i++)
        used[(size_t)i] = m->refs[(size_t)i] > 0;
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

int gi_kvmgr_fork_sequence(gi_kvmgr *m, int src_seq, int n_tokens, int *new_seq)
{
    if (!m || !new_seq)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_fork_sequence: NULL argument");
    std::lock_guard<std::mutex> g(m->mu);
    return fork_locked(m, src_seq, n_tokens, new_seq);
}

int gi_kvmgr_append_token_cow(gi_kvmgr *m, int seq_id, int32_t *block_id, int32_t *slot,
                              int32_t *copy_from)
{
    if (!m || !block_id || !slot || !copy_from)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_append_token_cow: NULL argument");
    std::lock_guard<std::mutex> g(m->mu);
    auto it = m->tables.find(seq_id);
    if (it == m->tables.end())
        return gi::set_error(GI_ERR_UNKNOWN_SEQ, "sequence " + std::to_string(seq_id) + " not found");
    return append_locked(m, it->second, seq_id, block_id, slot, copy_from);
}

int gi_kvmgr_append_tokens_cow(gi_kvmgr *m, int seq_id, int n, int32_t *block_ids,
                               int32_t *slots, int32_t *copy_src, int32_t *copy_dst, int *done)
{
    if (done)
        *done = 0;
    if (copy_src)
        *copy_src = -1;
    if (copy_dst)
        *copy_dst = -1;
    if (!m || n < 0 || (n > 0 && (!block_ids || !slots)) || !copy_src || !copy_dst)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_append_tokens_cow: bad argument");
    std::lock_guard<std::mutex> g(m->mu);
    auto it = m->tables.find(seq_id);
    if (it == m->tables.end())
        return gi::set_error(GI_ERR_UNKNOWN_SEQ, "sequence " + std::to_string(seq_id) + " not found");
    for (int i = 0; i < n; i++) {
        int32_t from = -1;
        int rc = append_locked(m, it->second, seq_id, block_ids + i, slots + i, &from);
        if (rc != GI_OK)
            return rc;
        if (from >= 0) {
            *copy_src = from;
            *copy_dst = block_ids[i];
        }
        if (done)
            *done = i + 1;
    }
    return GI_OK;
}

int gi_kvmgr_block_size(const gi_kvmgr *m) { return m ? m->block_size : 0; }

int gi_kvmgr_append_batch(gi_kvmgr *m, int n, const int *seq_ids, int32_t *block_ids, int32_t *slots,
                          int32_t *copy_src)
{
    if (!m || n < 0 || (n > 0 && (!seq_ids || !block_ids || !slots || !copy_src)))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_append_batch: bad argument");
    std::lock_guard<std::mutex> g(m->mu);
    // Check every sequence and count the blocks the step takes before
    // changing anything: a new block at a block boundary, a fresh copy of a
    // shared last block.
    // A last block shared by c sequences of the step and held r times takes
    // min(c, r - 1) copies: each copy drops a reference, and the last holder
    // writes in place.
    std::vector<gi_kvmgr::Table *> ts((size_t)n);
    std::unordered_map<int, int> seen;
    std::unordered_map<int32_t, uint32_t> sharers; // shared last block -> sequences of the step
    size_t need = 0;
    for (int i = 0; i < n; i++) {
        auto it = m->tables.find(seq_ids[i]);
        if (it == m->tables.end())
            return gi::set_error(GI_ERR_UNKNOWN_SEQ, "sequence " + std::to_string(seq_ids[i]) + " not found");
        if (!seen.emplace(seq_ids[i], i).second)
            return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_append_batch: sequence " +
                                                     std::to_string(seq_ids[i]) + " listed twice");
        gi_kvmgr::Table &t = it->second;
        ts[(size_t)i] = &t;
        if (t.ids.size() < (size_t)(t.num_tokens / m->block_size) + 1)
            need++;
        else if (m->refs[(size_t)t.ids.back()] > 1)
            sharers[t.ids.back()]++;
    }
    for (const auto &kv : sharers)
        need += std::min<size_t>(kv.second, m->refs[(size_t)kv.first] - 1);
    if (need > m->free_blocks.size())
        return gi::set_error(GI_ERR_POOL_EXHAUSTED, "out of paged KV memory (the step needs " +
                                                        std::to_string(need) + " blocks, " +
                                                        std::to_string(m->free_blocks.size()) + " free)");
    for (int i = 0; i < n; i++) {
        int rc = append_locked(m, *ts[(size_t)i], seq_ids[i], block_ids + i, slots + i, copy_src + i);
        if (rc != GI_OK) // cannot happen after the checks above
            return rc;
    }
    return GI_OK;
}

int gi_kvmgr_block_refs(gi_kvmgr *m, int32_t block_id, int *refs)
{
    if (!m || !refs)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_block_refs: NULL argument");
    std::lock_guard<std::mutex> g(m->mu);
    if (block_id < 0 || block_id >= m->total_blocks)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_kvmgr_block_refs: block id out of range");
    *refs = (int)m->refs[(size_t)block_id];
    return GI_OK;
}

} // extern "C"

// ---- PrefixCache over shared pages (prefix_cache.go:7-150) ----------------
//
// Each entry keeps a sequence forked from the stored one, so its pages stay
// referenced; a lookup forks that sequence again.  Keys are the token ids
// themselves (the reference joins them into a string, tokensKey, 32-41).

struct gi_prefix {
    std::mutex mu;
    gi_kvmgr *m = nullptr;
    int max_size = 32;
    std::unordered_map<std::string, int> entries; // key -> pinned sequence
    std::deque<std::string> order;                 // insertion order, for eviction
};

namespace {

std::string prefix_key(const int32_t *tokens, int n)
{
    return std::string(reinterpret_cast<const char *>(tokens), (size_t)n * sizeof(int32_t));
}

// Drops the entry under key (its pinned sequence included); caller holds both locks.
void prefix_drop_locked(gi_prefix *pc, const std::string &key)
{
    auto it = pc->entries.find(key);
    if (it == pc->entries.end())
        return;
    auto t = pc->m->tables.find(it->second);
    if (t != pc->m->tables.end()) {
        release_locked(pc->m, t->second);
        pc->m->tables.erase(t);
    }
    pc->entries.erase(it);
    for (auto o = pc->order.begin(); o != pc->order.end(); ++o)
        if (*o == key) {
            pc->order.erase(o);
            break;
        }
}

} // namespace

extern "C" {

int gi_prefix_create(gi_kvmgr *m, int max_size, gi_prefix **out)
{
    if (!out || !m)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_prefix_create: NULL argument");
    *out = nullptr;
    gi_prefix *pc = new (std::nothrow) gi_prefix();
    if (!pc)
        return gi::set_error(GI_ERR_OOM, "gi_prefix_create: out of host memory");
    pc->m = m;
    pc->max_size = max_size > 0 ? max_size : 32; // NewPrefixCache (prefix_cache.go:20-28)
    *out = pc;
    return GI_OK;
}

void gi_prefix_destroy(gi_prefix *pc)
{
    if (!pc)
        return;
    {
        std::lock_guard<std::mutex> g(pc->mu);
        std::lock_guard<std::mutex> gm(pc->m->mu);
        while (!pc->order.empty()) {
            const std::string key = pc->order.front();
            prefix_drop_locked(pc, key);
        }
    }
    delete pc;
}

int gi_prefix_store(gi_prefix *pc, const int32_t *tokens, int n, int seq_id)
{
    if (!pc || (n > 0 && !tokens))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_prefix_store: bad argument");
    if (n < 4) // prefix_cache.go:99-101
        return GI_OK;
    std::lock_guard<std::mutex> g(pc->mu);
    std::lock_guard<std::mutex> gm(pc->m->mu);
    auto st = pc->m->tables.find(seq_id);
    if (st == pc->m->tables.end())
        return gi::set_error(GI_ERR_UNKNOWN_SEQ, "sequence " + std::to_string(seq_id) + " not found");
    // The entry is keyed on all n tokens, so the sequence must hold them: a
    // shorter one would make a later hit report more cached tokens than the
    // fork has.  (cloneKVCachePrefix, prefix_cache.go:122-150, copies
    // prefixLen slots whatever the cache holds; refusing is the safe form.)
    if (n > st->second.num_tokens)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_prefix_store: " + std::to_string(n) + " tokens but sequence " +
                                                 std::to_string(seq_id) + " holds " +
                                                 std::to_string(st->second.num_tokens));
    // prefix_cache.go:106-112: a full cache drops one entry first
    if ((int)pc->entries.size() >= pc->max_size && !pc->order.empty()) {
        const std::string victim = pc->order.front();
        prefix_drop_locked(pc, victim);
    }
    const std::string key = prefix_key(tokens, n);
    prefix_drop_locked(pc, key); // entries[key] is replaced (prefix_cache.go:114-118)
    int pinned = 0;
    int rc = fork_locked(pc->m, seq_id, n, &pinned);
    if (rc)
        return rc;
    pc->entries[key] = pinned;
    pc->order.push_back(key);
    return GI_OK;
}

int gi_prefix_find_longest(gi_prefix *pc, const int32_t *tokens, int n, int *matched, int *new_seq)
{
    if (matched)
        *matched = 0;
    if (new_seq)
        *new_seq = 0;
    if (!pc || !matched || !new_seq || (n > 0 && !tokens))
        return gi::set_error(GI_ERR_BAD_ARG, "gi_prefix_find_longest: bad argument");
    std::lock_guard<std::mutex> g(pc->mu);
    std::lock_guard<std::mutex> gm(pc->m->mu);
    for (int l = n - 1; l >= 1; l--) { // prefix_cache.go:85-93
        auto it = pc->entries.find(prefix_key(tokens, l));
        if (it == pc->entries.end())
            continue;
        int rc = fork_locked(pc->m, it->second, l, new_seq);
        if (rc)
            return rc;
        *matched = l;
        return GI_OK;
    }
    return GI_OK;
}

int gi_prefix_size(gi_prefix *pc, int *n)
{
    if (!pc || !n)
        return gi::set_error(GI_ERR_BAD_ARG, "gi_prefix_size: NULL argument");
    std::lock_guard<std::mutex> g(pc->mu);
    *n = (int)pc->entries.size();
    return GI_OK;
}

} // extern "C"
