/*
 * goinfer_paged.h -- C ABI of the MI355X paged KV-cache library
 * (libgoinfer_paged.so).
 *
 * This is the device boundary that go-infer's Go engine binds through cgo, in
 * the same way c_bridge_cgo.go binds inference_core.h.  It replaces:
 *   - the block allocator pkg/engine/paged_kv.go:49-148 (PagedKVManager),
 *     kept host-side and mirrored here as gi_kvmgr_*;
 *   - the KV store of pkg/engine/kvcache.go:146-180 (KVCache.Write) and the
 *     inline stores of pkg/engine/forward.go:236-240 / 527-545, and the GPU
 *     seams metal.KVWrite / metal.KVWriteBatch (pkg/metal/metal_darwin.go:
 *     601-614, 984-999) -> gi_paged_append / gi_paged_append_at_len;
 *   - KVCache.Get / Clone / ForkAt (kvcache.go:183-284) -> gi_paged_gather;
 *   - the decode attention loop of forward.go:242-267 and metal.AttentionGQA
 *     (metal_darwin.go:711-727) -> gi_paged_decode_attention /
 *     gi_paged_decode_step;
 *   - the chunked-prefill attention of forward.go:547-577 and
 *     metal.AttentionGQABatch (metal_darwin.go:963-981) ->
 *     gi_paged_prefill_attention;
 *   - ApplyRoPE on q/k before the store (forward.go:228-240, 527-545,
 *     pkg/math/kernels.go:22-35) -> gi_paged_rope_append[_at_len] /
 *     gi_paged_rope_decode_step.
 *
 * Conventions (as in pkg/metal/metal_bridge.h and inference_core.h):
 *   - every call returns int: GI_OK (0) or a negative GI_ERR_* code, and a
 *     text reason is kept per thread for gi_last_error();
 *   - creation returns NULL-equivalent failure through the code, never
 *     aborts;
 *   - buffers passed to the compute entry points are DEVICE pointers (from
 *     gi_dev_alloc or any HIP allocation on the handle's device); work is
 *     queued on the handle's stream and gi_synchronize() waits for it and
 *     reports asynchronous errors (bad page ids seen by a kernel);
 *   - calls on one handle are serialised internally; distinct handles may be
 *     used from different threads;
 *   - no pointer passed in is retained after the call returns (cgo rules).
 */
#ifndef GOINFER_PAGED_H
#define GOINFER_PAGED_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes.  metal_bridge.h uses 0 / -1 unavailable / -2 buffer failure
 * (metal_bridge_darwin.m:3218, 3223); the same meanings are kept. */
#define GI_OK 0
#define GI_ERR_NO_DEVICE (-1)      /* no HIP device / not initialised      */
#define GI_ERR_OOM (-2)            /* device or host allocation failed     */
#define GI_ERR_BAD_ARG (-3)        /* invalid argument or unsupported shape */
#define GI_ERR_POOL_EXHAUSTED (-4) /* paged_kv.go:118-120 "out of paged KV memory" */
#define GI_ERR_HIP (-5)            /* HIP launch / runtime error            */
#define GI_ERR_UNKNOWN_SEQ (-6)    /* paged_kv.go:111-114 "sequence %d not found" */
#define GI_ERR_BAD_PAGE (-7)       /* a kernel saw a page id outside the pool */
#define GI_ERR_SHARED_PAGE (-8)    /* the append would write a page another sequence shares */

/* KV storage types.  f32, q8_0 and q4_0 are kvcache.go:11-15's KVTypeF32,
 * KVTypeQ8_0 and KVTypeQ4_0 (QuantizeQ8_0 / QuantizeQ4_0 of each token
 * vector, pkg/quant/quant.go:407-521); f16 stores FP32ToFP16
 * (pkg/quant/fp16.go:38-69) halves. */
#define GI_KV_F32 0
#define GI_KV_F16 1
#define GI_KV_Q8_0 2
#define GI_KV_Q4_0 3

/* ---- library / device ------------------------------------------------- */

/* Text of the last error raised on the calling thread ("" if none). */
const char *gi_last_error(void);

/* Number of visible HIP devices (0 when none); never fails. */
int gi_device_count(void);

/* Name of the current device, like model_device_name (inference_core.c:
 * 117-122).  Writes at most cap bytes including the terminator. */
int gi_device_name(char *buf, int cap);

/* ---- host block allocator: PagedKVManager (paged_kv.go:49-148) ---------- */

typedef struct gi_kvmgr gi_kvmgr;

/* NewPagedKVManager (paged_kv.go:62-87): block_size <= 0 -> 16,
 * total_blocks <= 0 -> 256; FreeBlocks = [0..total_blocks). */
int gi_kvmgr_create(int num_layers, int kv_dim, int total_blocks, int block_size,
                    gi_kvmgr **out);
void gi_kvmgr_destroy(gi_kvmgr *m);

/* AllocateSequence (paged_kv.go:90-104): ids count up from 1. */
int gi_kvmgr_allocate_sequence(gi_kvmgr *m, int *seq_id);

/* AppendToken (paged_kv.go:107-132): reserves the next token slot, popping a
 * block from the tail of the free list when the sequence needs one; returns
 * GI_ERR_UNKNOWN_SEQ or GI_ERR_POOL_EXHAUSTED like the reference's errors. */
int gi_kvmgr_append_token(gi_kvmgr *m, int seq_id, int32_t *block_id, int32_t *slot);

/* n calls of AppendToken in one go; writes n block ids and slots.  On an
 * error the tokens already reserved stay reserved and *done says how many. */
int gi_kvmgr_append_tokens(gi_kvmgr *m, int seq_id, int n, int32_t *block_ids, int32_t *slots,
                           int *done);

/* BlockSize of the manager (paged_kv.go:54, the value NewPagedKVManager
 * settled on); 0 for NULL. */
int gi_kvmgr_block_size(const gi_kvmgr *m);

/* FreeSequence (paged_kv.go:135-148): pushes the table's ids back onto the
 * free list in table order; unknown ids are ignored. */
int gi_kvmgr_free_sequence(gi_kvmgr *m, int seq_id);

/* Block table of a sequence: copies up to cap ids, sets *n_blocks and
 * *n_tokens (BlockTable.BlockIDs / NumTokens, paged_kv.go:41-46). */
int gi_kvmgr_block_table(gi_kvmgr *m, int seq_id, int32_t *ids, int cap, int *n_blocks,
                         int *n_tokens);

/* Free list (FreeBlocks, bottom to top): copies up to cap ids, sets *n. */
int gi_kvmgr_free_list(gi_kvmgr *m, int32_t *ids, int cap, int *n);

/* Replaces the free list (bottom to top); ids must be distinct, in range and
 * not held by a sequence.  Lets a caller start from a shuffled pool. */
int gi_kvmgr_set_free_list(gi_kvmgr *m, const int32_t *ids, int n);

/* ---- copy-on-write prefix sharing -------------------------------------- *
 * Replaces the deep copies of KVCache.Clone / ForkAt (kvcache.go:217-284)
 * and of PrefixCache's cloneKVCachePrefix (prefix_cache.go:122-150) with
 * shared pages.  Every block carries a reference count: a fork takes a
 * reference to the pages of its prefix, FreeSequence returns a block to the
 * free list only when its last reference goes, and an append that would
 * write a block with more than one reference first moves the appending
 * sequence to a fresh copy of it (the caller copies the page on the device
 * with gi_paged_copy_pages before writing). */

/* ForkAt(n_tokens) (kvcache.go:225-284): a new sequence (*new_seq) whose
 * first n_tokens tokens are src_seq's, sharing its pages.  n_tokens is
 * clamped to [0, src length] as ForkAt clamps maxSlot to [0, MaxSeq]. */
int gi_kvmgr_fork_sequence(gi_kvmgr *m, int src_seq, int n_tokens, int *new_seq);

/* AppendToken with copy-on-write: as gi_kvmgr_append_token, and *copy_from
 * is -1, or the shared block whose contents the caller must copy into
 * *block_id (all layers, gi_paged_copy_pages) before writing the token.
 * gi_kvmgr_append_token and gi_kvmgr_append_tokens return
 * GI_ERR_SHARED_PAGE, changing nothing, where this call would copy. */
int gi_kvmgr_append_token_cow(gi_kvmgr *m, int seq_id, int32_t *block_id, int32_t *slot,
                              int32_t *copy_from);

/* n tokens with copy-on-write; at most the first can need a copy, reported
 * as *copy_src -> *copy_dst (both -1 when none). */
int gi_kvmgr_append_tokens_cow(gi_kvmgr *m, int seq_id, int n, int32_t *block_ids,
                               int32_t *slots, int32_t *copy_src, int32_t *copy_dst, int *done);

/* One copy-on-write AppendToken for each of n distinct sequences, the
 * decode step of a running batch (Forward appends one token per sequence,
 * forward.go:236-240).  All or nothing: if the free list cannot cover the
 * blocks the step takes (a new block for each sequence at a block boundary,
 * a fresh copy for each whose last block is shared), nothing changes and
 * GI_ERR_POOL_EXHAUSTED is returned; an unknown or repeated id changes
 * nothing either.  block_ids[i] / slots[i] are AppendToken's results for
 * seq_ids[i]; copy_src[i] is -1, or the shared block the caller copies into
 * block_ids[i] before writing. */
int gi_kvmgr_append_batch(gi_kvmgr *m, int n, const int *seq_ids, int32_t *block_ids, int32_t *slots,
                          int32_t *copy_src);

/* References held on a block (0 when it is free). */
int gi_kvmgr_block_refs(gi_kvmgr *m, int32_t block_id, int *refs);

/* PrefixCache (prefix_cache.go:7-150) over shared pages.  max_size <= 0 ->
 * 32 entries.  The cache holds a forked sequence per entry (its pages stay
 * referenced until the entry is evicted or the cache destroyed). */
typedef struct gi_prefix gi_prefix;
int gi_prefix_create(gi_kvmgr *m, int max_size, gi_prefix **out);
void gi_prefix_destroy(gi_prefix *pc);

/* Store (prefix_cache.go:97-119): keeps tokens[0..n) of seq_id under the
 * key tokens; no-op for n < 4.  A full cache first evicts one entry (the
 * oldest; the reference drops whichever its map iteration yields). */
int gi_prefix_store(gi_prefix *pc, const int32_t *tokens, int n, int seq_id);

/* FindLongestPrefix (prefix_cache.go:76-95): the longest l in [1, n-1]
 * with an entry keyed tokens[0..l); *matched = l and *new_seq = a new
 * sequence forked from that entry (sharing its pages), or 0 and 0. */
int gi_prefix_find_longest(gi_prefix *pc, const int32_t *tokens, int n, int *matched,
                           int *new_seq);

/* Number of entries. */
int gi_prefix_size(gi_prefix *pc, int *n);

/* ---- device page pool -------------------------------------------------- */

typedef struct gi_paged gi_paged;

/* Creates a pool of num_pages pages on the current device, each page holding
 * page_tokens tokens of every layer (KVBlock, paged_kv.go:13-38), plus one
 * HIP stream (default priority).  kv_type is GI_KV_*.  head_dim must be a
 * multiple of 8 (32 for q8_0 and q4_0).  Pages are zero filled. */
int gi_paged_create(int num_layers, int num_kv_heads, int head_dim, int page_tokens,
                    int64_t num_pages, int kv_type, gi_paged **out);
void gi_paged_destroy(gi_paged *h);

/* Bytes of one page of one layer, and of the whole pool. */
int gi_paged_page_bytes(const gi_paged *h, int64_t *page_bytes, int64_t *pool_bytes);

/* Queue all further work of this handle on the given HIP stream
 * (hipStream_t as void*; NULL is HIP's default stream, which orders with
 * the work of other blocking streams).  A handle starts on a stream of its
 * own; gi_paged_stream returns the current one, so a caller can save it and
 * switch back.  Work queued before the switch completes first. */
int gi_paged_set_stream(gi_paged *h, void *stream);
void *gi_paged_stream(gi_paged *h);

/* Waits for queued work; returns GI_ERR_BAD_PAGE if a kernel saw a page id
 * or slot outside the pool since the last call (and clears the flag). */
int gi_synchronize(gi_paged *h);

/* Device memory helpers for callers without their own allocator. */
int gi_dev_alloc(gi_paged *h, size_t bytes, void **dptr);
int gi_dev_free(gi_paged *h, void *dptr);
int gi_memcpy_h2d(gi_paged *h, void *dst, const void *src, size_t bytes);
int gi_memcpy_d2h(gi_paged *h, void *dst, const void *src, size_t bytes);

/* ---- hot path (device pointers, queued on the handle's stream) --------- */

/* Appends n_tok token vectors of one layer: token i goes to page
 * block_ids[i], slot slots[i] (the pair AppendToken returned).  k and v are
 * [n_tok][num_kv_heads*head_dim] float32; f16 pages store the truncated
 * halves, q8_0 / q4_0 pages the QuantizeQ8_0 / QuantizeQ4_0 blocks of each
 * whole vector.
 * Replaces KVCache.Write (kvcache.go:146-180) and metal.KVWrite[Batch]. */
int gi_paged_append(gi_paged *h, int layer, int n_tok, const int32_t *block_ids,
                    const int32_t *slots, const float *k, const float *v);

/* Decode-step append: token b goes to position seq_lens[b]-1 of sequence b
 * through block_tables ([batch][max_blocks] int32). */
int gi_paged_append_at_len(gi_paged *h, int layer, int batch, const int32_t *block_tables,
                           int max_blocks, const int32_t *seq_lens, const float *k,
                           const float *v);

/* Copies whole pages, every layer: page dst_ids[i] becomes a copy of page
 * src_ids[i] (device int32 arrays of n ids; the copy-on-write step of a
 * forked sequence, see gi_kvmgr_append_token_cow). */
int gi_paged_copy_pages(gi_paged *h, int n, const int32_t *src_ids, const int32_t *dst_ids);

/* Gathers tokens [0, n_tok) of one layer of one sequence into the contiguous
 * [n_tok][kv_dim] layout that KVCache indexes (kvcache.go:183-284).
 * widen == 0: stored bytes (f32 4*kv_dim, f16 2*kv_dim, q8_0 kv_dim/32
 * blocks of 34 bytes: little-endian fp16 scale then 32 int8, quant.go:38-41;
 * q4_0 kv_dim/32 blocks of 18 bytes: the scale, then byte j = element j |
 * element j+16 << 4, quant.go:9-13, 504);
 * widen == 1: float32 values (FP16ToFP32 / DequantizeQ8_0 / DequantizeQ4_0).  block_table
 * must hold ceil(n_tok / page_tokens) ids. */
int gi_paged_gather(gi_paged *h, int layer, const int32_t *block_table, int n_tok, void *k_out,
                    void *v_out, int widen);

/* Decode attention (forward.go:242-267) of one layer for a batch read
 * directly from pages: q, out [batch][num_heads][head_dim] float32; sequence
 * b attends its first seq_lens[b] tokens.  q-head h reads kv head h /
 * (num_heads / num_kv_heads) (forward.go:249).
 *
 * Long sequences are cut into splits of equal token ranges, attended by
 * separate workgroups and merged by a second launch.  max_seq_len (>= 0; 0
 * means unknown: the longest sequence max_blocks maps) sizes that split
 * plan only: the last split of every sequence runs to its end, so every
 * seq_lens[b] token is attended whatever max_seq_len says (a short hint
 * costs balance, never tokens).  A length below zero or beyond max_blocks *
 * page_tokens is clamped and reported by gi_synchronize as GI_ERR_BAD_PAGE.
 *
 * Workspace: the handle keeps the partials of split sequences, batch *
 * num_kv_heads * splits slots of (num_heads / num_kv_heads) * (head_dim + 2)
 * floats, where splits falls as batch * num_kv_heads grows (about one
 * workgroup per CU).  A call that needs it to grow while the handle's stream
 * is capturing a graph fails with GI_ERR_BAD_ARG (make one eager call with
 * the same shape first); once any call has been captured, growth keeps the
 * old buffers alive until gi_paged_destroy, so captured graphs stay valid. */
int gi_paged_decode_attention(gi_paged *h, int layer, int batch, int num_heads, const float *q,
                              float *out, const int32_t *block_tables, int max_blocks,
                              const int32_t *seq_lens, int max_seq_len, float scale);

/* gi_paged_decode_attention that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, hosts that forbid it).  The
 * split partials live in a fixed 4 MiB scratch array that the library holds
 * on each device it runs on until the process ends, instead of the handle's
 * growable workspace.  On a 256-CU device every shape with up to 8 query
 * heads per kv head fits (fewer than 512 partial slots of 4 KiB); with 16
 * per kv head at head_dim 128 the batches with batch * num_kv_heads of 253
 * to 255 and contexts over 1024 tokens (two splits, 506 to 510 slots of
 * 8 KiB) would need up to 4.25 MB and fail with GI_ERR_BAD_ARG before any
 * launch.  Every call on one device shares that array.  The library orders
 * its eager users on the device: a call whose handle's stream differs from
 * the previous user's first makes its stream wait for an event recorded
 * after that user's launches (the event is created once per device, at the
 * first gi_paged_create there).  A stream that is capturing a graph neither
 * waits nor records, so replays of captured calls that could overlap other
 * users of the array on the device (other streams) race: serialise them.
 * Same arguments and results as gi_paged_decode_attention. */
int gi_paged_decode_attention_noalloc(gi_paged *h, int layer, int batch, int num_heads, const float *q,
                                      float *out, const int32_t *block_tables, int max_blocks,
                                      const int32_t *seq_lens, int max_seq_len, float scale);

/* One decode step of one layer: gi_paged_append_at_len of k/v, then
 * gi_paged_decode_attention over seq_lens[b] tokens (the new token
 * included), as Forward stores then attends (forward.go:236-267).  Where the
 * decode grid is one round of workgroups (small batches), the matrix-core
 * kernels store the token themselves in the same launch; the stored bytes
 * and the outputs are those of the two calls. */
int gi_paged_decode_step(gi_paged *h, int layer, int batch, int num_heads, const float *q,
                         const float *k, const float *v, float *out, const int32_t *block_tables,
                         int max_blocks, const int32_t *seq_lens, int max_seq_len, float scale);

/* ---- rotary embedding fused with the append ---------------------------- *
 * Forward turns q and k with ApplyRoPE (pkg/math/kernels.go:22-35) on every
 * head right before it stores k/v (forward.go:228-240 decode, 527-545
 * prefill; with a rope dimension below head_dim only the first rope_dim dims
 * of each head turn, forward.go:945-977).  These entry points do both in one
 * pass, so the rotated K is never written back to the caller and read again.
 * The rotation is bit-exact with ApplyRoPE: cos/sin come from a table built
 * as ApplyRoPE computes them (float64, rounded to float32) and each pair is
 * rotated with rounded products (no fused multiply-add). */

/* Builds the pool's RoPE table for positions [0, max_positions): theta is
 * llama.rope.freq_base (Config.RopeTheta, pkg/engine/config.go:13), rope_dim
 * (even, <= head_dim; <= 0 means head_dim) is rope.dimension_count
 * (engine.go:112-113).  Replaces any earlier table. */
int gi_paged_set_rope(gi_paged *h, float theta, int rope_dim, int max_positions);

/* RoPE + append, explicit form (the prefill store, forward.go:527-545):
 * token i is at position positions[i] and goes to (block_ids[i], slots[i]).
 * q [n_tok][num_heads][head_dim] float32 is rotated into q_out (which may be
 * q; num_heads 0 with q == q_out == NULL turns only k); k is rotated, then
 * k and v are stored as gi_paged_append stores them.  A position outside the
 * table skips the token (q_out row untouched) and is reported by
 * gi_synchronize as GI_ERR_BAD_PAGE. */
int gi_paged_rope_append(gi_paged *h, int layer, int n_tok, int num_heads, const int32_t *positions,
                         const int32_t *block_ids, const int32_t *slots, const float *q, float *q_out,
                         const float *k, const float *v);

/* RoPE + append, decode form: token b is at position seq_lens[b]-1 of
 * sequence b, stored through block_tables (as gi_paged_append_at_len). */
int gi_paged_rope_append_at_len(gi_paged *h, int layer, int batch, int num_heads,
                                const int32_t *block_tables, int max_blocks, const int32_t *seq_lens,
                                const float *q, float *q_out, const float *k, const float *v);

/* One decode step of one layer from the projections: q (rotated in place,
 * as ApplyRoPE turns a.Q) and k are turned at position seq_lens[b]-1, k/v
 * appended, then gi_paged_decode_attention over seq_lens[b] tokens
 * (forward.go:228-267). */
int gi_paged_rope_decode_step(gi_paged *h, int layer, int batch, int num_heads, float *q, const float *k,
                              const float *v, float *out, const int32_t *block_tables, int max_blocks,
                              const int32_t *seq_lens, int max_seq_len, float scale);

/* Chunked-prefill causal attention (forward.go:547-577) of one layer: the
 * chunk's K/V are already appended; query i of sequence b attends tokens
 * [0, start_pos[b] + i + 1).  q, out [batch][chunk_len][num_heads][head_dim]
 * float32. */
int gi_paged_prefill_attention(gi_paged *h, int layer, int batch, int chunk_len, int num_heads,
                               const float *q, float *out, const int32_t *block_tables,
                               int max_blocks, const int32_t *start_pos, float scale);

/* Which decode kernel serves this pool and head count: 0 vector ALU,
 * 1 matrix core (fp16 pages, head_dim 64/128, page_tokens % 16 == 0). */
int gi_paged_decode_kernel(const gi_paged *h, int num_heads);

/* The launch plan of this pool's attention calls for a batch, head count
 * and longest context (max_seq_len, as the decode calls take it; 0 counts as
 * 1), worked out without launching anything.  No counterpart in the
 * reference (its attention is inline CPU loops); a host checks here whether
 * its shapes run on the matrix-core kernels, since a shape they do not take
 * (head_dim other than 64/128, pages not a multiple of 16 tokens, f32 or
 * quantised pages with 16 query heads per kv head) is served by the
 * vector-ALU kernels, correct but several times slower (*_fallback). */
typedef struct gi_attention_plan {
    int decode_kernel;       /* 0 vector ALU, 1 matrix core */
    int decode_fallback;     /* 1: matrix core selected but the shape is not
                                supported, so the vector ALU serves it */
    int decode_splits;       /* split-K ranges per (sequence, kv head) */
    int decode_split_tokens; /* tokens per split (the last runs to the end) */
    int decode_waves;        /* waves per matrix-core workgroup (4 or 8) */
    int decode_step_fused;   /* gi_paged_decode_step stores the token inside
                                the decode launch (else an append launch) */
    int prefill_kernel;      /* 0 vector ALU, 1 matrix core */
    int prefill_fallback;    /* as decode_fallback, for prefill */
} gi_attention_plan;

int gi_paged_attention_plan(const gi_paged *h, int batch, int num_heads, int max_seq_len,
                            gi_attention_plan *plan);

/* Selects the attention kernels (decode and prefill): -1 automatic
 * (default), 0 vector ALU, 1 matrix core where supported.  For
 * comparisons; results agree within the attention tolerance. */
int gi_paged_set_decode_kernel(gi_paged *h, int kind);

/* ---- weight matrix times activations: the O-projection ------------------ *
 * After attention, Forward projects AttnOut through blk.%d.attn_output.weight
 * (pkg/engine/forward.go:270, 580: Weights.MatMul / MatMulBatch,
 * pkg/engine/weights.go:237-350), y = W x with W [rows][cols] in GGUF layout.
 * The GPU seam it replaces is metal.MatMulBatch(y, x, rawW, qType,
 * batchSize, rows, cols) (pkg/metal/metal_darwin.go:849-880).  Weights are
 * uploaded once into an operand layout (gi_weights), as the reference keeps
 * GPU buffers per tensor (Weights.GPUBufs, metal.MatMulBatchBuf). */

/* GGML type ids (pkg/gguf/types.go:25-31) with a device kernel. */
#define GI_GGML_F32 0
#define GI_GGML_F16 1
#define GI_GGML_Q4_0 2
#define GI_GGML_Q8_0 8

typedef struct gi_weights gi_weights;

/* Uploads a [rows][cols] weight matrix given as its GGUF bytes (host memory:
 * F32 / F16 rows, or rows of cols/32 Q4_0 / Q8_0 blocks) to the pool's
 * device.  cols must be a multiple of 32.  Other types: GI_ERR_BAD_ARG.
 * gi_matmul_batch needs the pool alive; gi_weights_destroy does not (it
 * waits for the device and frees the buffers itself). */
int gi_weights_upload(gi_paged *h, int ggml_type, int rows, int cols, const void *raw, gi_weights **out);
void gi_weights_destroy(gi_weights *w);

/* y[b][r] = sum_c W[r][c] x[b][c] for b < batch (DotVecF32 / DotVecF16 /
 * DotVecQ4_0 / DotVecQ8_0 of each row, pkg/math/gemv.go), on the pool's
 * stream; x [batch][cols], y [batch][rows] float32 device buffers.  Results
 * agree with the reference's float32 loops up to summation order.  Grows a
 * workspace held by w on first use at a batch size: the activations' hi/lo
 * halves and, for F16 / F32 weights at batches of 128 and more, the partial
 * products of the column slices (4 * slices * batch * rows bytes, rounded up;
 * 16 MiB at 256 x 4096 x 4096).  Growth fails with GI_ERR_BAD_ARG while the
 * stream captures a graph. */
int gi_matmul_batch(gi_weights *w, int batch, const float *x, float *y);

/* ---- continuous-batching decode driver ---------------------------------- *
 * The reference decodes one sequence at a time under Engine.mu
 * (pkg/engine/engine.go:417), each token a full Forward of that sequence.  A
 * gi_batch steps a running set of sequences together over one manager and
 * one pool:
 *   - gi_batch_step reserves one token for every running sequence
 *     (gi_kvmgr_append_batch, all or nothing) and updates the device-resident
 *     block tables and lengths in place (only changed entries are uploaded),
 *     queueing the page copies of copy-on-write appends;
 *   - gi_batch_decode_layer then runs the RoPE + append + paged attention of
 *     one layer (forward.go:228-267) for the whole set.
 * Rows are dense: row i of the q/k/v/out buffers is the i-th running
 * sequence (gi_batch_rows); removing a sequence moves the last row into its
 * place.  With h == NULL the driver keeps host bookkeeping only (for hosts
 * that drive their own kernels, and for tests). */
typedef struct gi_batch gi_batch;

/* max_batch running sequences of up to max_blocks blocks each.  Steps need
 * the manager and pool alive; gi_batch_destroy needs neither. */
int gi_batch_create(gi_kvmgr *m, gi_paged *h, int max_batch, int max_blocks, gi_batch **out);
void gi_batch_destroy(gi_batch *b);

/* Adds an allocated sequence (its tokens so far already in the pool) as the
 * last row; *row receives its row. */
int gi_batch_add(gi_batch *b, int seq_id, int *row);

/* Removes a running sequence (it stays allocated; FreeSequence is the
 * caller's).  GI_ERR_UNKNOWN_SEQ if it is not running. */
int gi_batch_remove(gi_batch *b, int seq_id);

/* One token for every running sequence; *n_rows = the running count.  After
 * it, row i's length (gi_batch_rows) includes the new token, which
 * gi_batch_decode_layer appends at position length-1.  On
 * GI_ERR_POOL_EXHAUSTED nothing changed: remove (preempt) a sequence and
 * step again. */
int gi_batch_step(gi_batch *b, int *n_rows);

/* Host view: running sequence ids and lengths by row (up to cap rows). */
int gi_batch_rows(gi_batch *b, int32_t *seq_ids, int32_t *seq_lens, int cap, int *n);

/* Host mirror of one row's block table. */
int gi_batch_row_table(gi_batch *b, int row, int32_t *ids, int cap, int *n_blocks);

/* The device table ([max_batch][max_blocks] int32) and lengths, for callers
 * that launch the attention entry points themselves. */
int gi_batch_device_tables(gi_batch *b, int32_t **block_tables, int32_t **seq_lens, int *max_blocks);

/* One layer of the step for every running row: q [n][num_heads][head_dim]
 * (rotated in place when rope != 0, which needs gi_paged_set_rope), k, v
 * [n][kv_dim], out [n][num_heads][head_dim]; gi_paged_rope_decode_step or
 * gi_paged_decode_step over the driver's tables. */
int gi_batch_decode_layer(gi_batch *b, int layer, int num_heads, float *q, const float *k, const float *v,
                          float *out, float scale, int rope);

#ifdef __cplusplus
}
#endif

#endif /* GOINFER_PAGED_H */
