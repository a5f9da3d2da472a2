// Launchers of the paged KV-cache kernels (internal to the library; the
// public C ABI is include/goinfer_paged.h).
#pragma once

#include "gi_common.h"

namespace gi {

hipError_t launch_append(const PoolLayout &L, uint8_t *base, int n_tok, const int32_t *block_ids,
                         const int32_t *slots, const float *k, const float *v, int *status,
                         hipStream_t st);

hipError_t launch_append_at_len(const PoolLayout &L, uint8_t *base, int batch,
                                const int32_t *block_tables, int max_blocks,
                                const int32_t *seq_lens, const float *k, const float *v,
                                int *status, hipStream_t st);

// Fused rotary embedding + append (pkg/math/kernels.go:22-35 ApplyRoPE on
// every q and k head, then the store of forward.go:236-240 / 527-545).
// table holds (cos, sin) of pair j at position p at table[p * rope_half + j]
// for p < max_pos.  Token i's position is positions[i] (explicit form, with
// block_ids/slots) or seq_lens[i] - 1 (decode form, with block_tables).
// q [n_tok][num_heads][head_dim] is rotated into q_out (q_out may be q);
// num_heads may be 0 (no q).  K is rotated and stored, V stored as is.
struct RopeArgs {
    const float2 *table;
    int rope_half; // rope_dim / 2
    int max_pos;
    int num_heads;
    const int32_t *positions; // explicit form only
    const float *q;
    float *q_out;
};

hipError_t launch_rope_append(const PoolLayout &L, uint8_t *base, int n_tok, const int32_t *block_ids,
                              const int32_t *slots, const int32_t *block_tables, int max_blocks,
                              const int32_t *seq_lens, const RopeArgs &R, const float *k,
                              const float *v, int *status, hipStream_t st);

hipError_t launch_gather(const PoolLayout &L, const uint8_t *base, const int32_t *table, int n_tok,
                         void *k_out, void *v_out, int widen, int *status, hipStream_t st);

// Whole-page copies in every layer: page dst[i] <- page src[i].
hipError_t launch_copy_pages(const PoolLayout &L, uint8_t *const *layer_base, int n, const int32_t *src,
                             const int32_t *dst, int *status, hipStream_t st);

// Attention over paged context.  Decode: q/out are [batch][num_heads][head_dim]
// float32, block_tables is [batch][max_blocks], sequence b attends its first
// seq_lens[b] tokens.  The same kernels serve chunked prefill on the vector
// path: n_q queries per sequence, query i of sequence b attends
// start_pos[b] + i + 1 tokens, q/out are [batch][n_q][num_heads][head_dim].
struct DecodeArgs {
    PoolLayout L;
    const uint8_t *base;
    const float *q;
    float *out;
    const int32_t *block_tables;
    int max_blocks;
    const int32_t *seq_lens;
    int batch;
    int n_q;                  // queries per sequence (1 for decode)
    const int32_t *start_pos; // prefill only: tokens cached before the chunk
    int num_heads;
    float scale;
    int split_tokens; // tokens per split, a multiple of the page size
    int num_splits;
    float *ws; // partials when num_splits > 1
    int *status;
    int kernel; // -1 automatic, 0 vector ALU, 1 matrix core
    int waves;  // matrix-core decode: waves per workgroup, 4 or 8 (decode_waves)
    // Decode step: the new token's K and V ([batch][kv_dim] float32) to store
    // at position seq_lens[b] - 1 before attending, as gi_paged_append_at_len
    // does; null for attention alone.  append_base is base, writable.
    const float *new_k, *new_v;
    uint8_t *append_base;
};

// Bytes of split-K workspace needed for a decode launch.
size_t decode_workspace_bytes(const PoolLayout &L, int batch, int num_heads, int num_splits);

// Whether a decode step's token store goes into the matrix-core decode
// launch (DecodeArgs.new_k) for this grid, rather than an append launch.
bool decode_fuses_append(const PoolLayout &L, int batch, int num_splits, int num_cus);

// Picks (split_tokens, num_splits) for a batch whose longest sequence has
// max_len tokens, so the grid fills the device.
void decode_plan(const PoolLayout &L, int batch, int num_heads, int max_len, int num_cus,
                 int *split_tokens, int *num_splits);

// Waves per workgroup of the matrix-core decode launch: 8 when the grid of
// (split, kv head, sequence) workgroups fits the CUs once, so that every
// SIMD still streams with two waves; 4 otherwise.
int decode_waves(const PoolLayout &L, int batch, int num_splits, int num_cus);

// Returns hipErrorInvalidValue for shapes without a kernel instance.
hipError_t launch_decode(const DecodeArgs &a, hipStream_t st);

// Which kernel launch_decode uses for a layout/head count and a requested
// kind (-1 automatic): 0 vector ALU, 1 matrix core.
int decode_kernel_kind(const PoolLayout &L, int num_heads, int requested);

bool mfma_decode_supported(const PoolLayout &L, int num_heads);
hipError_t launch_decode_mfma(const DecodeArgs &a, hipStream_t st);

// Chunked-prefill causal attention over paged context: query i of sequence b
// (i < chunk_len) attends tokens [0, start_pos[b] + i + 1).
struct PrefillArgs {
    PoolLayout L;
    const uint8_t *base;
    const float *q; // [batch][chunk_len][num_heads][head_dim]
    float *out;
    const int32_t *block_tables;
    int max_blocks;
    const int32_t *start_pos;
    int batch;
    int chunk_len;
    int num_heads;
    float scale;
    int *status;
    int kernel; // -1 automatic, 0 vector ALU, 1 matrix core
};

hipError_t launch_prefill(const PrefillArgs &a, hipStream_t st);

bool mfma_prefill_supported(const PoolLayout &L, int num_heads);
hipError_t launch_prefill_mfma(const PrefillArgs &a, hipStream_t st);

} // namespace gi
