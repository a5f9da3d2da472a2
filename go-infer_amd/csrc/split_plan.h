// Decode split plan and the split-K merge, shared by the decode kernels.
//
// A decode launch over a batch of sequences (pkg/engine/forward.go:242-267
// for each of them) is cut into work items of consecutive tokens of one
// sequence; the grid is (items, kv heads).  Every workgroup derives the plan
// from the lengths in device memory:
//
//   total = sum_b min(len_b, max_blocks * page_tokens)
//   chunk = max(plan_min, ceil(total / plan_target) rounded up to plan_unit)
//   sequence b takes n_b = max(1, ceil(len_b / chunk)) items, in batch order
//
// so the items are about equally long however ragged the lengths are, a
// captured graph sees the lengths of each replay, and no token is left out
// whatever length the host expected.  sum_b n_b <= batch + plan_target, which
// bounds the grid.
//
// A sequence with n_b > 1 leaves one partial per item (G rows of HD
// unnormalised accumulators, then (m, l) per row, m in natural-log units);
// merge_splits, launched next on the same stream, combines them.  (Merging
// in the decode launch by its last-arriving workgroup needs a device-scope
// release by every split workgroup, which writes back its XCD's L2: that
// measured 2.4x slower on ragged batches.)
#pragma once

#include "gi_kernels.h"

namespace gi {

// Workgroups per CU the plan aims at, and the shortest split in tokens.
constexpr int kDecodeWgPerCu = 2;
constexpr int kDecodeMinSplit = 1024;

struct PlanItem {
    int b;      // sequence
    int split;  // index of this item within the sequence
    int nsplit; // items of the sequence
    int len;    // tokens the sequence attends (clamped to its block table)
    int t0, t1; // token range of this item
};

__device__ __forceinline__ int plan_len(const DecodeArgs &a, int b, int64_t cap, bool &bad)
{
    int len = a.seq_lens[b];
    if (len < 0 || (int64_t)len > cap) {
        bad = true;
        len = len < 0 ? 0 : (int)cap;
    }
    return len;
}

// Workgroup-wide (NT threads, every thread calls it): the plan's chunk
// length.  Lengths below zero or beyond what the block table maps are clamped
// (and raise FLAG_BAD_SLOT when `flag` is set).
template <int NT>
__device__ int plan_chunk(const DecodeArgs &a, bool flag)
{
    constexpr int NW = NT / 64;
    __shared__ int64_t s_tot[NW];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t cap = (int64_t)a.max_blocks * a.L.page_tokens;
    bool bad = false;
    int64_t sum = 0;
    for (int b = tid; b < a.batch; b += NT)
        sum += plan_len(a, b, cap, bad);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        sum += __shfl_xor(sum, o);
    if (lane == 0)
        s_tot[w] = sum;
    if (bad && flag && a.status)
        atomicOr(a.status, FLAG_BAD_SLOT);
    __syncthreads();
    int64_t total = 0;
#pragma unroll
    for (int i = 0; i < NW; i++)
        total += s_tot[i];
    int64_t per = (total + a.plan_target - 1) / a.plan_target;
    per = (per + a.plan_unit - 1) / a.plan_unit * a.plan_unit;
    return (int)(per > a.plan_min ? (per < (1 << 30) ? per : (1 << 30)) : a.plan_min);
}

__device__ __forceinline__ int plan_items(int len, int chunk) { return max(1, (len + chunk - 1) / chunk); }

// Workgroup-wide: the plan entry of work item `item`; false for items past
// the end of the list.
template <int NT>
__device__ bool plan_item(const DecodeArgs &a, int item, PlanItem &it)
{
    constexpr int NW = NT / 64;
    __shared__ int s_cnt[NW];
    __shared__ int s_hit[4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t cap = (int64_t)a.max_blocks * a.L.page_tokens;
    if (tid == 0)
        s_hit[0] = -1;
    // (the barrier inside plan_chunk orders that store before the scan)
    const int chunk = plan_chunk<NT>(a, blockIdx.x == 0 && blockIdx.y == 0);
    int carry = 0;
    for (int base = 0; base < a.batch; base += NT) {
        const int b = base + tid;
        bool unused = false;
        const int len = b < a.batch ? plan_len(a, b, cap, unused) : 0;
        const int n = b < a.batch ? plan_items(len, chunk) : 0;
        int x = n; // inclusive scan over the wave
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o);
            if (lane >= o)
                x += y;
        }
        if (lane == 63)
            s_cnt[w] = x;
        __syncthreads();
        int before = carry, all = 0;
#pragma unroll
        for (int i = 0; i < NW; i++) {
            before += i < w ? s_cnt[i] : 0;
            all += s_cnt[i];
        }
        const int first = before + x - n;
        if (n > 0 && item >= first && item < first + n) {
            s_hit[0] = b;
            s_hit[1] = item - first;
            s_hit[2] = n;
            s_hit[3] = len;
        }
        carry += all;
        // the hit is visible, and s_cnt is free for the next round
        __syncthreads();
        if (s_hit[0] >= 0 || carry > item)
            break;
    }
    if (s_hit[0] < 0)
        return false;
    it.b = s_hit[0];
    it.split = s_hit[1];
    it.nsplit = s_hit[2];
    it.len = s_hit[3];
    it.t0 = it.split * chunk;
    it.t1 = min(it.len, it.t0 + chunk);
    return true;
}

// Workgroup-wide: the first item of sequence b and its item count.
template <int NT>
__device__ void plan_seq(const DecodeArgs &a, int b, int &first, int &n)
{
    constexpr int NW = NT / 64;
    __shared__ int s_first[NW];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t cap = (int64_t)a.max_blocks * a.L.page_tokens;
    const int chunk = plan_chunk<NT>(a, false);
    bool unused = false;
    int sum = 0;
    for (int c = tid; c < b; c += NT)
        sum += plan_items(plan_len(a, c, cap, unused), chunk);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        sum += __shfl_xor(sum, o);
    if (lane == 0)
        s_first[w] = sum;
    __syncthreads();
    first = 0;
#pragma unroll
    for (int i = 0; i < NW; i++)
        first += s_first[i];
    n = plan_items(plan_len(a, b, cap, unused), chunk);
}

// Partial slot of work item `item` for kv head kvh (G * (HD + 2) floats).
__device__ __forceinline__ float *plan_slot(const DecodeArgs &a, int item, int kvh, int G, int HD)
{
    return a.ws + ((int64_t)item * a.L.num_kv_heads + kvh) * ((int64_t)G * (HD + 2));
}

} // namespace gi
