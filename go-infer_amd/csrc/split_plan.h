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
// the last of its n_b workgroups to finish merges them into out (so no
// second launch is needed) and re-arms the sequence's arrival counter.
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

// Workgroup-wide (NT threads, every thread calls it): the plan entry of work
// item `item`; false for items past the end of the list.  Lengths below zero
// or beyond what the block table maps are clamped and raise FLAG_BAD_SLOT.
template <int NT>
__device__ bool plan_item(const DecodeArgs &a, int item, PlanItem &it)
{
    constexpr int NW = NT / 64;
    __shared__ int64_t s_tot[NW];
    __shared__ int s_cnt[NW];
    __shared__ int s_hit[4];
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
    if (tid == 0)
        s_hit[0] = -1;
    if (bad && blockIdx.x == 0 && blockIdx.y == 0 && a.status)
        atomicOr(a.status, FLAG_BAD_SLOT);
    __syncthreads();
    int64_t total = 0;
#pragma unroll
    for (int i = 0; i < NW; i++)
        total += s_tot[i];
    int64_t per = (total + a.plan_target - 1) / a.plan_target;
    per = (per + a.plan_unit - 1) / a.plan_unit * a.plan_unit;
    const int chunk = (int)(per > a.plan_min ? (per < (1 << 30) ? per : (1 << 30)) : a.plan_min);

    int carry = 0;
    for (int base = 0; base < a.batch; base += NT) {
        const int b = base + tid;
        bool unused = false;
        const int len = b < a.batch ? plan_len(a, b, cap, unused) : 0;
        const int n = b < a.batch ? max(1, (len + chunk - 1) / chunk) : 0;
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

// Partial slot of work item `item` for kv head kvh (G * (HD + 2) floats).
__device__ __forceinline__ float *plan_slot(const DecodeArgs &a, int item, int kvh, int G, int HD)
{
    return a.ws + ((int64_t)item * a.L.num_kv_heads + kvh) * ((int64_t)G * (HD + 2));
}

// Workgroup-wide, after this workgroup has written its partial to its slot:
// the last of the sequence's items to arrive merges every slot,
//   out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M),  M = max_s m_s,
// into out rows (b, kvh*G + g).
template <int NT>
__device__ void merge_if_last(const DecodeArgs &a, const PlanItem &it, int item, int kvh, int G, int HD)
{
    __shared__ int s_last;
    // this workgroup's partial is visible device-wide before it is counted
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0) {
        int *cnt = a.plan_cnt + (int64_t)it.b * a.L.num_kv_heads + kvh;
        const int last = atomicAdd(cnt, 1) == it.nsplit - 1;
        if (last)
            atomicExch(cnt, 0); // every item has arrived: ready for the next launch
        s_last = last;
    }
    __syncthreads();
    if (!s_last)
        return;
    // the other items' partials are read after their counts were seen
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const int KVH = a.L.num_kv_heads;
    const int64_t stride = (int64_t)G * (HD + 2), step = (int64_t)KVH * stride;
    const float *w0 = plan_slot(a, item - it.split, kvh, G, HD);
    for (int e = threadIdx.x; e < G * HD; e += NT) {
        const int g = e / HD, d = e - g * HD;
        float M = -INFINITY;
        for (int s = 0; s < it.nsplit; s++)
            M = fmaxf(M, w0[s * step + G * HD + 2 * g]);
        float num = 0.0f, den = 0.0f;
        if (M != -INFINITY) {
            for (int s = 0; s < it.nsplit; s++) {
                const float *w = w0 + s * step;
                const float m = w[G * HD + 2 * g];
                if (m == -INFINITY)
                    continue;
                const float f = expf(m - M);
                num = fmaf(w[g * HD + d], f, num);
                den = fmaf(w[G * HD + 2 * g + 1], f, den);
            }
        }
        a.out[((int64_t)it.b * a.num_heads + kvh * G + g) * HD + d] = den > 0.0f ? num / den : 0.0f;
    }
}

} // namespace gi
