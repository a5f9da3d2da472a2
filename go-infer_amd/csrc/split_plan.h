// Decode work plan and the split-K merge, shared by the decode kernels.
//
// A decode launch over a batch of sequences (pkg/engine/forward.go:242-267
// for each of them) works on the context of each kv head as one stream of
// 32-token blocks: sequence b holds blocks [S_b, S_b + n_b) of the stream,
// n_b = ceil(len_b / 32), S_b = sum of n over the sequences before it.  The
// stream is cut into equal ranges of cb blocks, one per work unit (a
// workgroup; its four waves take every fourth block of a segment):
//
//   cb = max(kMinUnitBlocks, ceil(total blocks / units))
//
// so every unit streams the same bytes however ragged the lengths are.  A
// unit walks the sequences its range touches.  A sequence that lies inside
// one range is finished there and written to out; a longer one leaves a
// partial (G rows of HD unnormalised accumulators, then (m, l) per row, m in
// natural-log units) in each unit it touches, and merge_splits, launched next
// on the same stream, combines them.  Every workgroup derives the plan from
// the lengths in device memory, so a captured graph sees the lengths of each
// replay, and no token is left out whatever length the host expected.
//
// Partial slots: a split sequence is the last segment of the first unit it
// touches (slot 1 of that unit) and the first segment of every later one
// (slot 0), so two slots per unit suffice and the workspace does not grow
// with the batch.  The first unit also leaves a merge descriptor (the
// sequence and its unit count), so merge_splits reads one descriptor per
// unit instead of planning again.  Empty sequences get their zero output
// from the unit whose range holds their (empty) start.
//
// (Merging in the decode launch by the last-arriving workgroup needs a
// device-scope release by every splitting workgroup, which writes back its
// XCD's L2: that measured 2.4x slower on ragged batches.)
#pragma once

#include "gi_kernels.h"

namespace gi {

// Workgroups per CU the grid aims at (two are resident per CU at the decode
// kernels' register use, so the units run in one round), and the shortest
// range of a unit (in 32-token blocks).
constexpr int kDecodeWgPerCu = 2;
constexpr int kMinUnitBlocks = 8;
constexpr int kPlanBlock = 32;

__device__ __forceinline__ int plan_len(const DecodeArgs &a, int b, int64_t cap, bool &bad)
{
    int len = a.seq_lens[b];
    if (len < 0 || (int64_t)len > cap) {
        bad = true;
        len = len < 0 ? 0 : (int)cap;
    }
    return len;
}

__device__ __forceinline__ int plan_nblk(int len) { return (len + kPlanBlock - 1) / kPlanBlock; }

// Workgroup-wide (NT threads, every thread calls it): blocks of the whole
// stream and the unit range cb.  Lengths below zero or beyond what the block
// table maps are clamped (and raise FLAG_BAD_SLOT when `flag` is set).
template <int NT>
__device__ void plan_range(const DecodeArgs &a, bool flag, int &total, int &cb)
{
    constexpr int NW = NT / 64;
    __shared__ int64_t s_tot[NW];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t cap = (int64_t)a.max_blocks * a.L.page_tokens;
    bool bad = false;
    int64_t sum = 0;
    for (int b = tid; b < a.batch; b += NT)
        sum += plan_nblk(plan_len(a, b, cap, bad));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        sum += __shfl_xor(sum, o);
    if (lane == 0)
        s_tot[w] = sum;
    if (bad && flag && a.status)
        atomicOr(a.status, FLAG_BAD_SLOT);
    __syncthreads();
    int64_t t = 0;
#pragma unroll
    for (int i = 0; i < NW; i++)
        t += s_tot[i];
    total = (int)t;
    const int per = (int)((t + a.plan_units - 1) / a.plan_units);
    cb = per > kMinUnitBlocks ? per : kMinUnitBlocks;
}

// A unit's walk over the block stream: the sequence it is in (b, whose first
// block is sblk) and its range [blk0, blk1).
struct UnitCursor {
    int b, sblk, blk0, blk1, unit, cb;
};

// The segment of sequence b (length len) inside the unit's range: tokens
// [t0, t1), and whether the sequence continues outside the range (then a
// partial goes to slot `slot` of the unit; otherwise out is written).
struct Segment {
    int t0, t1;
    bool split;
    int slot;
};

__device__ __forceinline__ Segment plan_segment(const UnitCursor &c, int len)
{
    const int nb = plan_nblk(len);
    Segment s;
    const int lo = max(c.blk0, c.sblk) - c.sblk, hi = min(c.blk1, c.sblk + nb) - c.sblk;
    s.t0 = lo * kPlanBlock;
    s.t1 = min(len, hi * kPlanBlock);
    s.split = c.sblk < c.blk0 || c.sblk + nb > c.blk1;
    s.slot = c.sblk < c.blk0 ? 0 : 1;
    return s;
}

// The cursor is the same in every lane: kept in scalar registers, so that
// the block-table entries it addresses are read through the scalar cache (as
// vector loads, each would wait for every K/V load in flight).
__device__ __forceinline__ void plan_uniform(UnitCursor &c)
{
    c.b = __builtin_amdgcn_readfirstlane(c.b);
    c.sblk = __builtin_amdgcn_readfirstlane(c.sblk);
    c.blk0 = __builtin_amdgcn_readfirstlane(c.blk0);
    c.blk1 = __builtin_amdgcn_readfirstlane(c.blk1);
    c.unit = __builtin_amdgcn_readfirstlane(c.unit);
    c.cb = __builtin_amdgcn_readfirstlane(c.cb);
}

// Zero output (an empty context, as the reference's Softmax returns early on
// an empty slice, kernels.go:49-51) of sequence b's heads of kv head kvh, by
// the calling wave.
__device__ __forceinline__ void plan_zero_rows(const DecodeArgs &a, int b, int kvh)
{
    const int HD = a.L.head_dim, G = a.num_heads / a.L.num_kv_heads;
    float *o = a.out + ((int64_t)b * a.num_heads + kvh * G) * HD;
    for (int e = threadIdx.x & 63; e < G * HD; e += 64)
        o[e] = 0.0f;
}

// Owner of an empty sequence whose blocks would start at S: the unit whose
// range holds S (the last unit for S at the very end), so that exactly one
// unit writes its zero output.
__device__ __forceinline__ int plan_empty_owner(const DecodeArgs &a, int S, int cb)
{
    return min(S / cb, a.plan_units - 1);
}

// Merge descriptor of unit u (two ints after the partial slots): the
// sequence that starts in u's range and continues past it, and how many units
// hold its partials; -1 when there is none.  Written by the kv head 0
// workgroup of each unit, read by merge_splits.
__device__ __forceinline__ int *plan_desc(const DecodeArgs &a, int u) { return a.plan_desc + 2 * u; }

// Batches of at most 64 sequences fit one wave's lanes: each wave then plans
// alone from one load per lane, with shuffles and no barrier (the prologue
// of a latency-bound small launch).
__device__ __forceinline__ void plan_wave(const DecodeArgs &a, bool flag, int &n, int &S, int &total, int &cb)
{
    const int lane = threadIdx.x & 63;
    const int64_t cap = (int64_t)a.max_blocks * a.L.page_tokens;
    bool bad = false;
    n = lane < a.batch ? plan_nblk(plan_len(a, lane, cap, bad)) : 0;
    if (flag && __ballot(bad) && threadIdx.x == 0 && a.status)
        atomicOr(a.status, FLAG_BAD_SLOT);
    int x = n; // inclusive scan over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o)
            x += y;
    }
    S = x - n;
    total = __shfl(x, 63);
    const int per = (total + a.plan_units - 1) / a.plan_units;
    cb = per > kMinUnitBlocks ? per : kMinUnitBlocks;
}

// Workgroup-wide (NT threads, every thread calls it): the cursor of work unit
// `unit` for kv head kvh.  False for a unit whose range is past the end of the
// stream.  `flag`: this workgroup reports clamped lengths (one per launch).
// Also writes the zero output of the empty sequences the unit owns, and
// clears the unit's merge descriptor (kv head 0).
template <int NT>
__device__ bool plan_unit(const DecodeArgs &a, int unit, int kvh, bool flag, UnitCursor &c)
{
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    c.unit = unit;
    if (kvh == 0 && tid == 0) {
        plan_desc(a, unit)[0] = -1;
        plan_desc(a, unit)[1] = 0;
    }
    if (a.batch <= 64) {
        int n, S, total, cb;
        plan_wave(a, flag, n, S, total, cb);
        uint64_t empty = __ballot(lane < a.batch && n == 0 && plan_empty_owner(a, S, cb) == unit);
        if (w == 0)
            for (; empty; empty &= empty - 1)
                plan_zero_rows(a, __ffsll((unsigned long long)empty) - 1, kvh);
        c.cb = cb;
        c.blk0 = unit * cb;
        c.blk1 = min(c.blk0 + cb, total);
        const uint64_t hit = __ballot(n > 0 && c.blk0 >= S && c.blk0 < S + n);
        if (!hit || c.blk0 >= total)
            return false;
        c.b = __ffsll((unsigned long long)hit) - 1;
        c.sblk = __shfl(S, c.b);
        plan_uniform(c);
        return true;
    }
    constexpr int NW = NT / 64;
    __shared__ int s_cnt[NW];
    __shared__ int s_hit[2];
    const int64_t cap = (int64_t)a.max_blocks * a.L.page_tokens;
    if (tid == 0)
        s_hit[0] = -1;
    // (the barrier inside plan_range orders that store before the scan)
    int total, cb;
    plan_range<NT>(a, flag, total, cb);
    const int start = unit * cb;
    int carry = 0;
    // rounds of NT sequences until the range (and the empty sequences at its
    // end) are placed
    for (int base = 0; base < a.batch && carry <= start + cb; base += NT) {
        const int b = base + tid;
        bool unused = false;
        const int n = b < a.batch ? plan_nblk(plan_len(a, b, cap, unused)) : 0;
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
        const int S = before + x - n;
        if (n > 0 && start >= S && start < S + n) {
            s_hit[0] = b;
            s_hit[1] = S;
        }
        for (uint64_t empty = __ballot(b < a.batch && n == 0 && plan_empty_owner(a, S, cb) == unit); empty;
             empty &= empty - 1)
            plan_zero_rows(a, base + 64 * w + __ffsll((unsigned long long)empty) - 1, kvh);
        carry += all;
        // the hit is visible, and s_cnt is free for the next round
        __syncthreads();
    }
    c.cb = cb;
    c.blk0 = start;
    c.blk1 = min(start + cb, total);
    c.b = s_hit[0];
    c.sblk = s_hit[1];
    plan_uniform(c);
    return c.b >= 0 && start < total;
}

// Moves the cursor to the next sequence with blocks in the unit's range
// (nblk: blocks of the current one); false when the range is done.  Uniform
// over the caller's threads.
__device__ __forceinline__ bool plan_next(const DecodeArgs &a, UnitCursor &c, int nblk)
{
    if (c.sblk + nblk >= c.blk1)
        return false;
    c.sblk += nblk;
    const int64_t cap = (int64_t)a.max_blocks * a.L.page_tokens;
    for (c.b++; c.b < a.batch; c.b++) {
        bool unused = false;
        if (plan_nblk(plan_len(a, c.b, cap, unused)) > 0)
            return true;
    }
    return false;
}

// Partial slot k (0 or 1) of unit u for kv head kvh (G * (HD + 2) floats).
__device__ __forceinline__ float *plan_slot(const DecodeArgs &a, int u, int k, int kvh, int G, int HD)
{
    return a.ws + ((int64_t)(2 * u + k) * a.L.num_kv_heads + kvh) * ((int64_t)G * (HD + 2));
}

} // namespace gi
