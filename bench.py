"""Decode-step benchmark of the paged KV-cache path on one MI355X.

Workload (default): Llama-3-8B-shaped KV path -- 32 layers, 32 q / 8 kv
heads, head_dim 128, fp16 KV, 16-token pages, batch 256, every sequence at
8192 tokens of context, pool fragmented (pages drawn from a shuffled free
list, then 10 % of the sequences freed and re-allocated).  One step = for
each of the 32 layers: append the new token's K/V (position 8191, through
the block table) then paged decode attention over all 8192 tokens, through
the product's decode-step entry point gi_paged_decode_step (which stores the
token inside the decode launch when the grid fills the CUs once, else in an
append launch before it).  The same step as two calls (gi_paged_append_at_len
then gi_paged_decode_attention) is timed beside it ("two_calls"), and once
more with every launch bracketed by events for the kernels' durations
(roofline).  The calls are prepared once (PagedKVCache.Prepare), so the host
time per call is the C ABI's own.  Inputs (q, k, v, block tables, lengths)
are resident in HBM before timing.

Prints one JSON line (see --help).  Without --config it times the workload
above, then the other configurations of the baseline -- the TinyLlama batch-1
case (A), the ragged batch 32 (B), the Llama-3-70B batch 8 x 32768 (D), the
q8_0 chunked prefill (E), and the workload above over Q8_0 and Q4_0 pages
(C_q8_0, C_q4_0) -- each over at most 10 steps with its parity sample, and
reports them under "other_configs".  --config selects one shape:
  llama8b_b32         Llama-3-8B shape, batch 32, context U[512, 4096]
  llama70b_b8         Llama-3-70B shape (64 q / 8 kv), page 32, batch 8 x 32768
  llama8b_q8_prefill  Llama-3-8B shape, Q8_0 KV: a 4096-token prefill of batch 4
                      in 512-token chunks (append with on-the-fly quantisation,
                      then causal paged attention over the context so far), all
                      32 layers; reports TFLOP/s of the attention
  llama8b_f16_prefill the same prefill over fp16 pages
  llama8b_q4_prefill  the same prefill over Q4_0 pages
  llama8b_f32_prefill the same prefill over f32 pages
  llama8b_b256_8k_rope the headline step with RoPE fused into the append: per
                      layer, q and k turned at position 8191 (theta 5e5) while
                      k/v are stored, then the same paged attention
  llama8b_b256_8k_q8  the headline step over Q8_0 pages (blocks of 32 int8 + fp16
                      scale, kvcache.go's KVTypeQ8_0)
  llama8b_b256_8k_q4  the headline step over Q4_0 pages (blocks of 32 4-bit
                      values + fp16 scale, kvcache.go's KVTypeQ4_0): append
                      with on-the-fly quantisation + paged attention
  llama8b_b64_8k_f32  the headline shape over f32 pages (kvcache.go's KVTypeF32)
                      at batch 64, so that the pool fits one GPU
  llama8b_b256_8k_driver the headline step driven by the continuous-batching
                      decoder (gi_batch): Step() reserves one token per sequence
                      and updates the device tables in place, then per layer
                      RoPE + append + paged attention for the whole batch
  llama8b_oproj_b256_f16 / _q8
                      the O-projection after attention for the same batch:
                      y = x W^T with W 4096 x 4096 (blk.N.attn_output.weight,
                      F16 or Q8_0 GGUF bytes), batch 256, one distinct weight
                      matrix per layer; reports TFLOP/s of the product
  tinyllama_b1        the reference's CPU-runnable case: TinyLlama-1.1B-shaped KV
                      (22 layers, 32 q / 4 kv heads, head_dim 64), f32 pages of
                      16 tokens allocated in order, batch 1; one step = a
                      128-token prompt appended, then 128 decode tokens (append
                      + attention over 129..256 tokens, every layer); reports
                      decode tokens/s, timed beside the oracle running the
                      whole case on one core
  llama8b_fork_b256   copy-on-write forks of 256 Llama-3-8B sequences (8197
                      tokens, fp16): the page copy each fork's first append needs;
                      reports GB/s of the copy against the reference's deep copy
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "paged decode-attn+append HBM GB/s (% of peak) and decode tokens/s, 1 MI355X"

CONFIGS = {
    "llama8b_b256_8k": dict(workload="llama3-8b-shape decode step: append + paged attention",
                            layers=32, q_heads=32, kv_heads=8, head_dim=128, page_tokens=16,
                            batch=256, context="8192", frag=True),
    "llama8b_b256_8k_rope": dict(workload="llama3-8b-shape decode step: RoPE + append + paged "
                                          "attention", layers=32, q_heads=32, kv_heads=8,
                                 head_dim=128, page_tokens=16, batch=256, context="8192",
                                 frag=True, rope_theta=500000.0),
    "llama8b_b256_8k_q4": dict(workload="llama3-8b-shape decode step over q4_0 pages: append + "
                                        "paged attention", layers=32, q_heads=32, kv_heads=8,
                               head_dim=128, page_tokens=16, batch=256, context="8192",
                               frag=True, kv_dtype="q4_0"),
    "llama8b_b256_8k_q8": dict(workload="llama3-8b-shape decode step over q8_0 pages: append + "
                                        "paged attention", layers=32, q_heads=32, kv_heads=8,
                               head_dim=128, page_tokens=16, batch=256, context="8192",
                               frag=True, kv_dtype="q8_0"),
    "llama8b_b64_8k_f32": dict(workload="llama3-8b-shape decode step over f32 pages: append + "
                                        "paged attention", layers=32, q_heads=32, kv_heads=8,
                               head_dim=128, page_tokens=16, batch=64, context="8192",
                               frag=True, kv_dtype="f32"),
    "llama8b_b256_8k_driver": dict(workload="llama3-8b-shape decode step through the batch driver: "
                                            "token reservation + RoPE + append + paged attention",
                                   layers=32, q_heads=32, kv_heads=8, head_dim=128, page_tokens=16,
                                   batch=256, context="8192", frag=True, rope_theta=500000.0,
                                   driver=True),
    "llama8b_oproj_b256_f16": dict(workload="llama3-8b-shape O-projection: 256 x 4096 activations "
                                            "times 4096 x 4096 F16 weights, all 32 layers",
                                   layers=32, dim=4096, batch=256, wtype="f16"),
    "llama8b_oproj_b256_q8": dict(workload="llama3-8b-shape O-projection: 256 x 4096 activations "
                                           "times 4096 x 4096 Q8_0 weights, all 32 layers",
                                  layers=32, dim=4096, batch=256, wtype="q8_0"),
    "tinyllama_b1": dict(workload="tinyllama-1.1b-shape KV path, batch 1: 128-token prompt then 128 "
                                  "decode steps (append + paged attention), all 22 layers",
                         layers=22, q_heads=32, kv_heads=4, head_dim=64, page_tokens=16, batch=1,
                         prompt=128, decode=128, tiny=True),
    "llama8b_b32": dict(workload="llama3-8b-shape decode step, ragged context",
                        layers=32, q_heads=32, kv_heads=8, head_dim=128, page_tokens=16,
                        batch=32, context="U[512,4096]", frag=True),
    "llama70b_b8": dict(workload="llama3-70b-shape decode step, long context",
                        layers=80, q_heads=64, kv_heads=8, head_dim=128, page_tokens=32,
                        batch=8, context="32768", frag=False),
    "llama8b_q8_prefill": dict(workload="llama3-8b-shape q8_0 chunked prefill: append + causal "
                                        "paged attention", layers=32, q_heads=32, kv_heads=8,
                               head_dim=128, page_tokens=16, batch=4, context="4096", chunk=512,
                               frag=True, prefill=True, kv_dtype="q8_0"),
    "llama8b_q4_prefill": dict(workload="llama3-8b-shape q4_0 chunked prefill: append + causal "
                                        "paged attention", layers=32, q_heads=32, kv_heads=8,
                               head_dim=128, page_tokens=16, batch=4, context="4096", chunk=512,
                               frag=True, prefill=True, kv_dtype="q4_0"),
    "llama8b_f32_prefill": dict(workload="llama3-8b-shape f32 chunked prefill: append + causal "
                                         "paged attention", layers=32, q_heads=32, kv_heads=8,
                                head_dim=128, page_tokens=16, batch=4, context="4096", chunk=512,
                                frag=True, prefill=True, kv_dtype="f32", outliers=False),
    "llama8b_fork_b256": dict(workload="llama3-8b-shape copy-on-write fork: 256 sequences forked "
                                        "mid-page, one append each (one page copy per fork, all "
                                        "layers, whatever the context length)",
                              layers=32, q_heads=32, kv_heads=8, head_dim=128, page_tokens=16,
                              batch=256, context="8192", fork=True),
    "llama8b_f16_prefill": dict(workload="llama3-8b-shape fp16 chunked prefill: append + causal "
                                         "paged attention", layers=32, q_heads=32, kv_heads=8,
                                head_dim=128, page_tokens=16, batch=4, context="4096", chunk=512,
                                frag=True, prefill=True, kv_dtype="f16"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def seq_lengths(cfg, seed):
    b = cfg["batch"]
    c = cfg["context"]
    if c.startswith("U["):
        lo, hi = [int(x) for x in c[2:-1].split(",")]
        return np.random.default_rng(seed).integers(lo, hi + 1, size=b).astype(np.int64)
    return np.full(b, int(c), np.int64)


def build_tables(gi, cfg, lens, seed, held=None):
    """Block tables from the host allocator (PagedKVManager), starting from a
    shuffled free list; with frag, 10 % of the sequences are then freed and
    allocated again so their pages come back in a different order."""
    P = cfg["page_tokens"]
    need = int(sum((int(n) + P - 1) // P for n in lens))
    pages = need + (need // 100 + 16 if cfg["frag"] else 0)
    rng = np.random.default_rng(seed)
    mgr = gi.PagedKVManager(cfg["layers"], cfg["kv_heads"] * cfg["head_dim"], pages, P)
    if cfg["frag"]:
        mgr.SetFreeList(rng.permutation(pages).astype(np.int32))
    seqs = []
    held = lens if held is None else held
    for n in held:
        s = mgr.AllocateSequence()
        mgr.AppendTokens(s, int(n))
        seqs.append(s)
    if cfg["frag"]:
        k = max(1, len(seqs) // 10)
        for i in rng.choice(len(seqs), size=k, replace=False):
            mgr.FreeSequence(seqs[i])
            s = mgr.AllocateSequence()
            mgr.AppendTokens(s, int(held[i]))
            seqs[i] = s
    max_blocks = max((int(n) + P - 1) // P for n in lens)
    bt = np.zeros((len(lens), max_blocks), np.int32)
    for i, s in enumerate(seqs):
        ids = mgr.Tables[s].BlockIDs
        bt[i, :len(ids)] = ids
    if held is not lens:
        return mgr, pages, bt, seqs
    return mgr, pages, bt


def fill_pool(torch, pool, cfg, lens, bt, dev, seed):
    """Writes every cached token of every layer through the append path
    (f32 N(0,1) -> truncated fp16), a chunk of sequences at a time."""
    P = cfg["page_tokens"]
    kv_dim = cfg["kv_heads"] * cfg["head_dim"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    chunk_tok = 1 << 19
    # (ids, slots) for all tokens of all sequences, in sequence order
    ids = np.concatenate([np.repeat(bt[i, :(int(n) + P - 1) // P], P)[:int(n)]
                          for i, n in enumerate(lens)]).astype(np.int32)
    slots = np.concatenate([np.arange(int(n), dtype=np.int32) % P for n in lens])
    ids_d = torch.from_numpy(ids).to(dev)
    slots_d = torch.from_numpy(slots).to(dev)
    total = ids.size
    kbuf = torch.empty((min(chunk_tok, total), kv_dim), dtype=torch.float32, device=dev)
    vbuf = torch.empty_like(kbuf)
    for l in range(cfg["layers"]):
        for a in range(0, total, chunk_tok):
            b = min(total, a + chunk_tok)
            kb, vb = kbuf[:b - a], vbuf[:b - a]
            kb.normal_(generator=gen)
            vb.normal_(generator=gen)
            pool.Write(l, ids_d[a:b], slots_d[a:b], kb, vb)
        if l % 8 == 7:
            pool.synchronize()
            log("filled layer", l)
    pool.synchronize()
    del kbuf, vbuf, ids_d, slots_d


def vec_bytes(kv_dtype, kv_dim):
    """Stored bytes of one token vector (kvcache.go:92-105)."""
    return {"f32": 4 * kv_dim, "f16": 2 * kv_dim, "q8_0": kv_dim // 32 * 34,
            "q4_0": kv_dim // 32 * 18}[kv_dtype]


def kv_type_of(gi, kv_dtype):
    return {"f32": gi.KV_F32, "f16": gi.KV_F16, "q8_0": gi.KV_Q8_0, "q4_0": gi.KV_Q4_0}[kv_dtype]


def append_kernel_name(gi, kv_dtype, rope):
    if rope:
        return "rope_append<%d,true>" % kv_type_of(gi, kv_dtype)
    return {"f32": "append_plain<0,true>", "f16": "append_plain<1,true>",
            "q8_0": "append_q8<true>", "q4_0": "append_q4<true>"}[kv_dtype]


def step_bytes(cfg, lens):
    """Algorithmic HBM bytes of one decode step, split into the attention
    kernel's and the append kernel's share (per step, all layers)."""
    P = cfg["page_tokens"]
    kv_dim = cfg["kv_heads"] * cfg["head_dim"]
    qd = cfg["q_heads"] * cfg["head_dim"]
    bpv = vec_bytes(cfg.get("kv_dtype", "f16"), kv_dim)
    L = np.asarray(lens, np.int64)
    attn = (2 * L * bpv + ((L + P - 1) // P) * 4 + qd * 4 + qd * 4 + 4).sum()
    append = len(L) * (2 * kv_dim * 4 + 2 * bpv + 4 + 4)
    if cfg.get("rope_theta"):
        append += len(L) * (2 * qd * 4 + (kv_dim // 2) * 8)   # q read + written, cos/sin row
    return int(attn) * cfg["layers"], int(append) * cfg["layers"]


def profiled_traffic(kernel, workload):
    """HBM bytes per launch of a kernel on a workload, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE summary committed under profiles/ (a line
    'TRAFFIC kernel=... workload=... bytes_per_launch=N'), or None."""
    import glob
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        for line in open(path):
            if not line.startswith("TRAFFIC "):
                continue
            kv = dict(x.split("=", 1) for x in line.split()[1:])
            if kv.get("kernel") == kernel and kv.get("workload") == workload:
                return int(kv["bytes_per_launch"]), os.path.relpath(path, ROOT)
    return None


def _timed_units(fn, budget_s, max_units):
    units, t0 = 0, time.perf_counter()
    while True:
        fn()
        units += 1
        el = time.perf_counter() - t0
        if el >= budget_s or units >= max_units:
            return units, el


def cpu_baseline(oracle, cfg, budget_s=10.0, mt_budget_s=6.0):
    """The oracle's decode (widen the stored vectors -> f32, then the
    reference loop of forward.go:242-267) timed on the host for a bounded
    sample of the same workload: whole (sequence, layer) units at the
    configured context, repeated until about budget_s of work, extrapolated to
    the full step by the number of units.  Two figures: one thread (the
    reference's decode attention is single-threaded, forward.go:247-267) and
    every host core the process may use (at most 16), with each unit's q-heads
    split over the threads as forward.go:1342-1378 splits heads over
    goroutines; the threaded rows are bit-identical to the one-thread ones."""
    H, kvh, hd = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"]
    kv_dim = kvh * hd
    lens = seq_lengths(cfg, 11)
    L = int(np.median(lens))
    kt = {"f32": 0, "f16": 1, "q8_0": 2, "q4_0": 3}[cfg.get("kv_dtype", "f16")]
    k = oracle.store_vectors(kt, oracle.normal(1, (L, kv_dim)))
    v = oracle.store_vectors(kt, oracle.normal(2, (L, kv_dim)))
    q = oracle.normal(3, (1, H * hd))
    sc = oracle.attn_scale(hd)
    off, ln = np.zeros(1, np.int64), np.array([L], np.int32)
    full_units = float(np.sum(lens)) / L * cfg["layers"]

    def figure(units, el, cores):
        step_s = el / units * full_units
        return {"value": round(cfg["batch"] / step_s, 4), "unit": "tokens/s", "cores": cores,
                "kind": "port",
                "sample": "%d (sequence, layer) decode units at L=%d on %d thread%s, %.1f s; "
                          "extrapolated x%.0f to the full step"
                          % (units, L, cores, "" if cores == 1 else "s", el, full_units / units),
                "ms_per_step": round(step_s * 1e3, 1)}

    u1, e1 = _timed_units(lambda: oracle.decode_batch(kt, q, k, v, off, ln, H, kvh, hd, sc),
                          budget_s, 256)
    one = figure(u1, e1, 1)
    n = oracle.host_threads()
    ran = [1]

    def mt():
        ran[0] = oracle.decode_batch(kt, q, k, v, off, ln, H, kvh, hd, sc, threads=n)[1]

    un, en = _timed_units(mt, mt_budget_s, 4096)
    res = figure(un, en, ran[0])
    res["one_thread"] = one
    res.update(host_cpus())
    return res


def host_cpus():
    """The host's CPU count as the machine reports it (nproc) and as this
    process may use it, beside the threads the all-cores figure ran on: the
    baseline takes at most 16, the host share of one GPU on these boxes."""
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = None
    return {"nproc": os.cpu_count(), "affinity_cpus": aff,
            "threads_note": "the all-cores figure uses min(affinity, 16) threads, the host share of one GPU"}


def cpu_baseline_prefill(oracle, cfg, budget_s=8.0, mt_budget_s=6.0):
    """The oracle's chunked-prefill attention (forward.go:547-577, over
    f32 K/V: quantised pages dequantised first, a pass over the context that is
    under 0.1 % of the work and left out) on the host for a bounded sample: 16
    queries at the end of the last chunk (context 4096), repeated until about
    budget_s of work, on one thread and on every host core the process may
    use (at most 16; rows split over threads).  Reported as TFLOP/s of the
    same algorithmic flop count as the GPU figure."""
    H, kvh, hd = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"]
    Ltot = int(cfg["context"])
    nq, start = 16, Ltot - 16
    k = oracle.normal(11, (Ltot, kvh * hd))
    v = oracle.normal(12, (Ltot, kvh * hd))
    q = oracle.normal(13, (nq, H * hd))
    sc = oracle.attn_scale(hd)
    flops = 4 * hd * H * sum(start + i + 1 for i in range(nq))

    def figure(units, el, cores):
        tflops = flops * units / el / 1e12
        full_s = prefill_flops(cfg) / (tflops * 1e12)
        return {"value": round(tflops, 6), "unit": "TFLOP/s", "cores": cores, "kind": "port",
                "sample": "%d units of 16 queries at positions %d..%d over f32 K/V (%.2f GFLOP "
                          "each) on %d thread%s, %.1f s; the whole prefill would take %.0f s"
                          % (units, start, Ltot - 1, flops / 1e9, cores,
                             "" if cores == 1 else "s", el, full_s)}

    u1, e1 = _timed_units(
        lambda: oracle.attention_prefill(q, k, v, H, kvh, hd, start, nq, 1 << 30, sc), budget_s, 64)
    n = oracle.host_threads()
    un, en = _timed_units(
        lambda: oracle.attention_prefill(q, k, v, H, kvh, hd, start, nq, 1 << 30, sc, threads=n),
        mt_budget_s, 1024)
    res = figure(un, en, n)
    res["one_thread"] = figure(u1, e1, 1)
    res.update(host_cpus())
    return res


def prefill_flops(cfg):
    """Exact causal attention flops of the whole prefill: per sequence and
    layer 2 products x 2 flops x head_dim x q_heads x sum_{i=1..L} i."""
    L = int(cfg["context"])
    return (4 * cfg["head_dim"] * cfg["q_heads"] * (L * (L + 1) // 2) * cfg["layers"]
            * cfg["batch"])


def run_fork(args, gi, torch, dev, cfg):
    """Forks each of `batch` sequences at its full length (a partial last
    page) and appends one token to every fork: the allocator hands out one
    copy-on-write pair per fork, and gi_paged_copy_pages copies those pages in
    all layers.  Times the device copy; the reference instead deep-copies the
    whole contiguous cache per fork (KVCache.ForkAt, kvcache.go:225-284)."""
    H, kvh, hd, P, layers = (cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"],
                             cfg["page_tokens"], cfg["layers"])
    B, L = cfg["batch"], int(cfg["context"])
    # only the partial last page is copied, so the sequences here hold 5
    # tokens (one page each); the context length matters to the reference's
    # deep copy, timed below at L tokens
    tail = 5
    need = 2 * B + 16
    mgr = gi.PagedKVManager(layers, kvh * hd, need, P)
    pool = gi.PagedKVCache(layers, kvh, hd, P, need, gi.KV_F16)
    seqs = [mgr.AllocateSequence() for _ in range(B)]
    for s in seqs:
        mgr.AppendTokens(s, tail)
    forks = [mgr.ForkSequence(s, tail) for s in seqs]
    pairs = []
    for f in forks:
        _, _, (src, dst) = mgr.AppendTokensCOW(f, 1)
        pairs.append((src, dst))
    assert all(p[0] >= 0 for p in pairs), "every fork of a mid-page sequence copies one page"
    src = torch.tensor([p[0] for p in pairs], dtype=torch.int32, device=dev)
    dst = torch.tensor([p[1] for p in pairs], dtype=torch.int32, device=dev)
    page_bytes = pool.page_bytes()[0]
    moved = 2 * B * layers * page_bytes  # read + write
    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        pool.CopyPages(src, dst)
    pool.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        pool.CopyPages(src, dst)
    e1.record(stream)
    torch.cuda.synchronize()
    pool.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    gbs = moved / (ms * 1e-3) / 1e9
    log("fork copy %.3f ms for %d forks (%.1f MB moved, %.1f GB/s)" % (ms, B, moved / 1e6, gbs))
    # parity: the copied page equals its source in every layer (sampled)
    ok = True
    if not args.no_parity:
        for l in (0, layers - 1):
            a, _ = pool.Get(l, src[:1].contiguous(), P)
            b, _ = pool.Get(l, dst[:1].contiguous(), P)
            pool.synchronize()
            ok = ok and bool(torch.equal(a, b))
    cpu = None
    if not args.no_cpu_baseline:
        # the reference's deep copy of one fork: ForkAt copies the contiguous
        # f32 cache, 2 x MaxSeq x kvDim x 4 B per layer (timed for one layer)
        kvd = kvh * hd
        srcb = np.ones(L * kvd, np.float32)
        dstb = np.empty_like(srcb)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 3.0:
            np.copyto(dstb, srcb)
            np.copyto(dstb, srcb)
            n += 1
        per_layer = (time.perf_counter() - t0) / n
        per_fork = per_layer * layers
        cpu = {"value": round(1.0 / per_fork, 4), "unit": "forks/s", "cores": 1, "kind": "port",
               "sample": "%d deep copies of one layer's K and V (%d tokens x %d f32 each) on 1 "
                         "thread, %.3f s per fork of %d layers" % (n, L, kvd, per_fork, layers)}
    res = {
        "metric": METRIC,
        "value": round(B / (ms * 1e-3), 1),
        "unit": "forks/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": cfg["workload"], "layers": layers, "kv_heads": kvh,
                   "head_dim": hd, "kv_dtype": "f16", "page_tokens": P, "batch": B,
                   "context": L},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "copy_pages_kernel", "bytes_per_launch": moved},
        "cpu_baseline": cpu,
        "parity": {"copied_pages_equal": ok, "pass": ok},
    }
    pool.close()
    return res


def run_prefill(args, gi, torch, dev, cfg):
    """Whole 4096-token prefill in 512-token chunks, all layers."""
    H, kvh, hd, P, layers = (cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"],
                             cfg["page_tokens"], cfg["layers"])
    kv_dim = kvh * hd
    B, Ltot, C = cfg["batch"], int(cfg["context"]), cfg["chunk"]
    lens = np.full(B, Ltot, np.int64)
    mgr, pages, bt = build_tables(gi, cfg, lens, args.seed)
    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    kv_type = kv_type_of(gi, cfg["kv_dtype"])
    pool = gi.PagedKVCache(layers, kvh, hd, P, pages, kv_type, stream=stream)
    pool.set_decode_kernel(args.decode_kernel)
    bt_d = torch.from_numpy(bt).to(dev)
    # per-chunk (ids, slots) of the batch's tokens, sequence-major
    ids = np.stack([np.repeat(bt[i], P)[:Ltot] for i in range(B)])
    slots = np.tile(np.arange(Ltot, dtype=np.int32) % P, (B, 1))
    chunk_ids = [torch.from_numpy(np.ascontiguousarray(ids[:, c:c + C]).reshape(-1)).to(dev)
                 for c in range(0, Ltot, C)]
    chunk_slots = [torch.from_numpy(np.ascontiguousarray(slots[:, c:c + C]).reshape(-1)).to(dev)
                   for c in range(0, Ltot, C)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)

    outliers = cfg.get("outliers", True)

    def outl(t):
        # N(0,1) with 1 % of entries at +-8 sigma (plain N(0,1) when the
        # config turns outliers off)
        if not outliers:
            return t
        m = torch.rand(t.shape, generator=gen, device=dev) < 0.01
        sgn = torch.where(torch.rand(t.shape, generator=gen, device=dev) < 0.5, -8.0, 8.0)
        return torch.where(m, sgn, t)

    q = outl(torch.randn((layers, B, C, H * hd), generator=gen, device=dev))
    kn = outl(torch.randn((layers, B * C, kv_dim), generator=gen, device=dev))
    vn = outl(torch.randn((layers, B * C, kv_dim), generator=gen, device=dev))
    out = torch.empty((layers, B, C, H * hd), device=dev)
    scale = gi.attn_scale(hd)
    nch = Ltot // C
    ev = []

    def prefill(record):
        for ci in range(nch):
            sp = torch.full((B,), ci * C, dtype=torch.int32, device=dev)
            for l in range(layers):
                pool.Write(l, chunk_ids[ci], chunk_slots[ci], kn[l], vn[l])
                if record:
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                pool.AttentionGQABatch(out[l], q[l], l, bt_d, sp, H, scale, C)
                if record:
                    e1.record(stream)
                    ev.append((e0, e1))

    for _ in range(args.warmup):
        prefill(False)
    pool.synchronize()
    torch.cuda.synchronize()
    s0 = torch.cuda.Event(enable_timing=True)
    s1 = torch.cuda.Event(enable_timing=True)
    s0.record(stream)
    for _ in range(args.steps):
        prefill(True)
    s1.record(stream)
    torch.cuda.synchronize()
    pool.synchronize()
    ms_step = s0.elapsed_time(s1) / args.steps
    attn_ms = sum(a.elapsed_time(b) for a, b in ev) / args.steps
    flops = prefill_flops(cfg)
    tflops = flops / (attn_ms * 1e-3) / 1e12
    # The kernels' own durations: the step's attention launches again, on
    # the filled cache (each reads what it read in the step: context before
    # its chunk plus the chunk, causally), back to back with events only at
    # the two ends.  An event pair around every launch, as in the step, adds
    # a few microseconds to each 0.1-0.2 ms launch.  Chunk order is kept, so
    # out ends as the step left it.
    sps = [torch.full((B,), ci * C, dtype=torch.int32, device=dev) for ci in range(nch)]

    def attention_only():
        for ci in range(nch):
            for l in range(layers):
                pool.AttentionGQABatch(out[l], q[l], l, bt_d, sps[ci], H, scale, C)

    attention_only()
    torch.cuda.synchronize()
    a0 = torch.cuda.Event(enable_timing=True)
    a1 = torch.cuda.Event(enable_timing=True)
    a0.record(stream)
    for _ in range(args.steps):
        attention_only()
    a1.record(stream)
    torch.cuda.synchronize()
    pool.synchronize()
    b2b_ms = a0.elapsed_time(a1) / args.steps
    k_tflops = flops / (b2b_ms * 1e-3) / 1e12
    launch_us = b2b_ms * 1e3 / (nch * layers)
    log("prefill %.3f ms (attention %.3f ms, %.1f TFLOP/s; launches back to back %.3f ms, %.1f us each, "
        "%.1f TFLOP/s)" % (ms_step, attn_ms, tflops, b2b_ms, launch_us, k_tflops))

    parity = None
    if not args.no_parity:
        import oracle
        # last chunk of sequence 0, layer 5: the oracle over the gathered pages
        i, l = 0, 5
        kw, vw = pool.Get(l, bt_d[i], Ltot, widen=True)
        pool.synchronize()
        want = oracle.attention_prefill(q[l, i].cpu().numpy(), kw.cpu().numpy(), vw.cpu().numpy(),
                                        H, kvh, hd, Ltot - C, C, 1 << 30, scale)
        got = out[l, i].cpu().numpy().astype(np.float64).reshape(-1, hd)
        w = want.astype(np.float64).reshape(-1, hd)
        err = float((np.abs(got - w).max(axis=1) / np.abs(w).max(axis=1)).max())
        tol = 1e-5 if cfg["kv_dtype"] == "f32" else 1e-3
        parity = {"sampled_seq_layer_chunk": [i, l, nch - 1], "max_rel_err": err, "tol": tol,
                  "pass": bool(err <= tol)}
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        cpu = cpu_baseline_prefill(oracle, cfg)
    res = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (N(0,1) with 1% outliers at +-8 sigma)" if outliers else "synthetic (N(0,1))",
        "config": {"workload": cfg["workload"], "layers": layers, "q_heads": H, "kv_heads": kvh,
                   "head_dim": hd, "kv_dtype": cfg["kv_dtype"], "page_tokens": P, "batch": B,
                   "context": Ltot, "chunk": C},
        "attention_ms_per_step": round(attn_ms, 4),
        "append_and_gaps_ms_per_step": round(ms_step - attn_ms, 4),
        "roofline": {"bound": "mfma", "achieved": round(k_tflops, 2), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(k_tflops / 2500.0, 4), "traffic": None,
                     "kernel": "paged prefill attention",
                     "flops_per_step": flops, "launches_per_step": nch * layers,
                     "launch_ms": round(launch_us * 1e-3, 5),
                     "timing": "the step's attention launches back to back, events at the two ends"},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    pool.close()
    return res


def run_driver(args, gi, torch, dev, cfg):
    """The headline decode step through the continuous-batching driver:
    every sequence holds 8191 tokens; each step gi_batch_step reserves token
    8191 + i for all 256 sequences (one batched AppendToken, device tables
    updated in place), then per layer RoPE + append + paged attention for the
    whole batch.  Lengths grow by one per step, from 8192 at the first
    step."""
    H, kvh, hd, P, layers = (cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"],
                             cfg["page_tokens"], cfg["layers"])
    kv_dim = kvh * hd
    extra = 10                                      # isolated Step() timings after the run
    grow = args.warmup + args.steps + extra
    lens = seq_lengths(cfg, args.seed) + grow       # pages for the whole run
    held = lens - grow - 1                          # 8191 tokens cached
    mgr, pages, bt, seqs = build_tables(gi, cfg, lens, args.seed, held=held)
    batch = len(seqs)
    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    pool = gi.PagedKVCache(layers, kvh, hd, P, pages, gi.KV_F16, stream=stream)
    pool.set_decode_kernel(args.decode_kernel)
    t0 = time.perf_counter()
    fill_pool(torch, pool, cfg, held, bt, dev, args.seed)
    log("pool filled (%.1f s)" % (time.perf_counter() - t0))
    max_len = int(held.max()) + grow
    pool.SetRoPE(cfg["rope_theta"], 0, max_len + 1)
    drv = gi.BatchDecoder(mgr, pool, batch, (max_len + P - 1) // P)
    for sq in seqs:
        drv.Add(sq)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 1)
    q = torch.randn((layers, batch, H * hd), generator=gen, device=dev)
    kn = torch.randn((layers, batch, kv_dim), generator=gen, device=dev)
    vn = torch.randn((layers, batch, kv_dim), generator=gen, device=dev)
    out = torch.empty((layers, batch, H * hd), device=dev)
    scale = gi.attn_scale(hd)
    def step():
        drv.Step()
        for l in range(layers):
            drv.DecodeLayer(l, H, q[l], kn[l], vn[l], out[l], scale, rope=True)

    for _ in range(args.warmup):
        step()
    pool.synchronize()
    torch.cuda.synchronize()
    _, lens0 = drv.Rows()
    s0 = torch.cuda.Event(enable_timing=True)
    s1 = torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    s0.record(stream)
    for _ in range(args.steps):
        step()
    s1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    pool.synchronize()
    ms_step = s0.elapsed_time(s1) / args.steps
    # algorithmic bytes at the mean length of the timed steps
    mean_lens = lens0.astype(np.int64) + (args.steps + 1) // 2
    attn_bytes, app_bytes = step_bytes(cfg, mean_lens)
    tot_gbs = (attn_bytes + app_bytes) / (ms_step * 1e-3) / 1e9
    tok_s = batch / (ms_step * 1e-3)
    _, lens_done = drv.Rows()    # what the last timed step attended
    # host cost of Step() alone (256 reservations, mirror updates, uploads
    # queued): isolated calls on an idle device; their tokens are reserved
    # but never written, and the parity check below uses lens_done
    host = []
    for _ in range(extra):
        torch.cuda.synchronize()
        h0 = time.perf_counter()
        drv.Step()
        host.append(time.perf_counter() - h0)
    torch.cuda.synchronize()
    log("driver step %.3f ms (wall %.3f ms), host Step() median %.1f us" %
        (ms_step, wall * 1e3 / args.steps, 1e6 * float(np.median(host))))
    parity = None
    if not args.no_parity:
        import oracle
        lens_now = lens_done
        rng = np.random.default_rng(args.seed + 7)
        worst, checked = 0.0, []
        for _ in range(2):
            r, l = int(rng.integers(batch)), int(rng.integers(layers))
            n = int(lens_now[r])
            t = torch.from_numpy(drv.RowTable(r)).to(dev)
            kw, vw = pool.Get(l, t, n, widen=True)
            pool.synchronize()
            want = oracle.attention_decode(q[l, r].cpu().numpy(), kw.cpu().numpy(), vw.cpu().numpy(),
                                           H, kvh, hd, n, scale)
            got = out[l, r].cpu().numpy().astype(np.float64).reshape(H, hd)
            w = want.astype(np.float64).reshape(H, hd)
            worst = max(worst, float((np.abs(got - w).max(axis=1) / np.abs(w).max(axis=1)).max()))
            checked.append([r, l])
        parity = {"sampled_row_layer": checked, "max_rel_err": worst, "tol": 1e-3,
                  "pass": bool(worst <= 1e-3)}
    res = {
        "metric": METRIC,
        "value": round(tot_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": cfg["workload"], "layers": layers, "q_heads": H, "kv_heads": kvh,
                   "head_dim": hd, "kv_dtype": "f16", "page_tokens": P, "batch": batch,
                   "context": "8191 + 1 per step", "pool_pages": pages,
                   "fragmented_pool": cfg["frag"], "rope_theta": cfg["rope_theta"]},
        "hbm_frac_of_peak": round(tot_gbs / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(tok_s, 1),
        "driver_host_us_per_step_median": round(1e6 * float(np.median(host)), 1),
        "parity": parity,
        "cpu_baseline": None,
        "roofline": None,
    }
    drv.close()
    pool.close()
    return res


def run_oproj(args, gi, torch, dev, cfg):
    """y = x W^T per layer (gi_matmul_batch), W uploaded from GGUF bytes,
    one matrix per layer so nothing is served from the caches across
    layers."""
    import oracle
    D, B, layers = cfg["dim"], cfg["batch"], cfg["layers"]
    t = {"f16": gi.GGML_F16, "q8_0": gi.GGML_Q8_0}[cfg["wtype"]]
    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    pool = gi.PagedKVCache(1, 1, 32, 16, 1, gi.KV_F16, stream=stream)
    W = oracle.normal(args.seed, (D, D)) * np.float32(1.0 / 64)
    raw = oracle.quantize_weights(t, W)
    t0 = time.perf_counter()
    ws = [gi.Weights(pool, t, D, D, raw) for _ in range(layers)]
    log("weights uploaded (%d x %.1f MB, %.1f s)" % (layers, raw.nbytes / 1e6, time.perf_counter() - t0))
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 1)
    x = torch.randn((layers, B, D), generator=gen, device=dev)
    y = torch.empty((layers, B, D), device=dev)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(layers * args.steps)]

    def step(rec=None):
        for l in range(layers):
            if rec is not None:
                ev[rec + l][0].record(stream)
            ws[l].MatMulBatch(y[l], x[l])
            if rec is not None:
                ev[rec + l][1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    s0 = torch.cuda.Event(enable_timing=True)
    s1 = torch.cuda.Event(enable_timing=True)
    s0.record(stream)
    for i in range(args.steps):
        step(i * layers)
    s1.record(stream)
    torch.cuda.synchronize()
    pool.synchronize()
    ms_step = s0.elapsed_time(s1) / args.steps
    launch_ms = float(np.mean([a.elapsed_time(b) for a, b in ev]))
    flops = 2.0 * B * D * D
    tflops = flops / (launch_ms * 1e-3) / 1e12
    wbytes = raw.nbytes
    log("oproj %.3f ms per step, %.4f ms per launch, %.1f TFLOP/s, weights %.0f GB/s" %
        (ms_step, launch_ms, tflops, wbytes / (launch_ms * 1e-3) / 1e9))
    parity = None
    if not args.no_parity:
        l = layers - 1
        rows = [0, B // 2, B - 1]
        xs = x[l, rows].cpu().numpy()
        want = oracle.matmul(t, raw, xs, D, D)
        got = y[l, rows].cpu().numpy()
        err = float((np.abs(got - want).max(axis=1) / np.abs(want).max(axis=1)).max())
        parity = {"sampled_layer_rows": [l, rows], "max_rel_err": err, "tol": 1e-5,
                  "pass": bool(err <= 1e-5)}
    cpu = None
    if not args.no_cpu_baseline:
        xs = x[0, :1].cpu().numpy()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 8.0:
            oracle.matmul(t, raw, xs, D, D)
            n += 1
        el = time.perf_counter() - t0
        cpu_tf = 2.0 * D * D * n / el / 1e12
        cpu = {"value": round(cpu_tf, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
               "sample": "%d single-row MatMul calls (4096 x 4096 %s) on 1 thread, %.1f s"
                         % (n, cfg["wtype"], el)}
    res = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (%s weights)" % cfg["wtype"],
        "data": "synthetic",
        "config": {"workload": cfg["workload"], "layers": layers, "dim": D, "batch": B,
                   "weight_type": cfg["wtype"]},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4), "traffic": None,
                     "kernel": "matmul_tile<%d>" % t, "launch_ms": round(launch_ms, 4),
                     "flops_per_launch": flops, "weight_bytes_per_launch": wbytes,
                     "weight_gbs": round(wbytes / (launch_ms * 1e-3) / 1e9, 1)},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    for w in ws:
        w.close()
    pool.close()
    return res


def run_tinyllama(args, gi, torch, dev, cfg):
    """Config A end to end on the device, step = prompt + 128 decode tokens."""
    import oracle
    H, kvh, hd, P, layers = (cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"],
                             cfg["page_tokens"], cfg["layers"])
    kv_dim = kvh * hd
    T0, ND = cfg["prompt"], cfg["decode"]
    total = T0 + ND
    pages = total // P
    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    pool = gi.PagedKVCache(layers, kvh, hd, P, pages, gi.KV_F32, stream=stream)
    pool.set_decode_kernel(args.decode_kernel)
    K = torch.from_numpy(np.stack([oracle.normal(1000 + l, (total, kv_dim)) for l in range(layers)])).to(dev)
    V = torch.from_numpy(np.stack([oracle.normal(2000 + l, (total, kv_dim)) for l in range(layers)])).to(dev)
    Q = torch.from_numpy(oracle.normal(3000, (ND, layers, H * hd))).to(dev)
    out = torch.empty((ND, layers, H * hd), device=dev)
    scale = gi.attn_scale(hd)
    # pages allocated in order, as the reference's allocator hands them out
    mgr = gi.PagedKVManager(layers, kv_dim, pages, P)
    sid = mgr.AllocateSequence()
    ids, slots = mgr.AppendTokens(sid, total)
    bt = torch.tensor(mgr.Tables[sid].BlockIDs, dtype=torch.int32, device=dev)[None, :].contiguous()
    ids_d = torch.from_numpy(ids[:T0].copy()).to(dev)
    slots_d = torch.from_numpy(slots[:T0].copy()).to(dev)
    lens = [torch.tensor([T0 + i + 1], dtype=torch.int32, device=dev) for i in range(ND)]

    def run():
        for l in range(layers):
            pool.Write(l, ids_d, slots_d, K[l, :T0], V[l, :T0])
        for i in range(ND):
            n = T0 + i + 1
            for l in range(layers):
                pool.DecodeStep(out[i, l], Q[i, l], K[l, n - 1:n], V[l, n - 1:n], l, bt, lens[i], H, scale,
                                max_seq_len=n)

    for _ in range(max(1, args.warmup)):
        run()
    torch.cuda.synchronize()
    s0 = torch.cuda.Event(enable_timing=True)
    s1 = torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    s0.record(stream)
    for _ in range(args.steps):
        run()
    s1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - w0) / args.steps
    pool.synchronize()
    ms_eager = s0.elapsed_time(s1) / args.steps
    ms_step, launch = ms_eager, "eager (one DecodeStep call per layer and token)"
    if not args.no_graph:
        # The step is 22 x 128 tiny launches, so host time bounds it.  The
        # entry points allocate nothing once the workspace is sized and never
        # synchronise, so the whole step can be captured as one HIP graph on
        # the pool's stream and replayed; every replay must reproduce the
        # eager outputs bit for bit.
        ref = out.clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            run()
        for _ in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            if not torch.equal(out, ref):
                raise RuntimeError("tinyllama: a graph replay differs from the eager step")
        pool.synchronize()
        g0 = torch.cuda.Event(enable_timing=True)
        g1 = torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        g0.record(stream)
        for _ in range(args.steps):
            graph.replay()
        g1.record(stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - w0) / args.steps
        pool.synchronize()
        ms_step = g0.elapsed_time(g1) / args.steps
        # one launch per layer and token when the decode launch stores the
        # token itself, else an append launch before each
        per_token = 1 if pool.decode_step_fuses(1, H, T0 + ND) else 2
        launch = "one HIP graph of the whole step (its %d launches captured once)" % (layers + ND * layers * per_token)
    tok_s = ND / (ms_step * 1e-3)
    # algorithmic bytes of one step: the prompt's append, then per decode
    # token and layer K+V over n tokens, q/out, the appended K/V
    e = 4
    byt = layers * T0 * 2 * kv_dim * (4 + e)
    for i in range(ND):
        n = T0 + i + 1
        byt += layers * (2 * n * kv_dim * e + ((n + P - 1) // P) * 4 + 2 * H * hd * 4
                         + 2 * kv_dim * (4 + e))
    gbs = byt / (ms_step * 1e-3) / 1e9
    log("tinyllama step %.3f ms (wall %.3f ms): %.0f decode tokens/s; eager %.3f ms (%.0f tokens/s)" %
        (ms_step, wall * 1e3, tok_s, ms_eager, ND / (ms_eager * 1e-3)))
    parity = None
    if not args.no_parity:
        Kh, Vh, Qh, Oh = K.cpu().numpy(), V.cpu().numpy(), Q.cpu().numpy(), out.cpu().numpy()
        worst = 0.0
        for i in (0, ND // 2, ND - 1):
            n = T0 + i + 1
            for l in (0, layers - 1):
                want = oracle.attention_decode(Qh[i, l], Kh[l, :n], Vh[l, :n], H, kvh, hd, n, scale)
                g = Oh[i, l].astype(np.float64).reshape(H, hd)
                w = want.astype(np.float64).reshape(H, hd)
                worst = max(worst, float((np.abs(g - w).max(axis=1) / np.abs(w).max(axis=1)).max()))
        parity = {"sampled_steps": [0, ND // 2, ND - 1], "max_rel_err": worst, "tol": 1e-5,
                  "pass": bool(worst <= 1e-5)}
    cpu = None
    if not args.no_cpu_baseline:
        # the whole case: the reference's decode loop on one core, then with
        # the q-heads split over every host core the process may use
        Kh, Vh, Qh = K.cpu().numpy(), V.cpu().numpy(), Q.cpu().numpy()

        def whole(threads):
            t0 = time.perf_counter()
            for i in range(ND):
                n = T0 + i + 1
                for l in range(layers):
                    oracle.attention_decode(Qh[i, l], Kh[l, :n], Vh[l, :n], H, kvh, hd, n, scale,
                                            threads=threads)
            el = time.perf_counter() - t0
            return {"value": round(ND / el, 2), "unit": "tokens/s", "cores": threads,
                    "kind": "port",
                    "sample": "the whole case (128 decode tokens x 22 layers, 129..256 tokens of "
                              "context) on %d thread%s: %.2f s"
                              % (threads, "" if threads == 1 else "s", el)}

        one = whole(1)
        cpu = whole(oracle.host_threads())
        cpu["one_thread"] = one
    res = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg["workload"], "layers": layers, "q_heads": H, "kv_heads": kvh,
                   "head_dim": hd, "kv_dtype": "f32", "page_tokens": P, "batch": 1,
                   "prompt": T0, "decode": ND},
        "tokens_per_s": round(tok_s, 1),
        "us_per_token": round(ms_step * 1e3 / ND, 2),
        "launch": launch,
        "eager_tokens_per_s": round(ND / (ms_eager * 1e-3), 1),
        "hbm_frac_of_peak": round(gbs / HBM_PEAK_GBS, 5),
        "roofline": None,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    pool.close()
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default=None, choices=sorted(CONFIGS),
                    help="one configuration (default: llama8b_b256_8k, followed by the other "
                         "configurations of the baseline, reported under other_configs)")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-parity", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="tinyllama_b1: time the eager calls instead of one HIP graph of the step")
    ap.add_argument("--decode-kernel", type=int, default=-1, choices=[-1, 0, 1],
                    help="-1 automatic, 0 vector ALU, 1 matrix core")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run one device copy of this many MiB (counter calibration)")
    ap.add_argument("--no-suite", action="store_true",
                    help="without --config: time llama8b_b256_8k only, not the other configurations")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the paged decode path runs on a single MI355X "
              "(--gpus %d is not supported; the kernels shard by sequence or kv head with no "
              "exchange, which one GPU's share shows)" % args.gpus,
              file=sys.stderr)
        sys.exit(2)

    import importlib
    import torch
    gi = importlib.import_module("go-infer_amd")
    gi.lib()
    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    suite = args.config is None and not args.no_suite
    if args.config is None:
        args.config = DEFAULT_CONFIG
    res = run_config(args, gi, torch, dev, args.config)
    if suite:
        res["other_configs"] = run_suite(args, gi, torch, dev)
    print(json.dumps(res), flush=True)


# Configurations the default run times after the headline (config C), so that
# every workload of the baseline is measured by the same invocation: the
# reference's CPU-runnable case (A), the ragged batch (B), the 70B long-context
# batch (D) and the q8_0 chunked prefill (E).
DEFAULT_CONFIG = "llama8b_b256_8k"
SUITE = (("A", "tinyllama_b1"), ("B", "llama8b_b32"), ("D", "llama70b_b8"), ("E", "llama8b_q8_prefill"),
         ("C_q8_0", "llama8b_b256_8k_q8"), ("C_q4_0", "llama8b_b256_8k_q4"))


def run_config(args, gi, torch, dev, name):
    cfg = CONFIGS[name]
    if cfg.get("fork"):
        return run_fork(args, gi, torch, dev, cfg)
    if cfg.get("driver"):
        return run_driver(args, gi, torch, dev, cfg)
    if cfg.get("wtype"):
        return run_oproj(args, gi, torch, dev, cfg)
    if cfg.get("tiny"):
        return run_tinyllama(args, gi, torch, dev, cfg)
    if cfg.get("prefill"):
        return run_prefill(args, gi, torch, dev, cfg)
    return run_decode(args, gi, torch, dev, cfg, name)


def run_suite(args, gi, torch, dev):
    """The SUITE configurations, each timed over at most 10 steps after 2
    warm-ups, with its parity sample and without its CPU baseline; a summary
    of each result line (or the error it raised)."""
    out = {}
    for letter, name in SUITE:
        sub = argparse.Namespace(**vars(args))
        sub.config = name
        sub.steps = min(args.steps, 10)
        sub.warmup = min(args.warmup, 2)
        sub.no_cpu_baseline = True
        torch.cuda.empty_cache()
        log("-- config %s (%s)" % (letter, name))
        try:
            r = run_config(sub, gi, torch, dev, name)
        except Exception as e:  # one configuration's failure leaves the others' results
            out[letter] = {"config": name, "error": "%s: %s" % (type(e).__name__, e)}
            continue
        roof = r.get("roofline") or {}
        par = r.get("parity") or {}
        out[letter] = {
            "config": name, "workload": r["config"]["workload"], "value": r["value"], "unit": r["unit"],
            "ms_per_step": r["ms_per_step"], "steps": r["steps"], "warmup": r["warmup"],
            "tokens_per_s": r.get("tokens_per_s"),
            "roofline": {k: roof.get(k) for k in ("bound", "achieved", "peak", "unit", "frac", "traffic",
                                                 "traffic_source", "kernel", "launch_ms") if k in roof} or None,
            "parity": {k: par.get(k) for k in ("max_rel_err", "tol", "pass") if k in par} or None,
        }
        for k in ("step_entry_point", "token_store", "two_calls"):
            if k in r:
                out[letter][k] = r[k]
    return out


def run_decode(args, gi, torch, dev, cfg, name):
    H, kvh, hd, P, layers = (cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"],
                             cfg["page_tokens"], cfg["layers"])
    kv_dim = kvh * hd
    lens = seq_lengths(cfg, args.seed)
    batch = len(lens)

    t_setup = time.perf_counter()
    mgr, pages, bt = build_tables(gi, cfg, lens, args.seed)
    log("tables built: %d pages, max_blocks %d (%.1f s)" % (pages, bt.shape[1],
                                                           time.perf_counter() - t_setup))
    stream = torch.cuda.Stream(dev)
    torch.cuda.set_stream(stream)
    kv_dtype = cfg.get("kv_dtype", "f16")
    pool = gi.PagedKVCache(layers, kvh, hd, P, pages, kv_type_of(gi, kv_dtype), stream=stream)
    pool.set_decode_kernel(args.decode_kernel)
    log("pool: %.1f GiB" % (pool.page_bytes()[1] / 2**30))
    fill_pool(torch, pool, cfg, lens, bt, dev, args.seed)
    log("pool filled (%.1f s)" % (time.perf_counter() - t_setup))

    bt_d = torch.from_numpy(bt).to(dev)
    sl_d = torch.from_numpy(lens.astype(np.int32)).to(dev)
    max_len = int(lens.max())
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 1)
    q = torch.randn((layers, batch, H * hd), generator=gen, device=dev)
    kn = torch.randn((layers, batch, kv_dim), generator=gen, device=dev)
    vn = torch.randn((layers, batch, kv_dim), generator=gen, device=dev)
    out = torch.empty((layers, batch, H * hd), device=dev)
    scale = gi.attn_scale(hd)
    rope = cfg.get("rope_theta")
    if rope:
        pool.SetRoPE(rope, 0, max_len)

    # The calls of one step, checked and converted once (Prepare), so that the
    # host time per call is the C ABI's own, as for a compiled caller:
    # - the product's decode step per layer (gi_paged_decode_step, or
    #   gi_paged_rope_decode_step): one launch where the grid fits the CUs
    #   once, else an append launch and the attention launch;
    # - the two-call form: the append (gi_paged_append_at_len, with RoPE
    #   gi_paged_rope_append_at_len), then gi_paged_decode_attention.
    # q is turned in place at position seq_lens-1 when RoPE is on.  The
    # kernels' durations come from runs of each kind of launch alone, back to
    # back with events only at the ends (an event pair around every launch
    # adds its own few microseconds, which short launches would count).
    prod, app, att = [], [], []
    for l in range(layers):
        if rope:
            prod.append(pool.Prepare("RoPEDecodeStep", out[l], q[l], kn[l], vn[l], l, bt_d, sl_d, H,
                                     scale, max_len))
            app.append(pool.Prepare("RoPEWriteAtLen", l, bt_d, sl_d, q[l], kn[l], vn[l]))
        else:
            prod.append(pool.Prepare("DecodeStep", out[l], q[l], kn[l], vn[l], l, bt_d, sl_d, H, scale,
                                     max_len))
            app.append(pool.Prepare("WriteAtLen", l, bt_d, sl_d, kn[l], vn[l]))
        att.append(pool.Prepare("AttentionGQA", out[l], q[l], l, bt_d, sl_d, H, scale, max_len))

    def step_product():
        for f in prod:
            f()

    def step_two_calls():
        for l in range(layers):
            app[l]()
            att[l]()

    def attention_only():
        for f in att:
            f()

    def append_only():
        for f in app:
            f()

    def timed(fn):
        """ms per step of fn over args.steps steps: events only around the
        whole run, none between the launches."""
        pool.synchronize()
        torch.cuda.synchronize()
        s0 = torch.cuda.Event(enable_timing=True)
        s1 = torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        s0.record(stream)
        for _ in range(args.steps):
            fn()
        s1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - w0
        pool.synchronize()
        return s0.elapsed_time(s1) / args.steps, wall * 1e3 / args.steps

    for _ in range(args.warmup):
        step_product()
        step_two_calls()
    ms_step, wall_step = timed(step_product)
    ms_two, _ = timed(step_two_calls)
    # appends first: with RoPE each append turns q in place again, and the
    # outputs the parity sample checks are the last attention run's
    app_ms = timed(append_only)[0] / layers
    attn_ms = timed(attention_only)[0] / layers
    attn_bytes, app_bytes = step_bytes(cfg, lens)
    tot_gbs = (attn_bytes + app_bytes) / (ms_step * 1e-3) / 1e9
    attn_gbs = (attn_bytes / layers) / (attn_ms * 1e-3) / 1e9
    tok_s = batch / (ms_step * 1e-3)
    fused = bool(pool.decode_step_fuses(batch, H, max_len))
    log("step %.3f ms (wall %.3f ms; token store %s), two calls %.3f ms, attention kernel %.3f ms/launch" %
        (ms_step, wall_step, "in the decode launch" if fused else "by an append launch", ms_two, attn_ms))

    if args.calibrate_copy:
        n = args.calibrate_copy * 2**20 // 4
        a = torch.empty(n, dtype=torch.float32, device=dev).fill_(1.0)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    parity = None
    if not args.no_parity:
        import oracle
        rng = np.random.default_rng(args.seed + 7)
        worst = 0.0
        checked = []
        for _ in range(2):
            i, l = int(rng.integers(batch)), int(rng.integers(layers))
            n = int(lens[i])
            kw, vw = pool.Get(l, bt_d[i], n, widen=True)
            pool.synchronize()
            want = oracle.attention_decode(q[l, i].cpu().numpy(), kw.cpu().numpy(),
                                           vw.cpu().numpy(), H, kvh, hd, n, scale)
            got = out[l, i].cpu().numpy().astype(np.float64).reshape(H, hd)
            w = want.astype(np.float64).reshape(H, hd)
            err = (np.abs(got - w).max(axis=1) / np.abs(w).max(axis=1)).max()
            worst = max(worst, float(err))
            checked.append([i, l])
        parity = {"sampled_seq_layer": checked, "max_rel_err": worst, "tol": 1e-3,
                  "pass": bool(worst <= 1e-3)}

    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        cpu = cpu_baseline(oracle, cfg)

    kind = pool.decode_kernel(H)
    if kind == 1:
        kname = {"f16": "attn_mfma_f16<%d>" % hd, "f32": "attn_mfma_f32<%d>" % hd}.get(
            kv_dtype, "attn_mfma_q<%d,%d>" % (kv_type_of(gi, kv_dtype), hd))
    else:
        kname = "attn_valu<%d,%d,%d>" % (kv_type_of(gi, kv_dtype), hd, H // kvh)
    traffic = profiled_traffic(kname, name)
    res = {
        "metric": METRIC,
        "value": round(tot_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"f32": "f32", "f16": "f16"}.get(kv_dtype, "f32 (%s pages)" % kv_dtype),
        "data": "synthetic",
        "config": {"workload": cfg["workload"], "layers": layers, "q_heads": H,
                   "kv_heads": kvh, "head_dim": hd, "kv_dtype": kv_dtype, "page_tokens": P,
                   "batch": batch, "context": cfg["context"], "pool_pages": pages,
                   "fragmented_pool": cfg["frag"], "rope_theta": rope},
        "hbm_frac_of_peak": round(tot_gbs / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(tok_s, 1),
        "step_entry_point": "gi_paged_rope_decode_step" if rope else "gi_paged_decode_step",
        "token_store": "in the decode launch" if fused else "append launch",
        "two_calls": {"entry_points": ["gi_paged_rope_append_at_len" if rope else "gi_paged_append_at_len",
                                       "gi_paged_decode_attention"],
                      "ms_per_step": round(ms_two, 4),
                      "value": round((attn_bytes + app_bytes) / (ms_two * 1e-3) / 1e9, 2),
                      "tokens_per_s": round(batch / (ms_two * 1e-3), 1)},
        "decode_kernel": ["vector-alu", "matrix-core"][kind],
        "append_kernel": append_kernel_name(gi, kv_dtype, rope),
        "append_ms_per_launch": round(app_ms, 4),
        "append_gbs": round((app_bytes / layers) / (app_ms * 1e-3) / 1e9, 1),
        "roofline": {"bound": "hbm", "achieved": round(attn_gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic[0] if traffic else None,
                     "traffic_source": traffic[1] if traffic else None,
                     "kernel": kname,
                     "launch_ms": round(attn_ms, 4),
                     "bytes_per_launch": attn_bytes // layers},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    pool.close()
    return res


if __name__ == "__main__":
    main()
