"""GPU parity at the full sizes of the measured workloads, one layer each.

  C  Llama-3-8B KV shape (32 q / 8 kv heads, head_dim 128), fp16 pages of 16
     tokens, batch 256 x 8192 tokens, pool fragmented exactly as bench.py
     builds it (shuffled free list, 10 % of the sequences freed and
     allocated again).  Tokens 0..8190 are written, then one decode step
     appends token 8191 and attends over all 8192 (forward.go:236-267).
  D  Llama-3-70B KV shape (64 q / 8 kv heads), fp16 pages of 32 tokens,
     batch 8 x 32768: the split of each sequence over several work items
     and their merge, every sequence checked.
  E  Llama-3-8B KV shape over Q8_0 pages, inputs N(0,1) with 1 % outliers
     at +-8 sigma: a 4096-token prefill of batch 4 in 512-token chunks,
     each chunk appended with on-the-fly quantisation, then causal
     attention over the context so far (forward.go:527-577).

Inputs are generated on the device; the oracle is fed the stored bits
gathered back from the pool (so the attention tolerance covers only the
reduction order and exp), and the stored bytes of whole sequences are
compared bit for bit with the oracle's store of the same float32 inputs.
Tolerance: max |gpu - oracle| <= 1e-3 * max |oracle| per (query, head) row.
"""
import numpy as np
import pytest

import bench
from gpu_util import rel_err_rows

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(*a):
    print(*a, flush=True)


def outliers(torch, t, gen):
    """N(0,1) values with 1 % of the entries at +-8 sigma."""
    m = torch.rand(t.shape, generator=gen, device=t.device) < 0.01
    sgn = torch.where(torch.rand(t.shape, generator=gen, device=t.device) < 0.5, -8.0, 8.0)
    return torch.where(m, sgn, t)


def fill_decode_pool(torch, gi, pool, bt, lens, P, kv_dim, dev, seed, keep, per_seq_tokens):
    """Writes tokens [0, per_seq_tokens) of every sequence through the append
    path, 64 sequences at a time; returns the float32 inputs (host) of the
    sequences in keep."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    kept = {}
    B = len(lens)
    step = 64
    for s0 in range(0, B, step):
        s1 = min(B, s0 + step)
        n = per_seq_tokens
        ids = np.concatenate([np.repeat(bt[i, :(n + P - 1) // P], P)[:n] for i in range(s0, s1)])
        slots = np.tile(np.arange(n, dtype=np.int32) % P, s1 - s0)
        k = torch.randn(((s1 - s0) * n, kv_dim), generator=gen, device=dev)
        v = torch.randn(((s1 - s0) * n, kv_dim), generator=gen, device=dev)
        pool.Write(0, torch.from_numpy(ids.astype(np.int32)).to(dev),
                   torch.from_numpy(slots).to(dev), k, v)
        for i in range(s0, s1):
            if i in keep:
                a = (i - s0) * n
                kept[i] = (k[a:a + n].cpu().numpy(), v[a:a + n].cpu().numpy())
        del k, v
    pool.synchronize()
    return kept


def check_decode(torch, gi, oracle, pool, bt_d, lens, q, out, kvh, hd, H, scale, sample, threads):
    o = out.cpu().numpy()
    assert np.isfinite(o).all(), "non-finite attention output"
    worst = 0.0
    for i in sample:
        n = int(lens[i])
        ks, vs = pool.Get(0, bt_d[i], n)
        pool.synchronize()
        kw = oracle.widen(pool.kv_type, kvh * hd, ks.cpu().numpy())
        vw = oracle.widen(pool.kv_type, kvh * hd, vs.cpu().numpy())
        want = oracle.attention_decode(q[i], kw, vw, H, kvh, hd, n, scale, threads=threads)
        worst = max(worst, float(rel_err_rows(o[i], want, H, hd).max()))
    return worst


@pytest.mark.parametrize("kv_name", ["KV_F16", "KV_Q8_0", "KV_Q4_0"], ids=["f16", "q8_0", "q4_0"])
def test_config_c_full_shape(gi, oracle, dev, kv_name):
    """The headline shape at full size (256 sequences of 8192 tokens on a
    fragmented pool), over fp16 pages and over the quantised pages that the
    bench also reports: the decode step's stored bytes of whole sequences
    equal the oracle's, and 16 sampled sequences' outputs match it."""
    import torch
    kv_type = getattr(gi, kv_name)
    cfg = bench.CONFIGS["llama8b_b256_8k"]
    H, kvh, hd, P = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"], cfg["page_tokens"]
    kv_dim = kvh * hd
    seed = 1234
    lens = bench.seq_lengths(cfg, seed)
    B, L = len(lens), int(lens[0])
    assert B == 256 and L == 8192 and cfg["frag"]
    mgr, pages, bt = bench.build_tables(gi, cfg, lens, seed)
    say("C: tables built, %d pages, max_blocks %d" % (pages, bt.shape[1]))
    pool = gi.PagedKVCache(1, kvh, hd, P, pages, kv_type)
    rng = np.random.default_rng(seed + 3)
    whole = sorted(int(x) for x in rng.choice(B, size=8, replace=False))
    kept = fill_decode_pool(torch, gi, pool, bt, lens, P, kv_dim, dev, seed, set(whole), L - 1)
    say("C: pool filled with tokens 0..%d" % (L - 2))
    bt_d = torch.from_numpy(bt).to(dev)
    sl = torch.from_numpy(lens.astype(np.int32)).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 1)
    qd = torch.randn((B, H * hd), generator=gen, device=dev)
    kn = torch.randn((B, kv_dim), generator=gen, device=dev)
    vn = torch.randn((B, kv_dim), generator=gen, device=dev)
    out = torch.full((B, H * hd), float("nan"), device=dev)
    scale = gi.attn_scale(hd)
    pool.DecodeStep(out, qd, kn, vn, 0, bt_d, sl, H, scale)
    pool.synchronize()
    say("C: decode step done (kernel %d)" % pool.decode_kernel(H))
    # append/gather bit-exact on whole sequences, the appended token included
    kh, vh = kn.cpu().numpy(), vn.cpu().numpy()
    for i in whole:
        k = np.concatenate([kept[i][0], kh[i:i + 1]])
        v = np.concatenate([kept[i][1], vh[i:i + 1]])
        ks, vs = pool.Get(0, bt_d[i], L)
        pool.synchronize()
        assert np.array_equal(ks.cpu().numpy(), oracle.store_vectors(kv_type, k)), i
        assert np.array_equal(vs.cpu().numpy(), oracle.store_vectors(kv_type, v)), i
    say("C: stored bytes of sequences %s equal the oracle's" % whole)
    sample = sorted(set(whole) | {int(x) for x in rng.choice(B, size=12, replace=False)} | {0, B - 1})
    assert len(sample) >= 16
    worst = check_decode(torch, gi, oracle, pool, bt_d, lens, qd.cpu().numpy(), out, kvh, hd, H,
                         scale, sample, oracle.host_threads())
    say("C: %d sequences vs the oracle, max rel err %.2e" % (len(sample), worst))
    assert worst <= TOL
    pool.close()
    torch.cuda.empty_cache()


def test_config_d_full_shape(gi, oracle, dev):
    import torch
    cfg = bench.CONFIGS["llama70b_b8"]
    H, kvh, hd, P = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"], cfg["page_tokens"]
    kv_dim = kvh * hd
    seed = 1234
    lens = bench.seq_lengths(cfg, seed)
    B, L = len(lens), int(lens[0])
    assert B == 8 and L == 32768 and P == 32
    mgr, pages, bt = bench.build_tables(gi, cfg, lens, seed)
    pool = gi.PagedKVCache(1, kvh, hd, P, pages, gi.KV_F16)
    kept = fill_decode_pool(torch, gi, pool, bt, lens, P, kv_dim, dev, seed, {3}, L - 1)
    say("D: pool filled, %d pages" % pages)
    bt_d = torch.from_numpy(bt).to(dev)
    sl = torch.from_numpy(lens.astype(np.int32)).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 1)
    qd = torch.randn((B, H * hd), generator=gen, device=dev)
    kn = torch.randn((B, kv_dim), generator=gen, device=dev)
    vn = torch.randn((B, kv_dim), generator=gen, device=dev)
    out = torch.full((B, H * hd), float("nan"), device=dev)
    scale = gi.attn_scale(hd)
    pool.DecodeStep(out, qd, kn, vn, 0, bt_d, sl, H, scale)
    pool.synchronize()
    ks, _ = pool.Get(0, bt_d[3], L)
    pool.synchronize()
    k = np.concatenate([kept[3][0], kn[3:4].cpu().numpy()])
    assert np.array_equal(ks.cpu().numpy(), oracle.store_vectors(gi.KV_F16, k))
    worst = check_decode(torch, gi, oracle, pool, bt_d, lens, qd.cpu().numpy(), out, kvh, hd, H,
                         scale, range(B), oracle.host_threads())
    say("D: all %d sequences vs the oracle, max rel err %.2e" % (B, worst))
    assert worst <= TOL
    pool.close()
    torch.cuda.empty_cache()


def test_config_e_full_shape(gi, oracle, dev):
    import torch
    cfg = bench.CONFIGS["llama8b_q8_prefill"]
    H, kvh, hd, P = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"], cfg["page_tokens"]
    kv_dim = kvh * hd
    B, Ltot, C = cfg["batch"], int(cfg["context"]), cfg["chunk"]
    seed = 1234
    lens = np.full(B, Ltot, np.int64)
    mgr, pages, bt = bench.build_tables(gi, cfg, lens, seed)
    pool = gi.PagedKVCache(1, kvh, hd, P, pages, gi.KV_Q8_0)
    bt_d = torch.from_numpy(bt).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    scale = gi.attn_scale(hd)
    nch = Ltot // C
    ids = np.stack([np.repeat(bt[i], P)[:Ltot] for i in range(B)])
    slots = np.tile(np.arange(Ltot, dtype=np.int32) % P, (B, 1))
    keep_k, keep_v, outs, qs = [], [], {}, {}
    sampled = {0: [0], 3: [1], nch - 1: list(range(B))}   # chunk -> sequences checked
    for ci in range(nch):
        cid = torch.from_numpy(np.ascontiguousarray(ids[:, ci * C:(ci + 1) * C]).reshape(-1)).to(dev)
        csl = torch.from_numpy(np.ascontiguousarray(slots[:, ci * C:(ci + 1) * C]).reshape(-1)).to(dev)
        k = outliers(torch, torch.randn((B * C, kv_dim), generator=gen, device=dev), gen)
        v = outliers(torch, torch.randn((B * C, kv_dim), generator=gen, device=dev), gen)
        q = outliers(torch, torch.randn((B, C, H * hd), generator=gen, device=dev), gen)
        pool.Write(0, cid, csl, k, v)
        keep_k.append(k[2 * C:3 * C].cpu().numpy())   # sequence 2's float32 inputs
        keep_v.append(v[2 * C:3 * C].cpu().numpy())
        out = torch.full((B, C, H * hd), float("nan"), device=dev)
        sp = torch.full((B,), ci * C, dtype=torch.int32, device=dev)
        pool.AttentionGQABatch(out, q, 0, bt_d, sp, H, scale, C)
        if ci in sampled:
            outs[ci], qs[ci] = out.cpu().numpy(), q.cpu().numpy()
        del k, v, q, out
    pool.synchronize()
    say("E: prefill of %d chunks done (4096 tokens, batch %d)" % (nch, B))
    # Q8_0 quantisation bit-exact over a whole sequence
    ks, vs = pool.Get(0, bt_d[2], Ltot)
    pool.synchronize()
    assert np.array_equal(ks.cpu().numpy(), oracle.store_vectors(gi.KV_Q8_0, np.concatenate(keep_k)))
    assert np.array_equal(vs.cpu().numpy(), oracle.store_vectors(gi.KV_Q8_0, np.concatenate(keep_v)))
    say("E: stored Q8_0 blocks of sequence 2 equal the oracle's")
    worst = 0.0
    threads = oracle.host_threads()
    for ci, seqs in sampled.items():
        assert np.isfinite(outs[ci]).all(), ci
        for i in seqs:
            n = (ci + 1) * C
            ks, vs = pool.Get(0, bt_d[i], n)
            pool.synchronize()
            kw = oracle.widen(gi.KV_Q8_0, kv_dim, ks.cpu().numpy())
            vw = oracle.widen(gi.KV_Q8_0, kv_dim, vs.cpu().numpy())
            want = oracle.attention_prefill(qs[ci][i], kw, vw, H, kvh, hd, ci * C, C, 1 << 30, scale,
                                            threads=threads)
            e = float(rel_err_rows(outs[ci][i], want, H, hd).max())
            worst = max(worst, e)
            say("E: chunk %d sequence %d max rel err %.2e" % (ci, i, e))
    assert worst <= TOL
    pool.close()
    torch.cuda.empty_cache()
