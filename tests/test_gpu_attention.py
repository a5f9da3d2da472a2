"""GPU parity of paged attention against the oracle.

Decode follows pkg/engine/forward.go:242-267, chunked prefill
forward.go:547-577; the oracle is fed the same stored K/V bits (f32, the
truncated halves, or Q8_0 blocks -- checked bit-exact by test_gpu_kv.py), so
the tolerance only covers reduction order, the online softmax and exp.

Tolerance (relative, per (query, head) row): max|gpu - oracle| <= tol *
max|oracle|, with tol = 1e-5 for f32 KV and 1e-3 for f16 / q8_0 / q4_0 KV."""
import numpy as np
import pytest

from gpu_util import Populated, rel_err_rows, seeded

pytestmark = pytest.mark.gpu

TOL = {0: 1e-5, 1: 1e-3, 2: 1e-3, 3: 1e-3}


def oracle_decode(oracle, pop, layer, q, H, lens, scale):
    out = np.zeros((len(lens), H * pop.hd), np.float32)
    for i, n in enumerate(lens):
        if n == 0:
            continue
        ks, vs = pop.stored(layer, i)
        kw = oracle.widen(pop.kv_type, pop.kv_dim, ks[:n])
        vw = oracle.widen(pop.kv_type, pop.kv_dim, vs[:n])
        out[i] = oracle.attention_decode(q[i], kw, vw, H, pop.kvh, pop.hd, n, scale)
    return out


def kernels_for(pool, H):
    """Every decode kernel that can serve this pool: the vector-ALU one
    always, the matrix-core one where supported (pages of 16-token
    multiples, head_dim 64 or 128; f32 and quantised pages with groups of 1,
    2, 4 or 8)."""
    pool.set_decode_kernel(1)
    ks = [0, 1] if pool.decode_kernel(H) == 1 else [0]
    pool.set_decode_kernel(-1)
    return ks


def run_decode(gi, oracle, dev, kv_type, H, kvh, hd, P, lens, layers=1, seed=1, max_seq_len=None):
    import torch
    pop = Populated(gi, dev, kv_type, layers, kvh, hd, P, lens, seed=seed)
    bt = pop.block_tables()
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    scale = oracle.attn_scale(hd)
    worst = {}
    for l in range(layers):
        qd, q = seeded((len(lens), H * hd), seed * 31 + l, dev)
        want = oracle_decode(oracle, pop, l, q, H, lens, scale)
        for kern in kernels_for(pop.pool, H):
            pop.pool.set_decode_kernel(kern)
            out = torch.full_like(qd, float("nan"))
            pop.pool.AttentionGQA(out, qd, l, bt, sl, H, scale, max_seq_len)
            pop.pool.synchronize()
            err = rel_err_rows(out.cpu().numpy(), want, H, hd)
            worst[kern] = max(worst.get(kern, 0.0), float(err.max()))
        pop.pool.set_decode_kernel(-1)
    print("decode max rel err by kernel:", worst)
    assert max(worst.values()) <= TOL[kv_type], worst
    return pop, worst


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
def test_decode_small_shapes(gi, oracle, dev, kv_type):
    # ragged lengths including 1, page edges and a multi-split sequence
    for (H, kvh, hd, P) in [(32, 4, 64, 16), (32, 8, 128, 16), (64, 8, 128, 32), (8, 8, 128, 16),
                            (16, 8, 64, 16), (32, 8, 64, 32), (32, 8, 128, 64)]:
        run_decode(gi, oracle, dev, kv_type, H, kvh, hd, P, [1, P, P + 1, 37, 300, 1500],
                   layers=2, seed=3 + kv_type)


def test_decode_tinyllama_prompt_then_128_steps(gi, oracle, dev):
    """TinyLlama KV path (22 layers, 32 q / 4 kv heads, hd 64, f32 KV, page
    16, batch 1): 128-token prompt appended, then 128 decode steps, each
    appending its token then attending over the whole context, every layer
    checked against the oracle."""
    import torch
    H, kvh, hd, P, layers = 32, 4, 64, 16, 22
    kv_dim = kvh * hd
    total = 256
    pages = total // P
    mgr = gi.PagedKVManager(layers, kv_dim, pages, P)   # pages allocated in order (LIFO)
    pool = gi.PagedKVCache(layers, kvh, hd, P, pages, 0)
    sid = mgr.AllocateSequence()
    ids, slots = mgr.AppendTokens(sid, 128)
    K = {l: oracle.normal(1000 + l, (total, kv_dim)) for l in range(layers)}
    V = {l: oracle.normal(2000 + l, (total, kv_dim)) for l in range(layers)}
    for l in range(layers):
        pool.Write(l, torch.from_numpy(ids).to(dev), torch.from_numpy(slots).to(dev),
                   torch.from_numpy(K[l][:128].copy()).to(dev),
                   torch.from_numpy(V[l][:128].copy()).to(dev))
    scale = oracle.attn_scale(hd)
    worst = 0.0
    for step in range(128):
        n = 129 + step
        mgr.AppendToken(sid)
        bt = torch.tensor([mgr.Tables[sid].BlockIDs], dtype=torch.int32, device=dev)
        sl = torch.tensor([n], dtype=torch.int32, device=dev)
        for l in range(layers):
            q = oracle.normal(3000 + 100 * step + l, (1, H * hd))
            out = torch.empty((1, H * hd), dtype=torch.float32, device=dev)
            pool.DecodeStep(out, torch.from_numpy(q).to(dev),
                            torch.from_numpy(K[l][n - 1:n].copy()).to(dev),
                            torch.from_numpy(V[l][n - 1:n].copy()).to(dev), l, bt, sl, H, scale)
            want = oracle.attention_decode(q[0], K[l][:n], V[l][:n], H, kvh, hd, n, scale)
            err = rel_err_rows(out.cpu().numpy(), want, H, hd)
            worst = max(worst, float(err.max()))
    pool.synchronize()
    assert worst <= 1e-5, worst


def test_decode_llama8b_batch32_random_pool(gi, oracle, dev):
    """Llama-3-8B KV shape (32 q / 8 kv heads, hd 128, fp16, page 16), batch
    32, per-sequence context U[512, 4096], block tables a random permutation
    of a shared pool; two layers."""
    rng = np.random.default_rng(2024)
    lens = [int(x) for x in rng.integers(512, 4097, size=32)]
    run_decode(gi, oracle, dev, 1, 32, 8, 128, 16, lens, layers=2, seed=8)


def test_decode_llama70b_long_context_split(gi, oracle, dev):
    """Llama-3-70B KV shape (64 q / 8 kv heads, hd 128, fp16, page 32), two
    sequences at 32768 context: the split-K partitions and their merge."""
    run_decode(gi, oracle, dev, 1, 64, 8, 128, 32, [32768, 20001], layers=1, seed=9)


def test_decode_empty_and_short(gi, oracle, dev):
    import torch
    pop = Populated(gi, dev, 1, 1, 8, 128, 16, [0, 1, 2], seed=4)
    bt = pop.block_tables()
    sl = torch.tensor([0, 1, 2], dtype=torch.int32, device=dev)
    qd, q = seeded((3, 32 * 128), 5, dev)
    scale = oracle.attn_scale(128)
    ks, vs = pop.stored(0, 1)
    v1 = oracle.widen(1, 1024, vs)[0]
    want = oracle_decode(oracle, pop, 0, q, 32, [0, 1, 2], scale)
    for kern in kernels_for(pop.pool, 32):
        pop.pool.set_decode_kernel(kern)
        out = torch.full_like(qd, float("nan"))
        pop.pool.AttentionGQA(out, qd, 0, bt, sl, 32, scale)
        pop.pool.synchronize()
        o = out.cpu().numpy()
        assert not o[0].any()                               # empty context -> zeros
        # one token: softmax weight 1, output = V of that token for every head
        for h in range(32):
            np.testing.assert_allclose(o[1, h * 128:(h + 1) * 128],
                                       v1[(h // 4) * 128:(h // 4 + 1) * 128], rtol=1e-6, atol=0)
        assert rel_err_rows(o[2], want[2], 32, 128).max() <= 1e-3


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
def test_decode_stale_nan_beyond_length_is_ignored(gi, oracle, dev, kv_type):
    """Slots past a sequence's length may hold anything (a freed page's old
    contents): NaN there (for quantised pages, values of 1e30 whose fp16
    block scales are Inf) must not reach the output, as the reference never
    reads past activeContext (forward.go:252, 259)."""
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    pop = Populated(gi, dev, kv_type, 1, kvh, hd, P, [40, 40], seed=12)
    # poison slots 20..39 of sequence 0 through the append path
    t = pop.table(0)
    ids = torch.from_numpy(np.repeat(t, P)[20:40].copy()).to(dev)
    slots = torch.from_numpy((np.arange(20, 40) % P).astype(np.int32)).to(dev)
    bad = float("nan") if kv_type in (0, 1) else 1e30
    nan = torch.full((20, kvh * hd), bad, device=dev)
    pop.pool.Write(0, ids, slots, nan, nan)
    bt = pop.block_tables()
    sl = torch.tensor([20, 40], dtype=torch.int32, device=dev)
    qd, q = seeded((2, H * hd), 13, dev)
    scale = oracle.attn_scale(hd)
    ks, vs = pop.stored(0, 0)
    kw, vw = oracle.widen(kv_type, 1024, ks[:20]), oracle.widen(kv_type, 1024, vs[:20])
    want = oracle.attention_decode(q[0], kw, vw, H, kvh, hd, 20, scale)
    for kern in kernels_for(pop.pool, H):
        pop.pool.set_decode_kernel(kern)
        out = torch.zeros_like(qd)
        pop.pool.AttentionGQA(out, qd, 0, bt, sl, H, scale)
        pop.pool.synchronize()
        o = out.cpu().numpy()
        assert np.isfinite(o[0]).all()
        assert rel_err_rows(o[0], want, H, hd).max() <= 1e-3


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
def test_prefill_stale_nan_beyond_context_is_ignored(gi, oracle, dev, kv_type):
    """Prefill of 12 queries at start 16 reads 28 tokens; slots 28..39 hold
    NaN (fp16) or 1e30 (quantised: Inf block scales), inside the last read
    page and beyond it.  Both kernels must ignore them (forward.go:547-577
    never reads past start + i)."""
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    pop = Populated(gi, dev, kv_type, 1, kvh, hd, P, [40], seed=17)
    t = pop.table(0)
    ids = torch.from_numpy(np.repeat(t, P)[28:40].copy()).to(dev)
    slots = torch.from_numpy((np.arange(28, 40) % P).astype(np.int32)).to(dev)
    bad = float("nan") if kv_type in (0, 1) else 1e30
    poison = torch.full((12, kvh * hd), bad, device=dev)
    pop.pool.Write(0, ids, slots, poison, poison)
    bt = pop.block_tables()
    sp = torch.tensor([16], dtype=torch.int32, device=dev)
    qd, q = seeded((1, 12, H * hd), 18, dev)
    scale = oracle.attn_scale(hd)
    ks, vs = pop.stored(0, 0)
    kw, vw = oracle.widen(kv_type, kvh * hd, ks[:28]), oracle.widen(kv_type, kvh * hd, vs[:28])
    want = oracle.attention_prefill(q[0], kw, vw, H, kvh, hd, 16, 12, 1 << 30, scale)
    tol = 1e-5 if kv_type == 0 else 1e-3
    for kern in (0, 1):
        pop.pool.set_decode_kernel(kern)
        out = torch.full_like(qd, float("nan"))
        pop.pool.AttentionGQABatch(out, qd, 0, bt, sp, H, scale, 12)
        pop.pool.synchronize()
        o = out.cpu().numpy()[0]
        assert np.isfinite(o).all(), kern
        assert rel_err_rows(o, want, H, hd).max() <= tol, kern
    pop.pool.set_decode_kernel(-1)


@pytest.mark.parametrize("kv_type", [2, 3], ids=["q8_0", "q4_0"])
def test_decode_quant_scale_spread(gi, oracle, dev, kv_type):
    """One token of every 32 (slot 29 of the block, deep inside a lane's
    8-token group) has values 200x the others, so its V block scales are
    far above the rest of the block's.  The matrix-core kernel's running
    cap must cover them: a cap taken from a subset of the scales lets that
    token's weights overflow fp16."""
    import torch
    H, kvh, hd, P, lens = 32, 8, 128, 16, [200, 64]
    kv_dim = kvh * hd
    pages = sum((n + P - 1) // P for n in lens) + 2
    mgr = gi.PagedKVManager(1, kv_dim, pages, P)
    mgr.SetFreeList(np.random.default_rng(13).permutation(pages).astype(np.int32))
    pool = gi.PagedKVCache(1, kvh, hd, P, pages, kv_type)
    tabs, ks, vs = [], [], []
    for i, n in enumerate(lens):
        sid = mgr.AllocateSequence()
        ids, slots = mgr.AppendTokens(sid, n)
        f = np.where(np.arange(n) % 32 == 29, 200.0, 1.0).astype(np.float32)[:, None]
        k = (oracle.normal(900 + i, (n, kv_dim)) * 0.2).astype(np.float32)
        v = (oracle.normal(950 + i, (n, kv_dim)) * f).astype(np.float32)
        pool.Write(0, torch.from_numpy(ids).to(dev), torch.from_numpy(slots).to(dev),
                   torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev))
        ks.append(oracle.widen(kv_type, kv_dim, oracle.store_vectors(kv_type, k)))
        vs.append(oracle.widen(kv_type, kv_dim, oracle.store_vectors(kv_type, v)))
        tabs.append(mgr.Tables[sid].BlockIDs)
    mb = max(len(t) for t in tabs)
    bt = torch.tensor([t + [0] * (mb - len(t)) for t in tabs], dtype=torch.int32, device=dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    q = oracle.normal(990, (len(lens), H * hd)).astype(np.float32)
    qd = torch.from_numpy(q).to(dev)
    scale = oracle.attn_scale(hd)
    worst = {}
    for kern in kernels_for(pool, H):
        pool.set_decode_kernel(kern)
        out = torch.full_like(qd, float("nan"))
        pool.AttentionGQA(out, qd, 0, bt, sl, H, scale)
        pool.synchronize()
        o = out.cpu().numpy()
        assert np.isfinite(o).all(), kern
        for i, n in enumerate(lens):
            want = oracle.attention_decode(q[i], ks[i], vs[i], H, kvh, hd, n, scale)
            worst[kern] = max(worst.get(kern, 0.0), float(rel_err_rows(o[i], want, H, hd).max()))
    pool.set_decode_kernel(-1)
    print("quantised scale-spread decode max rel err by kernel:", worst)
    assert max(worst.values()) <= 1e-3, worst


@pytest.mark.parametrize("H,kvh,hd", [(32, 8, 128), (32, 4, 64), (8, 8, 128)])
def test_decode_f32_wide_range(gi, oracle, dev, H, kvh, hd):
    """f32 pages whose magnitude changes by up to 10^9 from one 32-token
    block to the next (K from 1e-4 to 1e5, V from 1e-5 to 1e5, beyond fp16's
    range both ways): the matrix-core kernel's per-block power-of-two operand
    scales must keep the 1e-5 bound of the f32 path."""
    import torch
    P, lens = 16, [300, 77, 33]
    kv_dim = kvh * hd
    pages = sum((n + P - 1) // P for n in lens) + 2
    mgr = gi.PagedKVManager(1, kv_dim, pages, P)
    mgr.SetFreeList(np.random.default_rng(5).permutation(pages).astype(np.int32))
    pool = gi.PagedKVCache(1, kvh, hd, P, pages, gi.KV_F32)
    # K reaches 4e5 (beyond fp16) with q at 1e-5, so scores stay moderate
    kf = np.array([1e-4, 1.0, 3e4, 1e-2, 1e5, 0.5, 3e-3], np.float32)
    vf = np.array([1.0, 1e5, 1e-5, 3e3, 1e-3, 7.0, 2e4], np.float32)
    ks, vs, tabs = [], [], []
    for i, n in enumerate(lens):
        sid = mgr.AllocateSequence()
        ids, slots = mgr.AppendTokens(sid, n)
        blk = (np.arange(n) // 32 + i) % len(kf)
        k = (oracle.normal(300 + i, (n, kv_dim)) * kf[blk][:, None]).astype(np.float32)
        v = (oracle.normal(400 + i, (n, kv_dim)) * vf[blk][:, None]).astype(np.float32)
        pool.Write(0, torch.from_numpy(ids).to(dev), torch.from_numpy(slots).to(dev),
                   torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev))
        ks.append(k)
        vs.append(v)
        tabs.append(mgr.Tables[sid].BlockIDs)
    mb = max(len(t) for t in tabs)
    bt = torch.tensor([t + [0] * (mb - len(t)) for t in tabs], dtype=torch.int32, device=dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    q = (oracle.normal(500, (len(lens), H * hd)) * 1e-5).astype(np.float32)
    qd = torch.from_numpy(q).to(dev)
    scale = oracle.attn_scale(hd)
    kinds = kernels_for(pool, H)
    assert kinds == [0, 1], "f32 pages should have the matrix-core kernel"
    worst = {}
    for kern in kinds:
        pool.set_decode_kernel(kern)
        out = torch.full_like(qd, float("nan"))
        pool.AttentionGQA(out, qd, 0, bt, sl, H, scale)
        pool.synchronize()
        o = out.cpu().numpy()
        for i, n in enumerate(lens):
            want = oracle.attention_decode(q[i], ks[i], vs[i], H, kvh, hd, n, scale)
            worst[kern] = max(worst.get(kern, 0.0), float(rel_err_rows(o[i], want, H, hd).max()))
    pool.set_decode_kernel(-1)
    print("f32 wide-range decode max rel err by kernel:", worst)
    assert max(worst.values()) <= 1e-5, worst


def prefill_case(gi, oracle, dev, kv_type, H, kvh, hd, P, starts, chunk, seed):
    import torch
    lens = [s + chunk for s in starts]
    pop = Populated(gi, dev, kv_type, 1, kvh, hd, P, lens, seed=seed, append_chunk=chunk,
                    outliers=True)
    bt = pop.block_tables()
    sp = torch.tensor(starts, dtype=torch.int32, device=dev)
    qd, q = seeded((len(starts), chunk, H * hd), seed + 50, dev, outliers=True)
    scale = oracle.attn_scale(hd)
    wants = []
    for i, s in enumerate(starts):
        ks, vs = pop.stored(0, i)
        kw = oracle.widen(kv_type, pop.kv_dim, ks)
        vw = oracle.widen(kv_type, pop.kv_dim, vs)
        wants.append(oracle.attention_prefill(q[i], kw, vw, H, kvh, hd, s, chunk, 1 << 30, scale))
    # both attention kernels: vector ALU (0) and the matrix-core prefill (1;
    # f32 and q4_0 pages on the staged kernel only, q4_0 with head_dim 128:
    # other shapes fall back to the vector kernel)
    kinds = [0, 1]
    worst = {}
    for kern in kinds:
        pop.pool.set_decode_kernel(kern)
        out = torch.full_like(qd, float("nan"))
        pop.pool.AttentionGQABatch(out, qd, 0, bt, sp, H, scale, chunk)
        pop.pool.synchronize()
        o = out.cpu().numpy()
        for i in range(len(starts)):
            e = float(rel_err_rows(o[i], wants[i], H, hd).max())
            worst[kern] = max(worst.get(kern, 0.0), e)
    pop.pool.set_decode_kernel(-1)
    print("prefill max rel err by kernel:", worst)
    assert max(worst.values()) <= TOL[kv_type], worst


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
def test_prefill_chunk(gi, oracle, dev, kv_type):
    prefill_case(gi, oracle, dev, kv_type, 32, 8, 128, 16, [0, 100, 509], 64, seed=60 + kv_type)


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
@pytest.mark.parametrize("H,kvh,hd,P", [(8, 8, 64, 16), (16, 8, 64, 32), (64, 8, 128, 32),
                                        (32, 2, 128, 16), (16, 4, 128, 64)])
def test_prefill_shapes(gi, oracle, dev, kv_type, H, kvh, hd, P):
    """Group sizes 1, 2, 4, 8, 16, head_dim 64 and pages of 16/32/64 tokens on
    the matrix-core prefill; ragged chunk (37 queries) and start positions
    off the page grid."""
    prefill_case(gi, oracle, dev, kv_type, H, kvh, hd, P, [3, 45], 37, seed=80 + kv_type)


@pytest.mark.parametrize("hd,P,period,vcols", [(128, 16, 64, False), (64, 32, 64, False), (128, 32, 16, True),
                                                (128, 64, 24, True)],
                         ids=["hd128-p16-block", "hd64-p32-block", "hd128-p32-16tok-vcols", "hd128-p64-24tok-vcols"])
def test_prefill_f32_wide_range(gi, oracle, dev, hd, P, period, vcols):
    """f32 pages whose magnitude moves by up to 10^9 every `period` tokens
    (K 1e-4 .. 1e5 with q at 1e-5, V 1e-5 .. 1e5), and with vcols V's
    32-dimension groups also 1, 1e3, 1e-3 and 10 apart.  The kernels' operand
    scales (per 64-token block and workgroup in the staged kernel, per
    16-token group of K and 32-dimension group of V in the f32 ping-pong
    kernel) must keep the 1e-5 bound of the f32 path.  A 200-query chunk at
    start 300, batch 2."""
    import torch
    H, kvh = 16, 4
    kv_dim = kvh * hd
    starts, chunk = [300, 129], 200
    lens = [s + chunk for s in starts]
    pages = sum((n + P - 1) // P for n in lens) + 2
    mgr = gi.PagedKVManager(1, kv_dim, pages, P)
    mgr.SetFreeList(np.random.default_rng(9).permutation(pages).astype(np.int32))
    pool = gi.PagedKVCache(1, kvh, hd, P, pages, gi.KV_F32)
    kf = np.array([1e-4, 1.0, 3e4, 1e-2, 1e5, 0.5, 3e-3], np.float32)
    vf = np.array([1.0, 1e5, 1e-5, 3e3, 1e-3, 7.0, 2e4], np.float32)
    ks, vs, tabs = [], [], []
    for i, n in enumerate(lens):
        sid = mgr.AllocateSequence()
        ids, slots = mgr.AppendTokens(sid, n)
        blk = (np.arange(n) // period + i) % len(kf)
        k = (oracle.normal(600 + i, (n, kv_dim)) * kf[blk][:, None]).astype(np.float32)
        v = (oracle.normal(700 + i, (n, kv_dim)) * vf[blk][:, None]).astype(np.float32)
        if vcols:
            v *= np.array([1.0, 1e3, 1e-3, 10.0], np.float32)[(np.arange(kv_dim) % hd) // 32][None, :]
        pool.Write(0, torch.from_numpy(ids).to(dev), torch.from_numpy(slots).to(dev),
                   torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev))
        ks.append(k)
        vs.append(v)
        tabs.append(mgr.Tables[sid].BlockIDs)
    mb = max(len(t) for t in tabs)
    bt = torch.tensor([t + [0] * (mb - len(t)) for t in tabs], dtype=torch.int32, device=dev)
    sp = torch.tensor(starts, dtype=torch.int32, device=dev)
    q = (oracle.normal(800, (len(starts), chunk, H * hd)) * 1e-5).astype(np.float32)
    qd = torch.from_numpy(q).to(dev)
    scale = oracle.attn_scale(hd)
    worst = {}
    for kern in (0, 1):
        pool.set_decode_kernel(kern)
        out = torch.full_like(qd, float("nan"))
        pool.AttentionGQABatch(out, qd, 0, bt, sp, H, scale, chunk)
        pool.synchronize()
        o = out.cpu().numpy()
        for i, s0 in enumerate(starts):
            want = oracle.attention_prefill(q[i], ks[i], vs[i], H, kvh, hd, s0, chunk, 1 << 30, scale)
            worst[kern] = max(worst.get(kern, 0.0), float(rel_err_rows(o[i], want, H, hd).max()))
    pool.set_decode_kernel(-1)
    print("f32 wide-range prefill max rel err by kernel:", worst)
    assert max(worst.values()) <= 1e-5, worst


def test_prefill_q4_llama8b_chunks(gi, oracle, dev):
    """Q4_0 KV, Llama-3-8B shape, 256-token chunks: the last chunk of a
    768-token prefill, batch 2, inputs with 1 % outliers."""
    prefill_case(gi, oracle, dev, 3, 32, 8, 128, 16, [512, 256], 256, seed=75)


def test_prefill_q8_llama8b_chunks(gi, oracle, dev):
    """Llama-3-8B shape, Q8_0 KV, 512-token chunks appended with on-the-fly
    quantisation, N(0,1) inputs with 1 % outliers at +-8 sigma: the last
    chunk of a 1536-token prefill, batch 2."""
    prefill_case(gi, oracle, dev, 2, 32, 8, 128, 16, [1024, 512], 512, seed=70)


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
@pytest.mark.parametrize("P", [32, 64])
def test_prefill_llama8b_large_pages(gi, oracle, dev, kv_type, P):
    """Llama-3-8B shape over pages of 32 and 64 tokens with 256-query
    chunks, so that several tiles of 256 columns pair up in the ping-pong
    kernels (one per half of a workgroup's waves) and blocks span pages
    of every size the kernels take; starts 448 and 64, batch 2, inputs
    with 1 % outliers."""
    prefill_case(gi, oracle, dev, kv_type, 32, 8, 128, P, [448, 64], 256, seed=90 + kv_type + P)


@pytest.mark.parametrize("kv_type", [2, 3], ids=["q8_0", "q4_0"])
def test_prefill_quant_scale_spread(gi, oracle, dev, kv_type):
    """Quantised pages whose block scales move by up to 3e5 from token to
    token: K magnitudes cycle through 1e-3 .. 300 with period 5 and V
    through 1e-2 .. 200 with period 7, so every 32-dimension block of K
    and every V block row mixes tiny and huge scales.  The matrix-core
    prefill scales each k-step's product of K codes by its token's block
    scale and keeps V as exact hi + lo planes; both must hold the 1e-3
    bound.  Two sequences, 128-query chunks at starts 200 and 64."""
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    kv_dim = kvh * hd
    starts, chunk = [200, 64], 128
    lens = [s + chunk for s in starts]
    pages = sum((n + P - 1) // P for n in lens) + 2
    mgr = gi.PagedKVManager(1, kv_dim, pages, P)
    mgr.SetFreeList(np.random.default_rng(17).permutation(pages).astype(np.int32))
    pool = gi.PagedKVCache(1, kvh, hd, P, pages, kv_type)
    kf = np.array([1e-3, 1.0, 300.0, 0.05, 30.0], np.float32)
    vf = np.array([1.0, 200.0, 1e-2, 3.0, 0.2, 50.0, 0.7], np.float32)
    tabs, ks, vs = [], [], []
    for i, n in enumerate(lens):
        sid = mgr.AllocateSequence()
        ids, slots = mgr.AppendTokens(sid, n)
        t = np.arange(n)
        k = (oracle.normal(1100 + i, (n, kv_dim)) * kf[t % kf.size][:, None]).astype(np.float32)
        v = (oracle.normal(1150 + i, (n, kv_dim)) * vf[t % vf.size][:, None]).astype(np.float32)
        pool.Write(0, torch.from_numpy(ids).to(dev), torch.from_numpy(slots).to(dev),
                   torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev))
        ks.append(oracle.widen(kv_type, kv_dim, oracle.store_vectors(kv_type, k)))
        vs.append(oracle.widen(kv_type, kv_dim, oracle.store_vectors(kv_type, v)))
        tabs.append(mgr.Tables[sid].BlockIDs)
    mb = max(len(t) for t in tabs)
    bt = torch.tensor([t + [0] * (mb - len(t)) for t in tabs], dtype=torch.int32, device=dev)
    sp = torch.tensor(starts, dtype=torch.int32, device=dev)
    q = (oracle.normal(1190, (len(starts), chunk, H * hd)) * 0.1).astype(np.float32)
    qd = torch.from_numpy(q).to(dev)
    scale = oracle.attn_scale(hd)
    worst = {}
    for kern in (0, 1):
        pool.set_decode_kernel(kern)
        out = torch.full_like(qd, float("nan"))
        pool.AttentionGQABatch(out, qd, 0, bt, sp, H, scale, chunk)
        pool.synchronize()
        o = out.cpu().numpy()
        assert np.isfinite(o).all(), kern
        for i, s0 in enumerate(starts):
            want = oracle.attention_prefill(q[i], ks[i], vs[i], H, kvh, hd, s0, chunk, 1 << 30, scale)
            worst[kern] = max(worst.get(kern, 0.0), float(rel_err_rows(o[i], want, H, hd).max()))
    pool.set_decode_kernel(-1)
    print("quantised scale-spread prefill max rel err by kernel:", worst)
    assert max(worst.values()) <= 1e-3, worst


def test_decode_short_max_seq_len_attends_every_token(gi, oracle, dev):
    """max_seq_len sizes the split plan only: the last split of a sequence
    runs to its end, so a hint below the real lengths (one frozen at graph
    capture while lengths grew) still attends every token of every sequence,
    and 0 plans for the longest sequence the block tables map.  A ragged
    batch: hints 1 and 64 give one split per sequence, 2048 two splits of
    1024 tokens whose second runs on to 5000, 3000 three."""
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    lens = [1, 5000, 700, 2049, 64, 3333]
    pop = Populated(gi, dev, 1, 1, kvh, hd, P, lens, seed=21)
    bt = pop.block_tables()
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    qd, q = seeded((len(lens), H * hd), 22, dev)
    scale = oracle.attn_scale(hd)
    want = oracle_decode(oracle, pop, 0, q, H, lens, scale)
    for kern in kernels_for(pop.pool, H):
        pop.pool.set_decode_kernel(kern)
        for msl in (0, 1, 64, 2048, 3000):
            out = torch.full_like(qd, float("nan"))
            pop.pool.AttentionGQA(out, qd, 0, bt, sl, H, scale, msl)
            pop.pool.synchronize()
            err = float(rel_err_rows(out.cpu().numpy(), want, H, hd).max())
            assert err <= 1e-3, (kern, msl, err)
    pop.pool.set_decode_kernel(-1)


def test_decode_bad_lengths_are_clamped_and_reported(gi, oracle, dev):
    """A length beyond what the block table maps is clamped to the mapped
    tokens, a negative one to 0 (zero output); both are reported by
    gi_synchronize, and the other sequences are unaffected."""
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    lens = [100, 300, 50]
    pop = Populated(gi, dev, 1, 1, kvh, hd, P, lens, seed=23)
    bt = pop.block_tables()            # max_blocks = 19 pages = 304 tokens
    mapped = bt.shape[1] * P
    qd, q = seeded((len(lens), H * hd), 24, dev)
    scale = oracle.attn_scale(hd)
    want = oracle_decode(oracle, pop, 0, q, H, lens, scale)
    for kern in kernels_for(pop.pool, H):
        pop.pool.set_decode_kernel(kern)
        sl = torch.tensor([100, mapped + 500, -7], dtype=torch.int32, device=dev)
        out = torch.full_like(qd, float("nan"))
        pop.pool.AttentionGQA(out, qd, 0, bt, sl, H, scale)
        with pytest.raises(gi.GIError) as e:
            pop.pool.synchronize()
        assert e.value.code == -7, kern
        o = out.cpu().numpy()
        assert rel_err_rows(o[0], want[0], H, hd).max() <= 1e-3
        # sequence 1: every mapped token; its slots past 300 hold zeros
        ks, vs = pop.stored(0, 1)
        kw = np.zeros((mapped, kvh * hd), np.float32)
        vw = np.zeros((mapped, kvh * hd), np.float32)
        kw[:300] = oracle.widen(1, kvh * hd, ks)
        vw[:300] = oracle.widen(1, kvh * hd, vs)
        w1 = oracle.attention_decode(q[1], kw, vw, H, kvh, hd, mapped, scale)
        assert rel_err_rows(o[1], w1, H, hd).max() <= 1e-3
        assert not o[2].any()
    pop.pool.set_decode_kernel(-1)


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
def test_decode_bad_first_page_is_skipped(gi, oracle, dev, kv_type):
    """A block table whose first entry is outside the pool: that page's
    tokens are skipped (the wave that meets it first sees only masked
    scores, which must not turn into NaN), the sequence attends the rest,
    gi_synchronize reports the id, and the other sequence is unaffected."""
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    lens = [600, 300]
    pop = Populated(gi, dev, kv_type, 1, kvh, hd, P, lens, seed=25)
    bt = pop.block_tables()
    bt[0, 0] = pop.pool.num_pages + 5
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    qd, q = seeded((len(lens), H * hd), 26, dev)
    scale = oracle.attn_scale(hd)
    ks, vs = pop.stored(0, 0)
    kw = oracle.widen(kv_type, kvh * hd, ks)[P:]
    vw = oracle.widen(kv_type, kvh * hd, vs)[P:]
    want0 = oracle.attention_decode(q[0], kw, vw, H, kvh, hd, lens[0] - P, scale)
    want1 = oracle_decode(oracle, pop, 0, q, H, lens, scale)[1]
    for kern in kernels_for(pop.pool, H):
        pop.pool.set_decode_kernel(kern)
        out = torch.full_like(qd, float("nan"))
        pop.pool.AttentionGQA(out, qd, 0, bt, sl, H, scale)
        with pytest.raises(gi.GIError) as e:
            pop.pool.synchronize()
        assert e.value.code == -7, kern
        o = out.cpu().numpy()
        assert np.isfinite(o).all(), kern
        assert rel_err_rows(o[0], want0, H, hd).max() <= TOL[kv_type], kern
        assert rel_err_rows(o[1], want1, H, hd).max() <= TOL[kv_type], kern
    pop.pool.set_decode_kernel(-1)


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
def test_prefill_bad_page_is_skipped(gi, oracle, dev, kv_type):
    """A 64-query chunk at start 200 whose block table holds an id outside
    the pool for tokens 48..63 (inside every query's context): both prefill
    kernels skip that page's tokens -- the block it sits in runs the masked
    path, and its V is zeroed before the products -- report the id at
    gi_synchronize, and match the oracle over the context without those 16
    tokens (forward.go:547-577 with the page removed).  The second sequence
    of the batch is unaffected."""
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    starts, chunk = [200, 150], 64
    lens = [s + chunk for s in starts]
    pop = Populated(gi, dev, kv_type, 1, kvh, hd, P, lens, seed=31, append_chunk=chunk, outliers=True)
    bt = pop.block_tables()
    bt[0, 3] = pop.pool.num_pages + 7
    sp = torch.tensor(starts, dtype=torch.int32, device=dev)
    qd, q = seeded((len(starts), chunk, H * hd), 32, dev, outliers=True)
    scale = oracle.attn_scale(hd)
    keep = np.r_[0:3 * P, 4 * P:lens[0]]
    ks, vs = pop.stored(0, 0)
    kw = oracle.widen(kv_type, kvh * hd, ks)[keep]
    vw = oracle.widen(kv_type, kvh * hd, vs)[keep]
    want0 = oracle.attention_prefill(q[0], kw, vw, H, kvh, hd, starts[0] - P, chunk, 1 << 30, scale)
    ks, vs = pop.stored(0, 1)
    want1 = oracle.attention_prefill(q[1], oracle.widen(kv_type, kvh * hd, ks), oracle.widen(kv_type, kvh * hd, vs),
                                     H, kvh, hd, starts[1], chunk, 1 << 30, scale)
    for kern in (0, 1):
        pop.pool.set_decode_kernel(kern)
        out = torch.full_like(qd, float("nan"))
        pop.pool.AttentionGQABatch(out, qd, 0, bt, sp, H, scale, chunk)
        with pytest.raises(gi.GIError) as e:
            pop.pool.synchronize()
        assert e.value.code == -7, kern
        o = out.cpu().numpy()
        assert np.isfinite(o).all(), kern
        assert rel_err_rows(o[0], want0, H, hd).max() <= TOL[kv_type], kern
        assert rel_err_rows(o[1], want1, H, hd).max() <= TOL[kv_type], kern
    pop.pool.set_decode_kernel(-1)
