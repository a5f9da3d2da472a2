"""GPU parity of the fused RoPE + append (ApplyRoPE, pkg/math/kernels.go:
22-35, applied to q and k before the store of forward.go:228-240 / 527-545).

Bit-exact bar: the rotated q the kernel writes equals the oracle's ApplyRoPE
bit for bit, and the pages hold exactly the oracle's stored format (f32 bits,
truncated halves, Q8_0 blocks) of the oracle-rotated K and of V.  The decode
step's attention is checked against the oracle fed the same stored bits,
max|gpu - oracle| <= tol * max|oracle| per (query, head) row with tol 1e-5
(f32 KV) or 1e-3 (f16 / q8_0 / q4_0 KV)."""
import numpy as np
import pytest

from gpu_util import rel_err_rows

pytestmark = pytest.mark.gpu

TOL = {0: 1e-5, 1: 1e-3, 2: 1e-3, 3: 1e-3}
SHAPES = {
    # (q heads, kv heads, head_dim, page_tokens, rope_dim, theta)
    "tinyllama": (32, 4, 64, 16, 64, 10000.0),
    "llama8b": (32, 8, 128, 16, 128, 500000.0),
    "partial_rope": (16, 8, 128, 32, 64, 1000000.0),
}


def _setup(gi, dev, kv_type, shape, lens, max_pos, seed, slack=4):
    H, kvh, hd, P, rd, theta = SHAPES[shape]
    pages = sum((n + P - 1) // P for n in lens) + slack
    mgr = gi.PagedKVManager(1, kvh * hd, pages, P)
    mgr.SetFreeList(np.random.default_rng(seed).permutation(pages).astype(np.int32))
    pool = gi.PagedKVCache(1, kvh, hd, P, pages, kv_type)
    pool.SetRoPE(theta, rd, max_pos)
    return mgr, pool


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_rope_append_bit_exact(gi, oracle, dev, kv_type, shape):
    """Prefill form: chunks of tokens at explicit positions, fragmented
    pages, a chunk starting mid-page; q rotated out of place."""
    import torch
    H, kvh, hd, P, rd, theta = SHAPES[shape]
    kv_dim = kvh * hd
    lens = [1, P + 3, 77]
    mgr, pool = _setup(gi, dev, kv_type, shape, lens, 4096, seed=3 + kv_type)
    for i, n in enumerate(lens):
        sid = mgr.AllocateSequence()
        ids, slots = mgr.AppendTokens(sid, n)
        pos = np.arange(n, dtype=np.int32)
        q = oracle.normal(100 + i, (n, H * hd))
        k = oracle.normal(200 + i, (n, kv_dim))
        v = oracle.normal(300 + i, (n, kv_dim))
        qd = torch.from_numpy(q).to(dev)
        qo = torch.full_like(qd, float("nan"))
        step = 13
        for a in range(0, n, step):
            b = min(n, a + step)
            pool.RoPEWrite(0, torch.from_numpy(pos[a:b].copy()).to(dev),
                           torch.from_numpy(ids[a:b].copy()).to(dev),
                           torch.from_numpy(slots[a:b].copy()).to(dev),
                           qd[a:b], torch.from_numpy(k[a:b].copy()).to(dev),
                           torch.from_numpy(v[a:b].copy()).to(dev), q_out=qo[a:b])
        pool.synchronize()
        want_q = oracle.rope_heads(q, pos, H, hd, rd, theta)
        assert np.array_equal(qo.cpu().numpy().view(np.uint32), want_q.view(np.uint32)), i
        assert np.array_equal(qd.cpu().numpy(), q)                     # input untouched
        want_k = oracle.store_vectors(kv_type, oracle.rope_heads(k, pos, kvh, hd, rd, theta))
        want_v = oracle.store_vectors(kv_type, v)
        t = torch.tensor(mgr.Tables[sid].BlockIDs, dtype=torch.int32, device=dev)
        ko, vo = pool.Get(0, t, n)
        pool.synchronize()
        assert np.array_equal(ko.cpu().numpy(), want_k), i
        assert np.array_equal(vo.cpu().numpy(), want_v), i


def test_rope_in_place_and_long_positions(gi, oracle, dev):
    """q rotated in place; positions up to 131071 (theta 5e5, the Llama-3
    base); K-only call (no q)."""
    import torch
    H, kvh, hd, P, rd, theta = SHAPES["llama8b"]
    kv_dim = kvh * hd
    n = 40
    mgr, pool = _setup(gi, dev, 1, "llama8b", [n], 131072, seed=9)
    sid = mgr.AllocateSequence()
    ids, slots = mgr.AppendTokens(sid, n)
    pos = np.concatenate([np.arange(131072 - 20, 131072), np.arange(8180, 8200)]).astype(np.int32)
    q = oracle.normal(41, (n, H * hd))
    k = oracle.normal(42, (n, kv_dim))
    v = oracle.normal(43, (n, kv_dim))
    qd = torch.from_numpy(q).to(dev)
    pool.RoPEWrite(0, torch.from_numpy(pos).to(dev), torch.from_numpy(ids).to(dev),
                   torch.from_numpy(slots).to(dev), qd, torch.from_numpy(k).to(dev),
                   torch.from_numpy(v).to(dev))
    pool.synchronize()
    want_q = oracle.rope_heads(q, pos, H, hd, rd, theta)
    assert np.array_equal(qd.cpu().numpy().view(np.uint32), want_q.view(np.uint32))
    t = torch.tensor(mgr.Tables[sid].BlockIDs, dtype=torch.int32, device=dev)
    ko, _ = pool.Get(0, t, n)
    want_k = oracle.store_vectors(1, oracle.rope_heads(k, pos, kvh, hd, rd, theta))
    assert np.array_equal(ko.cpu().numpy(), want_k)
    # K only: the same tokens again without q give the same pages
    pool.RoPEWrite(0, torch.from_numpy(pos).to(dev), torch.from_numpy(ids).to(dev),
                   torch.from_numpy(slots).to(dev), None, torch.from_numpy(k).to(dev),
                   torch.from_numpy(v).to(dev))
    ko2, _ = pool.Get(0, t, n)
    pool.synchronize()
    assert np.array_equal(ko2.cpu().numpy(), want_k)


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
def test_rope_decode_step(gi, oracle, dev, kv_type):
    """forward.go:228-267 for a ragged batch: prompts appended with RoPE at
    positions 0..n-2, then one decode step appending position n-1 and
    attending over n tokens.  q is rotated in place."""
    import torch
    H, kvh, hd, P, rd, theta = SHAPES["llama8b"]
    kv_dim = kvh * hd
    lens = [1, 16, 17, 300, 1000]
    mgr, pool = _setup(gi, dev, kv_type, "llama8b", lens, 2048, seed=11 + kv_type)
    seqs = []
    K, V = {}, {}
    for i, n in enumerate(lens):
        sid = mgr.AllocateSequence()
        seqs.append(sid)
        K[i] = oracle.normal(500 + i, (n, kv_dim))
        V[i] = oracle.normal(600 + i, (n, kv_dim))
        if n > 1:
            ids, slots = mgr.AppendTokens(sid, n - 1)
            pos = np.arange(n - 1, dtype=np.int32)
            pool.RoPEWrite(0, torch.from_numpy(pos).to(dev), torch.from_numpy(ids).to(dev),
                           torch.from_numpy(slots).to(dev), None,
                           torch.from_numpy(K[i][:n - 1].copy()).to(dev),
                           torch.from_numpy(V[i][:n - 1].copy()).to(dev))
        mgr.AppendToken(sid)
    mb = max((n + P - 1) // P for n in lens)
    bt = np.zeros((len(lens), mb), np.int32)
    for i, sid in enumerate(seqs):
        b = mgr.Tables[sid].BlockIDs
        bt[i, :len(b)] = b
    btd = torch.from_numpy(bt).to(dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    q = oracle.normal(700, (len(lens), H * hd))
    kn = np.stack([K[i][-1] for i in range(len(lens))])
    vn = np.stack([V[i][-1] for i in range(len(lens))])
    qd = torch.from_numpy(q).to(dev)
    out = torch.full((len(lens), H * hd), float("nan"), dtype=torch.float32, device=dev)
    scale = oracle.attn_scale(hd)
    pool.RoPEDecodeStep(out, qd, torch.from_numpy(kn).to(dev), torch.from_numpy(vn).to(dev), 0,
                        btd, sl, H, scale)
    pool.synchronize()
    pos_new = np.array(lens, np.int32) - 1
    qr = oracle.rope_heads(q, pos_new, H, hd, rd, theta)
    assert np.array_equal(qd.cpu().numpy().view(np.uint32), qr.view(np.uint32))
    got = out.cpu().numpy()
    worst = 0.0
    for i, n in enumerate(lens):
        ks = oracle.store_vectors(kv_type, oracle.rope_heads(K[i], np.arange(n), kvh, hd, rd, theta))
        vs = oracle.store_vectors(kv_type, V[i])
        t = torch.from_numpy(bt[i, :(n + P - 1) // P].copy()).to(dev)
        ko, vo = pool.Get(0, t, n)
        assert np.array_equal(ko.cpu().numpy(), ks), i
        assert np.array_equal(vo.cpu().numpy(), vs), i
        want = oracle.attention_decode(qr[i], oracle.widen(kv_type, kv_dim, ks),
                                       oracle.widen(kv_type, kv_dim, vs), H, kvh, hd, n, scale)
        worst = max(worst, float(rel_err_rows(got[i], want, H, hd).max()))
    print("rope decode step max rel err", worst)
    assert worst <= TOL[kv_type], worst


def test_rope_bad_position_and_errors(gi, oracle, dev):
    import torch
    H, kvh, hd, P = 8, 2, 64, 16
    pool = gi.PagedKVCache(1, kvh, hd, P, 4, 1)
    ids = torch.tensor([1, 2], dtype=torch.int32, device=dev)
    slots = torch.tensor([0, 0], dtype=torch.int32, device=dev)
    k = torch.ones((2, kvh * hd), dtype=torch.float32, device=dev)
    q = torch.ones((2, H * hd), dtype=torch.float32, device=dev)
    with pytest.raises(gi.GIError) as ei:                 # no table yet: host check
        pool.RoPEWrite(0, torch.tensor([0, 1], dtype=torch.int32, device=dev), ids, slots, q, k, k)
    assert ei.value.code == -3
    for bad in [(10000.0, 65, 16), (10000.0, 128, 16), (0.0, 64, 16), (10000.0, 64, 0)]:
        with pytest.raises(gi.GIError):
            pool.SetRoPE(*bad)
    pool.SetRoPE(10000.0, 0, 16)
    qo = torch.zeros_like(q)
    pool.RoPEWrite(0, torch.tensor([3, 16], dtype=torch.int32, device=dev), ids, slots, q, k, k,
                   q_out=qo)
    with pytest.raises(gi.GIError) as ei:                 # position 16 is past the table
        pool.synchronize()
    assert ei.value.code == -7 and "RoPE" in str(ei.value)
    pool.synchronize()                                    # flag cleared
    qo = qo.cpu().numpy()
    assert qo[0].any() and not qo[1].any()                # the bad token was skipped whole
    t = torch.tensor([2], dtype=torch.int32, device=dev)
    ko, _ = pool.Get(0, t, 1)
    pool.synchronize()
    assert not ko.cpu().numpy().any()                     # nothing stored for it
