"""GPU parity for copy-on-write prefix sharing: random allocate / append /
fork / free on a device pool, with the copy each copy-on-write append asks
for done by gi_paged_copy_pages, keep every live sequence's pages bit-exact
with the reference's deep-copied KVCache (ForkAt, kvcache.go:225-284)
restated in the oracle; decode attention over a forked sequence matches the
oracle over the model's contents; a paged PrefixCache hit reads the stored
prefix."""
import random

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class DevPool:
    def __init__(self, gi, dev, kv_type, L, kvh, hd, N, P):
        import torch
        self.torch, self.dev = torch, dev
        self.mgr = gi.PagedKVManager(L, kvh * hd, N, P)
        self.pool = gi.PagedKVCache(L, kvh, hd, P, N, kv_type)
        self.L, self.kv_dim = L, kvh * hd
        self.copies = 0

    def append(self, sid, k, v):
        """k, v: [L, kv_dim] float32 (host) of one token."""
        t = self.torch
        b, s, c = self.mgr.AppendTokenCOW(sid)
        if c >= 0:
            self.pool.CopyPages(t.tensor([c], dtype=t.int32, device=self.dev),
                                t.tensor([b], dtype=t.int32, device=self.dev))
            self.copies += 1
        ids = t.tensor([b], dtype=t.int32, device=self.dev)
        slots = t.tensor([s], dtype=t.int32, device=self.dev)
        for l in range(self.L):
            self.pool.Write(l, ids, slots, t.from_numpy(np.ascontiguousarray(k[l][None])).to(self.dev),
                            t.from_numpy(np.ascontiguousarray(v[l][None])).to(self.dev))

    def table(self, sid):
        t = self.mgr.Tables[sid]
        return np.array(t.BlockIDs or [0], np.int32), t.NumTokens

    def gather(self, sid, layer):
        ids, n = self.table(sid)
        k, v = self.pool.Get(layer, self.torch.from_numpy(ids).to(self.dev), n)
        self.pool.synchronize()
        return k.cpu().numpy(), v.cpu().numpy()


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
def test_fork_cow_differential_on_device(gi, oracle, dev, kv_type):
    rng = random.Random(3 + kv_type)
    L, kvh, hd, P, N = 2, 2, 64, 16, 64
    dp = DevPool(gi, dev, kv_type, L, kvh, hd, N, P)
    D = kvh * hd
    model, live, gen = {}, [], 0
    print("fork/cow differential kv_type", kv_type, flush=True)
    for step in range(160):
        op = rng.random()
        if not live or op < 0.12:
            sid = dp.mgr.AllocateSequence()
            model[sid] = oracle.RefKVCache(kv_type, L, D, 512)
            live.append(sid)
        elif op < 0.62:
            sid = rng.choice(live)
            for _ in range(rng.randint(1, 24)):
                if len(dp.mgr.FreeBlocks) < 2:
                    break
                k = oracle.normal(300 + gen, (L, D))
                v = oracle.normal(700 + gen, (L, D))
                gen += 1
                dp.append(sid, k, v)
                m = model[sid]
                for l in range(L):
                    m.Write(l, m.CurPos, k[l], v[l])
                m.CurPos += 1
        elif op < 0.85:
            src = rng.choice(live)
            n = rng.randint(0, model[src].CurPos)
            sid = dp.mgr.ForkSequence(src, n)
            f = model[src].ForkAt(n)
            f.CurPos = n
            model[sid] = f
            live.append(sid)
        else:
            sid = live.pop(rng.randrange(len(live)))
            dp.mgr.FreeSequence(sid)
            del model[sid]
        if step % 40 == 39:
            for sid in live:
                m = model[sid]
                for l in range(L):
                    k, v = dp.gather(sid, l)
                    assert np.array_equal(k, m.K[l, :m.CurPos]), (step, sid, l)
                    assert np.array_equal(v, m.V[l, :m.CurPos]), (step, sid, l)
    assert dp.copies > 0


def test_decode_attention_on_forked_sequence(gi, oracle, dev):
    """Two sequences forked from one prompt and extended differently attend
    over their own contexts (fp16 pages, Llama-style GQA 8 q / 2 kv heads)."""
    import torch
    L, kvh, hd, P, H = 1, 2, 128, 16, 8
    dp = DevPool(gi, dev, 1, L, kvh, hd, 32, P)
    D = kvh * hd
    a = dp.mgr.AllocateSequence()
    ma = oracle.RefKVCache(1, L, D, 256)
    for t in range(37):
        k = oracle.normal(10 + t, (L, D))
        v = oracle.normal(90 + t, (L, D))
        dp.append(a, k, v)
        ma.Write(0, t, k[0], v[0])
    ma.CurPos = 37
    b = dp.mgr.ForkSequence(a, 37)
    mb = ma.ForkAt(37)
    for t in range(9):
        for sid, m, seed in ((a, ma, 500), (b, mb, 600)):
            k = oracle.normal(seed + t, (L, D))
            v = oracle.normal(seed + 50 + t, (L, D))
            dp.append(sid, k, v)
            m.Write(0, m.CurPos, k[0], v[0])
            m.CurPos += 1
    assert dp.copies == 1  # the shared partial page, copied by the first appender
    q = oracle.normal(7, (2, H * hd))
    tabs = [dp.table(a)[0], dp.table(b)[0]]
    mb_ = max(len(x) for x in tabs)
    bt = np.zeros((2, mb_), np.int32)
    for i, x in enumerate(tabs):
        bt[i, :len(x)] = x
    lens = np.array([ma.CurPos, mb.CurPos], np.int32)
    out = torch.empty((2, H * hd), dtype=torch.float32, device=dev)
    scale = gi.attn_scale(hd)
    dp.pool.AttentionGQA(out, torch.from_numpy(q).to(dev), 0, torch.from_numpy(bt).to(dev),
                         torch.from_numpy(lens).to(dev), H, scale)
    dp.pool.synchronize()
    got = out.cpu().numpy()
    for i, m in enumerate((ma, mb)):
        n = m.CurPos
        kw = oracle.widen(1, D, m.K[0, :n])
        vw = oracle.widen(1, D, m.V[0, :n])
        want = oracle.attention_decode(q[i], kw, vw, H, kvh, hd, n, scale).reshape(H, hd)
        err = (np.abs(got[i].reshape(H, hd) - want).max(axis=1) / np.abs(want).max(axis=1)).max()
        assert err <= 1e-3, (i, err)


def test_prefix_cache_hit_on_device(gi, oracle, dev):
    """prefix_cache_test.go:7-47 on device pages: the hit's gathered prefix
    equals the stored sequence's, and extending the hit leaves the entry
    intact for the next lookup."""
    L, kvh, hd, P = 2, 1, 64, 16
    dp = DevPool(gi, dev, 2, L, kvh, hd, 16, P)
    D = kvh * hd
    pc = gi.PrefixCache(dp.mgr, 10)
    a = dp.mgr.AllocateSequence()
    for t in range(10):
        dp.append(a, oracle.normal(40 + t, (L, D)), oracle.normal(80 + t, (L, D)))
    pc.Store([101, 202, 303, 404, 505], a)
    ka = [dp.gather(a, l) for l in range(L)]
    dp.mgr.FreeSequence(a)  # the entry keeps its own references
    for rep in range(2):
        n, sid = pc.FindLongestPrefix([101, 202, 303, 404, 505, 606, 707])
        assert n == 5
        for l in range(L):
            k, v = dp.gather(sid, l)
            assert np.array_equal(k, ka[l][0][:5]) and np.array_equal(v, ka[l][1][:5])
        dp.append(sid, oracle.normal(900 + rep, (L, D)), oracle.normal(901 + rep, (L, D)))
        dp.mgr.FreeSequence(sid)
    assert dp.copies == 2
    assert pc.FindLongestPrefix([999, 888, 777]) == (0, None)
    pc.close()
