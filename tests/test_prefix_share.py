"""Copy-on-write prefix sharing: the allocator's fork / copy-on-write append /
refcounted free, and the paged PrefixCache, against the reference's deep-copy
semantics (KVCache.ForkAt / Clone, kvcache.go:217-284; PrefixCache,
prefix_cache.go:7-150) restated in the oracle.

These tests run on the CPU: the device pool is simulated with the oracle's
reference-layout page pool, and the copy that a copy-on-write append asks for
is done there.  The GPU versions (tests/test_gpu_prefix.py) run the same
checks through gi_paged_copy_pages / append / gather."""
import random

import numpy as np
import pytest


class SimPool:
    """Pages on the host (oracle RefPagedPool: [block][layer][token][bytes]) driven
    by the library's allocator, the way a device pool is."""

    def __init__(self, gi, oracle, kv_type, num_layers, kv_dim, num_blocks, block_size):
        self.gi, self.oracle = gi, oracle
        self.mgr = gi.PagedKVManager(num_layers, kv_dim, num_blocks, block_size)
        self.pool = oracle.RefPagedPool(kv_type, num_layers, kv_dim, num_blocks, block_size)
        self.L, self.P = num_layers, block_size
        self.blk = num_layers * block_size * self.pool.bpv  # bytes of one block, all layers
        self.copies = 0

    def copy_page(self, src, dst):
        for a in (self.pool.k, self.pool.v):
            a[dst * self.blk:(dst + 1) * self.blk] = a[src * self.blk:(src + 1) * self.blk]
        self.copies += 1

    def append(self, sid, k, v):
        """k, v: [layers, kv_dim] float32 of one token."""
        b, s, c = self.mgr.AppendTokenCOW(sid)
        if c >= 0:
            self.copy_page(c, b)
        for l in range(self.L):
            self.pool.store(l, [b], [s], k[l][None], v[l][None])

    def gather(self, sid, layer):
        t = self.mgr.Tables[sid]
        return self.pool.gather(layer, np.array(t.BlockIDs or [0], np.int32), t.NumTokens)


def check_refcounts(sp, live):
    """Each block's references = the live tables (and cache entries) holding it;
    free blocks are exactly the unreferenced ones."""
    counts = {}
    for sid in live:
        for b in sp.mgr.Tables[sid].BlockIDs:
            counts[b] = counts.get(b, 0) + 1
    free = sp.mgr.FreeBlocks
    assert len(set(free)) == len(free)
    for b in range(sp.mgr.TotalBlocks):
        r = sp.mgr.BlockRefs(b)
        if b in free:
            assert r == 0, (b, r)
        else:
            assert r >= counts.get(b, 0) and r > 0, (b, r, counts.get(b))


def check_contents(sp, model, live):
    for sid in live:
        m = model[sid]
        n = sp.mgr.Tables[sid].NumTokens
        assert n == m.CurPos
        for l in range(sp.L):
            k, v = sp.gather(sid, l)
            assert np.array_equal(k, m.K[l, :n]), (sid, l)
            assert np.array_equal(v, m.V[l, :n]), (sid, l)


def test_reference_clone_and_fork(gi, oracle):
    """kvcache_test.go:7-71 restated on pages: populate slots, fork, and
    writing the fork leaves the original untouched."""
    for kv_type in (oracle.KV_F32, oracle.KV_Q8_0):
        sp = SimPool(gi, oracle, kv_type, 2, 64, 16, 4)
        a = sp.mgr.AllocateSequence()
        kvec = np.arange(1, 65, dtype=np.float32)
        vvec = kvec * 2
        zeros = np.zeros(64, np.float32)
        for tok in range(4):  # CurPos = 4; slot 0 of layer 0 and slot 1 of layer 1 hold data
            k = np.stack([kvec if tok == 0 else zeros, kvec if tok == 1 else zeros])
            v = np.stack([vvec if tok == 0 else zeros, vvec if tok == 1 else zeros])
            sp.append(a, k, v)
        clone = sp.mgr.ForkSequence(a, 4)
        assert sp.mgr.Tables[clone].NumTokens == 4
        assert sp.mgr.Tables[clone].BlockIDs == sp.mgr.Tables[a].BlockIDs
        k0, v0 = sp.gather(clone, 0)
        ka, va = sp.gather(a, 0)
        assert np.array_equal(k0, ka) and np.array_equal(v0, va)
        fork1 = sp.mgr.ForkSequence(a, 1)
        assert sp.mgr.Tables[fork1].NumTokens == 1
        # the clone's next token goes to a fresh block (4 tokens fill the page);
        # fork1 writes into the shared first page, which is copied first
        newk = np.zeros((2, 64), np.float32)
        newk[:, 0] = 999.0
        sp.append(fork1, newk, newk)
        assert sp.copies == 1
        ka2, va2 = sp.gather(a, 0)
        assert np.array_equal(ka2, ka) and np.array_equal(va2, va)
        kf, _ = sp.gather(fork1, 0)
        assert np.array_equal(kf[0], ka[0])
        assert not np.array_equal(kf[1], ka[1])


def test_fork_refcounts_and_cow(gi, oracle):
    sp = SimPool(gi, oracle, 0, 1, 8, 32, 16)
    m = sp.mgr
    a = m.AllocateSequence()
    for _ in range(40):
        sp.append(a, np.ones((1, 8), np.float32), np.ones((1, 8), np.float32))
    ta = list(m.Tables[a].BlockIDs)
    assert ta == [31, 30, 29]  # LIFO pops (paged_kv.go:122-123)
    b = m.ForkSequence(a, 40)
    assert [m.BlockRefs(x) for x in ta] == [2, 2, 2]
    # the shared, partly filled last page is copied by whichever appends first
    blk, slot, cp = m.AppendTokenCOW(b)
    assert (blk, slot, cp) == (28, 8, 29)
    assert m.Tables[b].BlockIDs == [31, 30, 28]
    assert [m.BlockRefs(x) for x in (31, 30, 29, 28)] == [2, 2, 1, 1]
    blk, slot, cp = m.AppendTokenCOW(a)  # the original now owns page 29 alone
    assert (blk, slot, cp) == (29, 8, -1)
    # a fork on a page boundary never copies
    c = m.ForkSequence(a, 32)
    assert m.Tables[c].BlockIDs == [31, 30]
    blk, slot, cp = m.AppendTokenCOW(c)
    assert (blk, slot, cp) == (27, 0, -1)
    # forks clamp to the source length, like ForkAt clamps maxSlot (kvcache.go:241-246)
    d = m.ForkSequence(a, 1000)
    assert m.Tables[d].NumTokens == m.Tables[a].NumTokens
    # freeing returns a block only with its last reference, in table order
    m.FreeSequence(a)
    assert m.BlockRefs(29) == 1 and 29 not in m.FreeBlocks
    m.FreeSequence(d)
    assert m.FreeBlocks[-1] == 29
    m.FreeSequence(b)
    m.FreeSequence(c)
    assert sorted(m.FreeBlocks) == list(range(32))
    with pytest.raises(gi.GIError) as e:
        m.ForkSequence(12345, 1)
    assert e.value.code == -6


def test_plain_append_refuses_shared_page(gi, oracle):
    m = gi.PagedKVManager(1, 8, 8, 4)
    a = m.AllocateSequence()
    m.AppendTokens(a, 3)
    b = m.ForkSequence(a, 3)
    for fn in (lambda: m.AppendToken(b), lambda: m.AppendTokens(a, 2)):
        with pytest.raises(gi.GIError) as e:
            fn()
        assert e.value.code == -8
    assert m.Tables[b].NumTokens == 3 and m.Tables[a].NumTokens == 3
    ids, slots, (cs, cd) = m.AppendTokensCOW(a, 3)
    assert cs == m.Tables[b].BlockIDs[0] and cd == ids[0] and list(slots) == [3, 0, 1]


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3])
def test_fork_cow_differential(gi, oracle, kv_type):
    """Random allocate / append / fork / free: every live sequence's pages hold
    exactly what the reference's deep-copied KVCache would (ForkAt semantics),
    bit for bit, and reference counts stay consistent."""
    rng = random.Random(17 + kv_type)
    L, D, P, N = 3, 64, 4, 96
    sp = SimPool(gi, oracle, kv_type, L, D, N, P)
    model, live = {}, []
    gen = 0
    for step in range(300):
        op = rng.random()
        if not live or op < 0.12:
            sid = sp.mgr.AllocateSequence()
            model[sid] = oracle.RefKVCache(kv_type, L, D, 256)
            live.append(sid)
        elif op < 0.62:
            sid = rng.choice(live)
            for _ in range(rng.randint(1, 6)):
                if len(sp.mgr.FreeBlocks) < 2:
                    break
                k = oracle.normal(1000 + gen, (L, D))
                v = oracle.normal(2000 + gen, (L, D))
                gen += 1
                sp.append(sid, k, v)
                m = model[sid]
                for l in range(L):
                    m.Write(l, m.CurPos, k[l], v[l])
                m.CurPos += 1
        elif op < 0.85:
            src = rng.choice(live)
            n = rng.randint(0, model[src].CurPos)
            sid = sp.mgr.ForkSequence(src, n)
            f = model[src].ForkAt(n)
            f.CurPos = n  # a paged fork continues at its fork point
            model[sid] = f
            live.append(sid)
        else:
            sid = live.pop(rng.randrange(len(live)))
            sp.mgr.FreeSequence(sid)
            del model[sid]
        if step % 25 == 0 or step == 299:
            check_contents(sp, model, live)
            check_refcounts(sp, live)
    assert sp.copies > 0


def test_reference_prefix_cache(gi, oracle):
    """prefix_cache_test.go:7-47 restated: a stored 5-token prompt matches a
    7-token query at length 5 with the same cached data; a miss is (0, nil)."""
    sp = SimPool(gi, oracle, 0, 4, 64, 16, 4)
    pc = gi.PrefixCache(sp.mgr, 10)
    a = sp.mgr.AllocateSequence()
    for t in range(10):
        k = np.arange(t * 64 + 1, t * 64 + 65, dtype=np.float32)[None].repeat(4, 0)
        sp.append(a, k, k + 1)
    pc.Store([101, 202, 303, 404, 505], a)
    n, sid = pc.FindLongestPrefix([101, 202, 303, 404, 505, 606, 707])
    assert n == 5 and sid is not None
    k0, _ = sp.gather(sid, 0)
    ka, _ = sp.gather(a, 0)
    assert k0.shape[0] == 5 and np.array_equal(k0, ka[:5])
    assert pc.FindLongestPrefix([999, 888, 777]) == (0, None)
    assert len(pc) == 1
    # an entry keyed on more tokens than the sequence holds is refused: a hit
    # on it would report 12 cached tokens for a 10-token fork
    with pytest.raises(gi.GIError) as e:
        pc.Store(list(range(12)), a)
    assert e.value.code == -3
    assert len(pc) == 1 and pc.FindLongestPrefix(list(range(12)) + [0]) == (0, None)
    pc.close()


def test_prefix_cache_differential(gi, oracle):
    """Random Store / FindLongestPrefix against the restated reference cache:
    same matched lengths, same KV contents, entries never corrupted by
    appends to the sequences they were stored from or handed out to."""
    rng = random.Random(5)
    L, D, P = 2, 32, 4
    sp = SimPool(gi, oracle, 2, L, D, 160, P)
    pc = gi.PrefixCache(sp.mgr, 3)
    ref = oracle.RefPrefixCache(3)
    vocab = [1, 2, 3]
    gen = 0
    seqs = {}
    for step in range(120):
        toks = [rng.choice(vocab) for _ in range(rng.randint(2, 9))]
        if rng.random() < 0.5:
            # a fresh sequence run over toks, then stored
            sid = sp.mgr.AllocateSequence()
            m = oracle.RefKVCache(2, L, D, 64)
            for _ in toks:
                k = oracle.normal(50 + gen, (L, D))
                v = oracle.normal(90 + gen, (L, D))
                gen += 1
                sp.append(sid, k, v)
                for l in range(L):
                    m.Write(l, m.CurPos, k[l], v[l])
                m.CurPos += 1
            pc.Store(toks, sid)
            ref.Store(toks, m.Clone())
            seqs[sid] = m
        else:
            n, sid = pc.FindLongestPrefix(toks)
            rn, rkv = ref.FindLongestPrefix(toks)
            assert n == rn, (toks, n, rn)
            if n:
                assert sp.mgr.Tables[sid].NumTokens == n
                for l in range(L):
                    k, v = sp.gather(sid, l)
                    assert np.array_equal(k, rkv.K[l, :n]) and np.array_equal(v, rkv.V[l, :n])
                # extend the hit (copy-on-write must keep the entry intact)
                k = oracle.normal(7000 + step, (L, D))
                sp.append(sid, k, k)
                sp.mgr.FreeSequence(sid)
        assert len(pc) == len(ref.entries)
    # the sequences entries were stored from can be freed: entries keep their pages
    for sid in list(seqs):
        sp.mgr.FreeSequence(sid)
    for key, rkv in ref.entries.items():
        n, sid = pc.FindLongestPrefix(list(key) + [0])
        assert n == len(key)
        k, _ = sp.gather(sid, 0)
        assert np.array_equal(k, rkv.K[0, :n])
        sp.mgr.FreeSequence(sid)
    pc.close()
    assert sorted(sp.mgr.FreeBlocks) == list(range(160))
