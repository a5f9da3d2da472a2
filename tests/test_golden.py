"""The oracle and the host allocator against the committed golden fixtures
(tests/golden/*.npz, written by tests/golden/make_golden.py).

The fixtures freeze the oracle's outputs after it was pinned by
tests/test_oracle*.py; a change to the oracle that alters any stored byte,
dequantised value, rotated element or attention output fails here.  The
allocator fixture is replayed on both the oracle's PagedKVManager and the
library's C++ one (host code, no GPU)."""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def test_golden_quant(oracle):
    g = load("quant")
    x = g["x"]
    kv_dim = x.shape[1]
    for name, kt in (("f16", oracle.KV_F16), ("q8_0", oracle.KV_Q8_0), ("q4_0", oracle.KV_Q4_0)):
        st = oracle.store_vectors(kt, x)
        assert np.array_equal(st, g["stored_" + name]), name
        assert np.array_equal(bits(oracle.widen(kt, kv_dim, st)), bits(g["widened_" + name])), name


def test_golden_rope(oracle):
    g = load("rope")
    for name in ("llama8b", "tinyllama", "partial"):
        H, hd, rd = (int(v) for v in g[name + "_shape"])
        theta = float(g[name + "_theta"])
        pos = g[name + "_pos"]
        y = oracle.rope_heads(g[name + "_x"], pos, H, hd, rd, theta)
        assert np.array_equal(bits(y), bits(g[name + "_y"])), name
        tab = np.stack([oracle.rope_table(theta, rd, int(p), 1)[0] for p in pos])
        assert np.array_equal(bits(tab), bits(g[name + "_table"])), name


@pytest.mark.parametrize("name,kt", [("f32", 0), ("f16", 1), ("q8_0", 2), ("q4_0", 3)])
def test_golden_attention(oracle, name, kt):
    g = load("attn")
    H, kvh, hd, L = (int(v) for v in g["shape"])
    kv_dim = kvh * hd
    scale = np.float32(g["scale"])
    assert scale == oracle.attn_scale(hd)
    ks = oracle.store_vectors(kt, g["k"])
    vs = oracle.store_vectors(kt, g["v"])
    if kt != 0:
        assert np.array_equal(ks, g["ks_" + name]) and np.array_equal(vs, g["vs_" + name])
    kw, vw = oracle.widen(kt, kv_dim, ks), oracle.widen(kt, kv_dim, vs)
    dec = oracle.attention_decode(g["q"], kw, vw, H, kvh, hd, L, scale)
    assert np.array_equal(bits(dec), bits(g["decode_" + name]))
    pre = oracle.attention_prefill(g["q_prefill"], kw, vw, H, kvh, hd, L - 12, 12, 1 << 30, scale)
    assert np.array_equal(bits(pre), bits(g["prefill_" + name]))


def _replay(mgr_cls, err_cls, g):
    m = mgr_cls(2, 64, 6, 4)
    seqs = [m.AllocateSequence(), m.AllocateSequence()]
    for step, ((op, sid), res) in enumerate(zip(g["ops"], g["results"])):
        if op == 0:
            if res[0] == -4:
                with pytest.raises(err_cls):
                    m.AppendToken(int(sid))
            else:
                got = m.AppendToken(int(sid))
                assert tuple(got) == tuple(int(x) for x in res), step
        else:
            m.FreeSequence(int(sid))
        for i, s in enumerate(seqs):
            want = [int(x) for x in g["tables"][step][i] if x >= 0]
            t = m.Tables[s] if s in m.Tables else None
            ids = [] if t is None else (t["BlockIDs"] if isinstance(t, dict) else t.BlockIDs)
            assert list(ids) == want, (step, i)
        assert list(m.FreeBlocks) == [int(x) for x in g["free"][step] if x >= 0], step


def test_golden_allocator(gi, oracle):
    g = load("alloc")
    _replay(oracle.PagedKVManager, oracle.OutOfPages, g)
    _replay(gi.PagedKVManager, gi.GIError, g)
    # the fixture encodes the reference's LIFO contract: first block N-1
    assert int(g["results"][0][0]) == 5
