"""The HIP path against the committed golden fixtures (tests/golden/*.npz).

Append + gather must reproduce the fixtures' stored bytes and dequantised
floats exactly; RoPE + append the rotated q and stored K exactly; decode and
chunked-prefill attention the fixtures' outputs within the attention
tolerance, max|gpu - golden| <= tol * max|golden| per (query, head) row with
tol 1e-5 (f32 KV) or 1e-3 (f16 / q8_0 / q4_0 KV), on every kernel that can
serve the pool."""
import os

import numpy as np
import pytest

from gpu_util import rel_err_rows

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = {0: 1e-5, 1: 1e-3, 2: 1e-3, 3: 1e-3}
KT = {"f32": 0, "f16": 1, "q8_0": 2, "q4_0": 3}


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def _pool_with_tokens(gi, dev, kt, kvh, hd, P, n, k, v, seed):
    """n tokens of one sequence written in chunks of 7 into pages drawn
    from a shuffled pool; returns (pool, device block table)."""
    import torch
    pages = (n + P - 1) // P + 3
    mgr = gi.PagedKVManager(1, kvh * hd, pages, P)
    mgr.SetFreeList(np.random.default_rng(seed).permutation(pages).astype(np.int32))
    pool = gi.PagedKVCache(1, kvh, hd, P, pages, kt)
    sid = mgr.AllocateSequence()
    ids, slots = mgr.AppendTokens(sid, n)
    for a in range(0, n, 7):
        b = min(n, a + 7)
        pool.Write(0, torch.from_numpy(ids[a:b].copy()).to(dev), torch.from_numpy(slots[a:b].copy()).to(dev),
                   torch.from_numpy(np.ascontiguousarray(k[a:b])).to(dev),
                   torch.from_numpy(np.ascontiguousarray(v[a:b])).to(dev))
    table = torch.tensor(mgr.Tables[sid].BlockIDs, dtype=torch.int32, device=dev)
    return pool, table


@pytest.mark.parametrize("name", ["f16", "q8_0", "q4_0"])
def test_golden_append_gather(gi, dev, name):
    g = load("quant")
    x = g["x"]
    pool, table = _pool_with_tokens(gi, dev, KT[name], 2, 128, 16, x.shape[0], x, -x, seed=1)
    ko, _ = pool.Get(0, table, x.shape[0])
    kw, _ = pool.Get(0, table, x.shape[0], widen=True)
    pool.synchronize()
    assert np.array_equal(ko.cpu().numpy(), g["stored_" + name])
    assert np.array_equal(kw.cpu().numpy().view(np.uint32), g["widened_" + name].view(np.uint32))


@pytest.mark.parametrize("case", ["llama8b", "tinyllama", "partial"])
def test_golden_rope_append(gi, dev, case):
    import torch
    g = load("rope")
    H, hd, rd = (int(v) for v in g[case + "_shape"])
    x, pos, y = g[case + "_x"], g[case + "_pos"], g[case + "_y"]
    n = pos.size
    # H kv heads, so the same vectors serve as q and as k
    pool = gi.PagedKVCache(1, H, hd, 16, 4, gi.KV_F32)
    pool.SetRoPE(float(g[case + "_theta"]), rd, 131072)
    ids = torch.tensor([2] * 10, dtype=torch.int32, device=dev)
    slots = torch.arange(n, dtype=torch.int32, device=dev)
    xd = torch.from_numpy(x).to(dev)
    qo = torch.empty_like(xd)
    pool.RoPEWrite(0, torch.from_numpy(pos).to(dev), ids, slots, xd, xd, xd, q_out=qo)
    ko, vo = pool.Get(0, torch.tensor([2], dtype=torch.int32, device=dev), n)
    pool.synchronize()
    assert np.array_equal(qo.cpu().numpy().view(np.uint32), y.view(np.uint32))
    assert np.array_equal(ko.cpu().numpy(), y.view(np.uint8).reshape(n, -1))
    assert np.array_equal(vo.cpu().numpy(), x.view(np.uint8).reshape(n, -1))


@pytest.mark.parametrize("name", ["f32", "f16", "q8_0", "q4_0"])
def test_golden_attention(gi, dev, name):
    import torch
    g = load("attn")
    H, kvh, hd, L = (int(v) for v in g["shape"])
    scale = float(g["scale"])
    kt = KT[name]
    pool, table = _pool_with_tokens(gi, dev, kt, kvh, hd, 16, L, g["k"], g["v"], seed=2)
    if kt != 0:
        ko, vo = pool.Get(0, table, L)
        pool.synchronize()
        assert np.array_equal(ko.cpu().numpy(), g["ks_" + name])
        assert np.array_equal(vo.cpu().numpy(), g["vs_" + name])
    bt = table[None, :].contiguous()
    q = torch.from_numpy(g["q"][None, :].copy()).to(dev)
    qp = torch.from_numpy(g["q_prefill"][None].copy()).to(dev)
    sl = torch.tensor([L], dtype=torch.int32, device=dev)
    sp = torch.tensor([L - 12], dtype=torch.int32, device=dev)
    pool.set_decode_kernel(1)
    kinds = [0, 1] if pool.decode_kernel(H) == 1 else [0]
    worst = {}
    for kern in kinds:
        pool.set_decode_kernel(kern)
        out = torch.full_like(q, float("nan"))
        pool.AttentionGQA(out, q, 0, bt, sl, H, scale)
        outp = torch.full_like(qp, float("nan"))
        pool.AttentionGQABatch(outp, qp, 0, bt, sp, H, scale, 12)
        pool.synchronize()
        e = max(float(rel_err_rows(out.cpu().numpy(), g["decode_" + name], H, hd).max()),
                float(rel_err_rows(outp.cpu().numpy(), g["prefill_" + name], H, hd).max()))
        worst[kern] = e
    print("golden attention", name, worst)
    assert max(worst.values()) <= TOL[kt], worst
