"""GPU parity: append and gather through the C ABI are bit-exact with the
oracle (KVCache.Write / Get semantics, pkg/engine/kvcache.go:146-214, with
FP32ToFP16 and QuantizeQ8_0 from pkg/quant), on fragmented block tables,
ragged lengths and planted special values."""
import numpy as np
import pytest

from gpu_util import Populated

pytestmark = pytest.mark.gpu

SHAPES = {
    # (kv_heads, head_dim, page_tokens): TinyLlama KV, Llama-3-8B KV, 70B (page 32)
    "tinyllama": (4, 64, 16),
    "llama8b": (8, 128, 16),
    "llama70b_p32": (8, 128, 32),
}


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_append_gather_bit_exact(gi, oracle, dev, kv_type, shape):
    kvh, hd, P = SHAPES[shape]
    lens = [1, P - 1, P, P + 1, 3 * P + 5, 70]
    pop = Populated(gi, dev, kv_type, 2, kvh, hd, P, lens, seed=5 + kv_type, specials=True,
                    append_chunk=23)
    import torch
    ref = oracle.RefPagedPool(kv_type, 2, pop.kv_dim, pop.pool.num_pages, P)
    for l in range(2):
        for i, n in enumerate(lens):
            t = pop.table(i)
            ko, vo = pop.pool.Get(l, torch.from_numpy(t).to(dev), n)
            pop.pool.synchronize()
            ks, vs = pop.stored(l, i)
            assert np.array_equal(ko.cpu().numpy(), ks), (l, i)
            assert np.array_equal(vo.cpu().numpy(), vs), (l, i)
            # widened values = FP16ToFP32 / DequantizeQ8_0 of the stored bits
            kw, vw = pop.pool.Get(l, torch.from_numpy(t).to(dev), n, widen=True)
            want_k = oracle.widen(kv_type, pop.kv_dim, ks)
            want_v = oracle.widen(kv_type, pop.kv_dim, vs)
            assert np.array_equal(kw.cpu().numpy().view(np.uint32), want_k.view(np.uint32))
            assert np.array_equal(vw.cpu().numpy().view(np.uint32), want_v.view(np.uint32))
            # the reference-layout paged pool restated by the oracle agrees
            ids = np.repeat(t, P)[:n]
            slots = np.arange(n, dtype=np.int32) % P
            ref.store(l, ids, slots, pop.k[(l, i)], pop.v[(l, i)])
            rk, rv = ref.gather(l, t, n)
            assert np.array_equal(rk, ks) and np.array_equal(rv, vs)


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_bulk_append_bit_exact(gi, oracle, dev, kv_type, shape):
    """Whole sequences appended in one call each (512 and 300 tokens, the
    second not a multiple of 16), with NaN / Inf / subnormal / rounding-tie
    values planted: the bulk append writes runs of 8 tokens of a V row at
    once where their slots are consecutive on one page, and the stored bytes
    must equal the oracle's KVCache.Write (kvcache.go:146-180) bit for bit."""
    import torch
    kvh, hd, P = SHAPES[shape]
    lens = [512, 300]
    pop = Populated(gi, dev, kv_type, 1, kvh, hd, P, lens, seed=41 + kv_type, specials=True)
    for i, n in enumerate(lens):
        t = pop.table(i)
        ko, vo = pop.pool.Get(0, torch.from_numpy(t).to(dev), n)
        pop.pool.synchronize()
        ks, vs = pop.stored(0, i)
        assert np.array_equal(ko.cpu().numpy(), ks), i
        assert np.array_equal(vo.cpu().numpy(), vs), i


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
def test_append_unaligned_inputs(gi, oracle, dev, kv_type):
    """K/V inputs that start 4 bytes past a 16-byte boundary (a caller's
    float pointer) take the per-element append; the stored bytes equal the
    oracle's KVCache.Write all the same."""
    import torch
    kvh, hd, P = SHAPES["llama8b"]
    kv_dim = kvh * hd
    n = 100
    pages = (n + P - 1) // P + 2
    mgr = gi.PagedKVManager(1, kv_dim, pages, P)
    pool = gi.PagedKVCache(1, kvh, hd, P, pages, kv_type)
    sid = mgr.AllocateSequence()
    ids, slots = mgr.AppendTokens(sid, n)
    k = oracle.normal(51, (n, kv_dim))
    v = oracle.normal(52, (n, kv_dim))
    kb = torch.zeros(n * kv_dim + 1, device=dev)
    vb = torch.zeros(n * kv_dim + 1, device=dev)
    kb[1:] = torch.from_numpy(k.reshape(-1)).to(dev)
    vb[1:] = torch.from_numpy(v.reshape(-1)).to(dev)
    ku, vu = kb[1:].view(n, kv_dim), vb[1:].view(n, kv_dim)
    assert ku.data_ptr() % 16 == 4
    pool.Write(0, torch.from_numpy(ids).to(dev), torch.from_numpy(slots).to(dev), ku, vu)
    t = torch.tensor(mgr.Tables[sid].BlockIDs, dtype=torch.int32, device=dev)
    ko, vo = pool.Get(0, t, n)
    pool.synchronize()
    assert np.array_equal(ko.cpu().numpy(), oracle.store_vectors(kv_type, k))
    assert np.array_equal(vo.cpu().numpy(), oracle.store_vectors(kv_type, v))
    pool.close()


def test_reference_kvcache_tests_on_pages(gi, oracle, dev):
    import torch
    # kvcache_test.go:7-71 values i+1 / 2(i+1) and engine_test.go:251-273
    # (Q8_0, k[i] = i, |deq[10] - 10| <= 0.5), stored into page slots.
    for kv_type in (0, 1, 2):
        pool = gi.PagedKVCache(2, 1, 64, 16, 4, kv_type)
        k = (np.arange(64, dtype=np.float32) + 1)[None, :]
        v = 2 * k
        ids = torch.tensor([2], dtype=torch.int32, device=dev)
        slots = torch.tensor([5], dtype=torch.int32, device=dev)
        pool.Write(1, ids, slots, torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev))
        table = torch.tensor([0, 0, 2, 0], dtype=torch.int32, device=dev)
        kw, vw = pool.Get(1, table[2:3], 6, widen=True)
        pool.synchronize()
        kw, vw = kw.cpu().numpy(), vw.cpu().numpy()
        if kv_type == 0:
            assert kw[5, 0] == 1.0 and vw[5, 0] == 2.0
        assert np.all(np.abs(kw[5] - k[0]) <= (0.5 if kv_type == 2 else 0.03 * k[0]))
        assert not kw[:5].any()               # untouched slots stay zero
        ql = np.arange(32, dtype=np.float32)[None, :]
        pool8 = gi.PagedKVCache(1, 1, 32, 4, 1, 2)
        pool8.Write(0, torch.tensor([0], dtype=torch.int32, device=dev),
                    torch.tensor([0], dtype=torch.int32, device=dev),
                    torch.from_numpy(ql).to(dev), torch.from_numpy(2 * ql).to(dev))
        kr, _ = pool8.Get(0, torch.tensor([0], dtype=torch.int32, device=dev), 1, widen=True)
        assert abs(float(kr[0, 10]) - 10.0) <= 0.5


def test_decode_step_append_at_len(gi, oracle, dev):
    """gi_paged_append_at_len writes position seq_lens[b]-1 through the
    block table, bit-exact with an explicit append."""
    import torch
    kvh, hd, P = 8, 128, 16
    for kv_type in (1, 2, 3):
        lens = [17, 32, 5, 100]
        pop = Populated(gi, dev, kv_type, 1, kvh, hd, P, lens, seed=77, slack_pages=8)
        bt = pop.block_tables()
        # grow every sequence by one token and append it at len-1
        new_lens = []
        for i, sid in enumerate(pop.seqs):
            pop.mgr.AppendToken(sid)
            new_lens.append(lens[i] + 1)
        pop.max_blocks = max((n + P - 1) // P for n in new_lens)
        bt = pop.block_tables()
        kn = oracle.normal(900 + kv_type, (len(lens), pop.kv_dim))
        vn = oracle.normal(901 + kv_type, (len(lens), pop.kv_dim))
        sl = torch.tensor(new_lens, dtype=torch.int32, device=dev)
        pop.pool.WriteAtLen(0, bt, sl, torch.from_numpy(kn).to(dev), torch.from_numpy(vn).to(dev))
        pop.pool.synchronize()
        for i, n in enumerate(new_lens):
            t = np.array(pop.mgr.Tables[pop.seqs[i]].BlockIDs, np.int32)
            ko, vo = pop.pool.Get(0, torch.from_numpy(t).to(dev), n)
            ko, vo = ko.cpu().numpy(), vo.cpu().numpy()
            ks = oracle.store_vectors(kv_type, np.concatenate([pop.k[(0, i)], kn[i:i + 1]]))
            vs = oracle.store_vectors(kv_type, np.concatenate([pop.v[(0, i)], vn[i:i + 1]]))
            assert np.array_equal(ko, ks) and np.array_equal(vo, vs)


def test_reference_q4_0_kvcache_tests_on_pages(gi, oracle, dev):
    """engine_test.go:275-297 (Q4_0, kvDim 32, k[i] = i, |deq[10] - 10| <=
    3) and kvcache_test.go:7-71 (values i+1 / 2(i+1), kvDim 64) on pages,
    bit-exact with the oracle's QuantizeQ4_0 blocks."""
    import torch
    pool = gi.PagedKVCache(1, 1, 32, 4, 2, gi.KV_Q4_0)
    k = np.arange(32, dtype=np.float32)[None, :]
    z = torch.tensor([1], dtype=torch.int32, device=dev)
    pool.Write(0, z, torch.tensor([2], dtype=torch.int32, device=dev),
               torch.from_numpy(k).to(dev), torch.from_numpy(2 * k).to(dev))
    kw, vw = pool.Get(0, z, 3, widen=True)
    kr, vr = pool.Get(0, z, 3)
    pool.synchronize()
    assert abs(float(kw[2, 10]) - 10.0) <= 3.0
    assert np.array_equal(kr.cpu().numpy()[2], oracle.quantize_q4_0(k[0]))
    assert np.array_equal(vr.cpu().numpy()[2], oracle.quantize_q4_0(2 * k[0]))
    assert not kr.cpu().numpy()[:2].any()
    pool64 = gi.PagedKVCache(2, 1, 64, 16, 2, gi.KV_Q4_0)
    k = (np.arange(64, dtype=np.float32) + 1)[None, :]
    pool64.Write(1, z, torch.tensor([0], dtype=torch.int32, device=dev),
                 torch.from_numpy(k).to(dev), torch.from_numpy(2 * k).to(dev))
    kr, vr = pool64.Get(1, z, 1)
    pool64.synchronize()
    assert kr.shape == (1, 36)
    assert np.array_equal(kr.cpu().numpy()[0], oracle.quantize_q4_0(k[0]))
    assert np.array_equal(vr.cpu().numpy()[0], oracle.quantize_q4_0(2 * k[0]))


def test_bad_page_ids_are_reported(gi, dev):
    import torch
    pool = gi.PagedKVCache(1, 2, 64, 16, 4, 1)
    k = torch.zeros((2, 128), dtype=torch.float32, device=dev)
    ids = torch.tensor([1, 9], dtype=torch.int32, device=dev)       # 9 is outside the pool
    slots = torch.tensor([0, 3], dtype=torch.int32, device=dev)
    pool.Write(0, ids, slots, k, k)
    with pytest.raises(gi.GIError) as ei:
        pool.synchronize()
    assert ei.value.code == -7
    pool.synchronize()                                              # flag was cleared
    bad_slot = torch.tensor([16, 0], dtype=torch.int32, device=dev)
    pool.Write(0, torch.tensor([1, 2], dtype=torch.int32, device=dev), bad_slot, k, k)
    with pytest.raises(gi.GIError):
        pool.synchronize()
    table = torch.tensor([0, -1], dtype=torch.int32, device=dev)
    pool.Get(0, table, 20)
    with pytest.raises(gi.GIError):
        pool.synchronize()
    with pytest.raises(gi.GIError) as ei:
        pool.Write(3, ids, slots, k, k)                              # bad layer, host check
    assert ei.value.code == -3
