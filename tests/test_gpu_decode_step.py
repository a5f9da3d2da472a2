"""The decode step (gi_paged_decode_step, forward.go:236-267): the new
token's K/V stored at position seq_lens[b]-1, then attention over
seq_lens[b] tokens.  The matrix-core decode kernels store the token
themselves in the same launch (the workgroup whose token range holds it);
the vector path appends in a launch of its own first.  Either way the pool
must end up with the bytes gi_paged_append_at_len writes (bit for bit), the
output must equal that of the separate append followed by the attention
(bit for bit: same kernels on the same bytes), and both must match the
oracle on the stored bits within the usual tolerance."""
import numpy as np
import pytest

from gpu_util import Populated, rel_err_rows, seeded
from test_gpu_attention import TOL, kernels_for

pytestmark = pytest.mark.gpu


def gathered(pop, i):
    """Stored bytes of sequence i, layer 0 (K, V as uint8 [n, bytes])."""
    import torch
    bt = torch.from_numpy(pop.table(i)).to(pop.dev)
    k, v = pop.pool.Get(0, bt, pop.lens[i])
    pop.pool.synchronize()
    return k.cpu().numpy(), v.cpu().numpy()


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
@pytest.mark.parametrize("H,kvh,hd,P", [(32, 8, 128, 16), (32, 4, 64, 16), (64, 8, 128, 32), (32, 8, 128, 64)])
def test_decode_step_stores_like_the_append(gi, oracle, dev, kv_type, H, kvh, hd, P):
    """Two pools built alike; one takes DecodeStep, the other WriteAtLen then
    AttentionGQA.  Lengths 1, P, P+1, 37, 1500 and 3000 with a 4096-token
    hint: the 1500-token sequence's new token falls in a split that is not
    the last (splits of 1024), the 1-token one in split 0 of a single page."""
    import torch
    lens = [1, P, P + 1, 37, 1500, 3000]
    B = len(lens)
    scale = oracle.attn_scale(hd)
    seed = 500 + 10 * kv_type + hd
    kn, kn_h = seeded((B, kvh * hd), seed + 1, dev, outliers=True)
    vn, vn_h = seeded((B, kvh * hd), seed + 2, dev, outliers=True)
    qd, q = seeded((B, H * hd), seed + 3, dev)
    for kern in kernels_for(Populated(gi, dev, kv_type, 1, kvh, hd, P, [1], seed=seed).pool, H):
        fused = Populated(gi, dev, kv_type, 1, kvh, hd, P, lens, seed=seed)
        split = Populated(gi, dev, kv_type, 1, kvh, hd, P, lens, seed=seed)
        bt = fused.block_tables()
        assert torch.equal(bt, split.block_tables())
        sl = torch.tensor(lens, dtype=torch.int32, device=dev)
        fused.pool.set_decode_kernel(kern)
        split.pool.set_decode_kernel(kern)
        out_f = torch.full_like(qd, float("nan"))
        out_s = torch.full_like(qd, float("nan"))
        fused.pool.DecodeStep(out_f, qd, kn, vn, 0, bt, sl, H, scale, max_seq_len=4096)
        split.pool.WriteAtLen(0, bt, sl, kn, vn)
        split.pool.AttentionGQA(out_s, qd, 0, bt, sl, H, scale, 4096)
        fused.pool.synchronize()
        split.pool.synchronize()
        assert torch.equal(out_f, out_s), kern
        got = out_f.cpu().numpy()
        for i, n in enumerate(lens):
            kf, vf = gathered(fused, i)
            ks, vs = gathered(split, i)
            assert np.array_equal(kf, ks) and np.array_equal(vf, vs), (kern, i)
            # the oracle on the stored bits, with the new token's own vector
            fused.k[(0, i)][n - 1] = kn_h[i]
            fused.v[(0, i)][n - 1] = vn_h[i]
            kst, vst = fused.stored(0, i)
            assert np.array_equal(kf, kst) and np.array_equal(vf, vst), (kern, i)
            kw = oracle.widen(kv_type, kvh * hd, kst)
            vw = oracle.widen(kv_type, kvh * hd, vst)
            want = oracle.attention_decode(q[i], kw, vw, H, kvh, hd, n, scale)
            err = float(rel_err_rows(got[i], want, H, hd).max())
            assert err <= TOL[kv_type], (kern, i, err)


def test_decode_step_bad_lengths_store_nothing(gi, oracle, dev):
    """A length past what the block table maps, and a length of 0: nothing
    is stored for those sequences, gi_synchronize reports it, and the valid
    sequence is stored and attended as usual."""
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    lens = [100, 300, 50]
    scale = oracle.attn_scale(hd)
    kn, kn_h = seeded((3, kvh * hd), 71, dev)
    vn, vn_h = seeded((3, kvh * hd), 72, dev)
    qd, q = seeded((3, H * hd), 73, dev)
    for kern in kernels_for(Populated(gi, dev, 1, 1, kvh, hd, P, [1], seed=70).pool, H):
        pop = Populated(gi, dev, 1, 1, kvh, hd, P, lens, seed=70)
        pop.pool.set_decode_kernel(kern)
        bt = pop.block_tables()
        mapped = bt.shape[1] * P
        before = [gathered(pop, i) for i in range(3)]
        sl = torch.tensor([100, mapped + 500, 0], dtype=torch.int32, device=dev)
        out = torch.full_like(qd, float("nan"))
        pop.pool.DecodeStep(out, qd, kn, vn, 0, bt, sl, H, scale)
        with pytest.raises(gi.GIError) as e:
            pop.pool.synchronize()
        assert e.value.code == -7, kern
        for i in (1, 2):
            after = gathered(pop, i)
            assert np.array_equal(after[0], before[i][0]) and np.array_equal(after[1], before[i][1]), (kern, i)
        pop.k[(0, 0)][99] = kn_h[0]
        pop.v[(0, 0)][99] = vn_h[0]
        ks, vs = pop.stored(0, 0)
        got_k, got_v = gathered(pop, 0)
        assert np.array_equal(got_k, ks) and np.array_equal(got_v, vs), kern
        want = oracle.attention_decode(q[0], oracle.widen(1, kvh * hd, ks), oracle.widen(1, kvh * hd, vs), H, kvh,
                                       hd, 100, scale)
        assert float(rel_err_rows(out[0].cpu().numpy(), want, H, hd).max()) <= 1e-3, kern
        assert not out[2].cpu().numpy().any(), kern


def test_attention_plan_reports_kernels_waves_and_fusion(gi, oracle, dev):
    """gi_paged_attention_plan on a 256-CU device: the Llama-3-8B shape at
    batch 32 x 4096 gets one workgroup per (sequence, kv head), 256 of them,
    so eight waves each and the token store fused; batch 256 x 8192 gets
    2,048 four-wave workgroups and an append launch; the Llama-3-70B shape
    at 8 x 32768 (pages of 32) takes 4 splits of 8,192 in eight-wave
    workgroups.  Pages of 8 tokens are not a matrix-core shape: the plan
    says the vector ALU serves them as a fallback.  f32 pages keep four
    waves (32 KiB of LDS staging per wave)."""
    import torch
    if torch.cuda.get_device_properties(dev).multi_processor_count != 256:
        pytest.skip("the plans are worked out for a 256-CU device")
    f16 = gi.PagedKVCache(1, 8, 128, 16, 64, gi.KV_F16)
    p = f16.attention_plan(32, 32, 4096)
    assert (p["decode_kernel"], p["decode_fallback"], p["decode_splits"], p["decode_waves"],
            p["decode_step_fused"], p["prefill_kernel"]) == (1, 0, 1, 8, 1, 1), p
    p = f16.attention_plan(256, 32, 8192)
    assert (p["decode_splits"], p["decode_waves"], p["decode_step_fused"]) == (1, 4, 0), p
    d70 = gi.PagedKVCache(1, 8, 128, 32, 64, gi.KV_F16)
    p = d70.attention_plan(8, 64, 32768)
    assert (p["decode_splits"], p["decode_split_tokens"], p["decode_waves"], p["decode_step_fused"]) == \
        (4, 8192, 8, 1), p
    p8 = gi.PagedKVCache(1, 8, 128, 8, 64, gi.KV_F16)
    p = p8.attention_plan(4, 32, 1000)
    assert (p["decode_kernel"], p["decode_fallback"], p["decode_waves"], p["prefill_kernel"],
            p["prefill_fallback"]) == (0, 1, 0, 0, 1), p
    p8.set_decode_kernel(0)
    p = p8.attention_plan(4, 32, 1000)
    assert (p["decode_kernel"], p["decode_fallback"], p["prefill_fallback"]) == (0, 0, 0), p
    f32 = gi.PagedKVCache(1, 8, 128, 16, 64, gi.KV_F32)
    assert f32.attention_plan(32, 32, 4096)["decode_waves"] == 4
    for pool in (f16, d70, p8, f32):
        pool.close()


@pytest.mark.parametrize("kv_type,P", [(1, 16), (1, 32), (2, 16), (3, 16)],
                         ids=["f16-p16", "f16-p32", "q8_0-p16", "q4_0-p16"])
def test_decode_four_and_eight_wave_workgroups_match_the_oracle(gi, oracle, dev, kv_type, P):
    """33 sequences x 8 kv heads make 264 workgroups, more than the CUs: four
    waves each.  The first 32 make 256: eight waves each, every wave taking
    every eighth 32-token block (fp16 pages then stage K through LDS).  Both
    against the oracle on the stored bits, with lengths that leave each wave
    a different number of blocks (and some waves none)."""
    import torch
    H, kvh, hd = 32, 8, 128
    rng = np.random.default_rng(77 + kv_type + P)
    lens = [int(x) for x in rng.integers(1, 700, size=33)]
    lens[0], lens[1], lens[2] = 1, 32 * 8, 32 * 8 + 1
    pop = Populated(gi, dev, kv_type, 1, kvh, hd, P, lens, seed=78 + kv_type)
    bt = pop.block_tables()
    scale = oracle.attn_scale(hd)
    qd, q = seeded((len(lens), H * hd), 79 + kv_type, dev)
    for B in (33, 32):
        plan = pop.pool.attention_plan(B, H, max(lens[:B]))
        if torch.cuda.get_device_properties(dev).multi_processor_count == 256:
            assert plan["decode_waves"] == (4 if B == 33 else 8), plan
        sl = torch.tensor(lens[:B], dtype=torch.int32, device=dev)
        out = torch.full_like(qd[:B], float("nan"))
        pop.pool.AttentionGQA(out, qd[:B].contiguous(), 0, bt[:B].contiguous(), sl, H, scale)
        pop.pool.synchronize()
        got = out.cpu().numpy()
        for i in range(B):
            ks, vs = pop.stored(0, i)
            n = lens[i]
            want = oracle.attention_decode(q[i], oracle.widen(kv_type, kvh * hd, ks[:n]),
                                           oracle.widen(kv_type, kvh * hd, vs[:n]), H, kvh, hd, n, scale)
            err = float(rel_err_rows(got[i], want, H, hd).max())
            assert err <= TOL[kv_type], (B, i, n, err)
