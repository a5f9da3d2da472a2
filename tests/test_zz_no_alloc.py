"""The decode entry point that allocates nothing
(gi_paged_decode_attention_noalloc): its split partials live in the
library's fixed per-device scratch array instead of the handle's workspace.
Called through the C ABI, its output must equal gi_paged_decode_attention's
bit for bit (same kernels, same split plan, same merge order) on two calls in
a row, the second with a smaller batch and shorter contexts (the scratch keeps
the first call's contents), and both must match the oracle (forward.go:
242-267) within the fp16 tolerance 1e-3.  A shape whose partials would not
fit the fixed maximum is refused."""
import numpy as np
import pytest

from gpu_util import Populated, rel_err_rows, seeded

pytestmark = pytest.mark.gpu


def test_noalloc_decode_matches_the_allocating_entry_point(gi, oracle, dev):
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    lens = [5000, 300, 2048, 1, 4100, 777]
    pop = Populated(gi, dev, 1, 1, kvh, hd, P, lens, seed=41)
    bt = pop.block_tables()
    scale = oracle.attn_scale(hd)
    qd, q = seeded((len(lens), H * hd), 42, dev)
    # second call: fewer sequences and shorter contexts
    small = [0, 5, 1]
    lens2 = [1500, 777, 64]
    for rows, ls in ((list(range(len(lens))), lens), (small, lens2)):
        idx = torch.tensor(rows, device=dev)
        btr = bt[idx].contiguous()
        sl = torch.tensor(ls, dtype=torch.int32, device=dev)
        qr = qd[idx].contiguous()
        want = torch.full_like(qr, float("nan"))
        got = torch.full_like(qr, float("nan"))
        pop.pool.AttentionGQA(want, qr, 0, btr, sl, H, scale)
        pop.pool.AttentionGQANoAlloc(got, qr, 0, btr, sl, H, scale)
        pop.pool.synchronize()
        assert torch.equal(got, want), rows
        o = got.cpu().numpy()
        for r, (i, n) in enumerate(zip(rows, ls)):
            ks, vs = pop.stored(0, i)
            w = oracle.attention_decode(q[i], oracle.widen(1, kvh * hd, ks[:n]),
                                        oracle.widen(1, kvh * hd, vs[:n]), H, kvh, hd, n, scale)
            assert float(rel_err_rows(o[r], w, H, hd).max()) <= 1e-3, (i, n)


def test_noalloc_decode_refuses_a_shape_beyond_its_scratch(gi, oracle, dev):
    """A sequence is cut into splits until there is about one workgroup per
    CU: with 253 sequences x 1 kv head that is 2 splits each, 506 partial
    slots of 16 heads x (128 + 2) floats, 4.21 MB, beyond the fixed 4 MiB
    scratch, and the call is refused before any launch.  (The refusal comes
    before the block tables are read; the rows repeat one sequence.)"""
    import torch
    H, kvh, hd, P = 16, 1, 128, 16
    pop = Populated(gi, dev, 1, 1, kvh, hd, P, [1100], seed=43)
    if torch.cuda.get_device_properties(dev).multi_processor_count != 256:
        pytest.skip("the refused shape is worked out for a 256-CU device")
    B = 253
    bt = pop.block_tables()[torch.zeros(B, dtype=torch.long, device=dev)].contiguous()
    sl = torch.full((B,), 1100, dtype=torch.int32, device=dev)
    q = torch.zeros((B, H * hd), device=dev)
    out = torch.zeros_like(q)
    with pytest.raises(gi.GIError) as e:
        pop.pool.AttentionGQANoAlloc(out, q, 0, bt, sl, H, oracle.attn_scale(hd))
    assert e.value.code == -3 and "scratch" in str(e.value)
    # one sequence fewer: 252 x 1 kv head, 504 slots, 4.19 MB, fits and
    # matches the allocating entry point
    want = torch.full_like(out[:252], float("nan"))
    got = torch.full_like(out[:252], float("nan"))
    args = (q[:252].contiguous(), 0, bt[:252].contiguous(), sl[:252].contiguous(), H, oracle.attn_scale(hd))
    pop.pool.AttentionGQA(want, *args)
    pop.pool.AttentionGQANoAlloc(got, *args)
    pop.pool.synchronize()
    assert torch.equal(got, want)


def test_noalloc_decode_orders_two_handles_on_two_streams(gi, oracle, dev):
    """Two pools on two streams share the device's scratch array.  Calls
    alternate between them with no host synchronisation in between, each
    with split sequences (partials in the array), and every output must
    equal the allocating entry point's bit for bit: the library makes each
    stream wait for the previous user's launches on the other stream."""
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    scale = oracle.attn_scale(hd)
    pops, args, want = [], [], []
    for t, lens in enumerate(([20000, 9000, 4097], [12000, 3000])):
        pop = Populated(gi, dev, 1, 1, kvh, hd, P, lens, seed=51 + t)
        s = torch.cuda.Stream(dev)
        pop.pool.set_stream(s.cuda_stream)
        bt = pop.block_tables()
        sl = torch.tensor(lens, dtype=torch.int32, device=dev)
        qd, _ = seeded((len(lens), H * hd), 61 + t, dev)
        w = torch.full_like(qd, float("nan"))
        torch.cuda.synchronize()
        pop.pool.AttentionGQA(w, qd, 0, bt, sl, H, scale)
        pop.pool.synchronize()
        pops.append(pop)
        args.append((qd, bt, sl))
        want.append(w)
    outs = [(t, torch.full_like(args[t][0], float("nan"))) for _ in range(3) for t in (0, 1)]
    torch.cuda.synchronize()
    for t, got in outs:
        qd, bt, sl = args[t]
        pops[t].pool.AttentionGQANoAlloc(got, qd, 0, bt, sl, H, scale)
    for pop in pops:
        pop.pool.synchronize()
    for i, (t, got) in enumerate(outs):
        assert torch.equal(got, want[t]), (i, t)
