"""The decode and prefill entry points captured in one HIP graph.

A serving loop of tiny launches (one sequence, 22 layers x 128 tokens)
is bound by host time, so callers capture the step once and replay it.
The entry points allocate nothing once the decode workspace is sized and
record no memset, so the graph holds only their kernels.  Every replay
must give the eager outputs bit for bit, with eager work of the program
and synchronisations between the replays, and the eager outputs are
checked against the oracle (decode: forward.go:236-267, prefill:
forward.go:547-577) to the usual tolerance."""
import numpy as np
import pytest

from gpu_util import Populated, rel_err_rows, seeded

pytestmark = pytest.mark.gpu

TOL = {0: 1e-5, 1: 1e-3, 2: 1e-3, 3: 1e-3}


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3])
def test_decode_and_prefill_graph_replays(gi, oracle, dev, kv_type):
    import torch
    H, kvh, hd, P, C = 32, 8, 128, 16, 64
    # 1100 tokens take two splits and the merge kernel; 70 is a ragged
    # tail.
    lens = [300, 70, 1100]
    pop = Populated(gi, dev, kv_type, 2, kvh, hd, P, lens, seed=11 + kv_type)
    stream = torch.cuda.Stream(dev)
    pop.pool.set_stream(stream.cuda_stream)
    bt = pop.block_tables()
    B, kv_dim = len(lens), kvh * hd
    scale = oracle.attn_scale(hd)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    start = torch.tensor([n - C for n in lens], dtype=torch.int32, device=dev)
    # The decode step re-appends each sequence's last token with its own
    # values, so every replay rewrites the same bits.
    kd = torch.from_numpy(np.stack([pop.k[(0, i)][n - 1] for i, n in enumerate(lens)])).to(dev)
    vd = torch.from_numpy(np.stack([pop.v[(0, i)][n - 1] for i, n in enumerate(lens)])).to(dev)
    qd, q = seeded((B, H * hd), 501 + kv_type, dev)
    qp, qp_h = seeded((B, C, H * hd), 601 + kv_type, dev)
    od = torch.empty((B, H * hd), device=dev)
    op = torch.empty((B, C, H * hd), device=dev)

    def step():
        pop.pool.DecodeStep(od, qd, kd, vd, 0, bt, sl, H, scale, max_seq_len=max(lens))
        pop.pool.AttentionGQABatch(op, qp, 1, bt, start, H, scale, C)

    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    ref_d, ref_p = od.clone(), op.clone()

    want_d = np.zeros((B, H * hd), np.float32)
    for i, n in enumerate(lens):
        ks, vs = pop.stored(0, i)
        kw = oracle.widen(kv_type, kv_dim, ks[:n])
        vw = oracle.widen(kv_type, kv_dim, vs[:n])
        want_d[i] = oracle.attention_decode(q[i], kw, vw, H, kvh, hd, n, scale)
    assert float(rel_err_rows(ref_d.cpu().numpy(), want_d, H, hd).max()) <= TOL[kv_type]
    got_p = ref_p.cpu().numpy()
    for i, n in enumerate(lens):
        ks, vs = pop.stored(1, i)
        kw = oracle.widen(kv_type, kv_dim, ks[:n])
        vw = oracle.widen(kv_type, kv_dim, vs[:n])
        want = oracle.attention_prefill(qp_h[i], kw, vw, H, kvh, hd, n - C, C, 1 << 30, scale)
        assert float(rel_err_rows(got_p[i], want, H, hd).max()) <= TOL[kv_type], (i, n)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    other = torch.empty_like(od)
    for r in range(4):
        od.fill_(float("nan"))
        op.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(od, ref_d), ("decode replay", r)
        assert torch.equal(op, ref_p), ("prefill replay", r)
        # eager work of the program between replays, on the same pool
        with torch.cuda.stream(stream):
            pop.pool.AttentionGQA(other, qd * 0.5, 0, bt, sl, H, scale, max(lens))
            other.mul_(2.0).add_(1.0)
        torch.cuda.synchronize()


def test_workspace_growth_keeps_captured_graphs_valid(gi, oracle, dev):
    """The decode workspace (the partials of split sequences) grows with the
    batch and with the query heads per kv head.  A graph captured with 3
    sequences must keep replaying bit for bit after an eager call with 24
    sequences grew it (the buffers the graph holds stay alive), and a call
    that would need it to grow while the stream captures (24 sequences with
    twice the heads per kv head) is refused (GI_ERR_BAD_ARG) without
    synchronising or freeing anything; the first graph still replays
    afterwards."""
    import torch
    H, kvh, hd, P = 32, 8, 128, 16
    lens = [300, 70, 1100]
    pop = Populated(gi, dev, 1, 1, kvh, hd, P, lens, seed=31)
    stream = torch.cuda.Stream(dev)
    pop.pool.set_stream(stream.cuda_stream)
    bt = pop.block_tables()
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    qd, q = seeded((3, H * hd), 32, dev)
    od = torch.empty((3, H * hd), device=dev)
    scale = oracle.attn_scale(hd)

    def step():
        pop.pool.AttentionGQA(od, qd, 0, bt, sl, H, scale, max(lens))

    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    ref = od.clone()
    want = np.zeros((3, H * hd), np.float32)
    for i, n in enumerate(lens):
        ks, vs = pop.stored(0, i)
        want[i] = oracle.attention_decode(q[i], oracle.widen(1, kvh * hd, ks),
                                          oracle.widen(1, kvh * hd, vs), H, kvh, hd, n, scale)
    assert float(rel_err_rows(ref.cpu().numpy(), want, H, hd).max()) <= 1e-3

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()

    def replay_matches(tag):
        od.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(od, ref), tag

    replay_matches("first replay")
    # eager call with 24 rows and no length hint: 2 splits of 24 x 8
    # (sequence, kv head) pairs (fewer pairs than CUs), 8x the partials of
    # the captured call
    big = 24
    bt_big = bt[torch.arange(big, device=dev) % 3].contiguous()
    sl_big = sl[torch.arange(big, device=dev) % 3].contiguous()
    q_big = qd[torch.arange(big, device=dev) % 3].contiguous()
    o_big = torch.empty((big, H * hd), device=dev)
    with torch.cuda.stream(stream):
        pop.pool.AttentionGQA(o_big, q_big, 0, bt_big, sl_big, H, scale, 0)
    torch.cuda.synchronize()
    pop.pool.synchronize()
    got = o_big.cpu().numpy()
    for r in range(big):
        assert float(rel_err_rows(got[r], want[r % 3], H, hd).max()) <= 1e-3, r
    replay_matches("replay after growth")
    # growth while capturing is refused: 64 query heads (8 per kv head)
    # double the partials of the 24-row call
    q64 = torch.zeros((big, 2 * H * hd), device=dev)
    o64 = torch.empty_like(q64)
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(gi.GIError) as e:
        with torch.cuda.graph(g2, stream=stream):
            o64.fill_(0.0)
            pop.pool.AttentionGQA(o64, q64, 0, bt_big, sl_big, 2 * H, scale, 0)
    assert e.value.code == -3
    assert "capturing" in str(e.value)
    torch.cuda.synchronize()
    replay_matches("replay after the refused capture")
