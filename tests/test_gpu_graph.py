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
    # 1100 tokens take two splits and the merge kernel; 70 is a ragged tail.
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
