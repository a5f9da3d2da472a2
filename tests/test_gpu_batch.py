"""GPU parity of the continuous-batching decode driver (gi_batch_*): a
running set of sequences with joins, leaves and copy-on-write forks, each step
one token per sequence and, per layer, RoPE + append + paged attention
(forward.go:228-267) for the whole set.

Model: per sequence and layer, the list of K vectors after ApplyRoPE
(pkg/math/kernels.go:22-35) at their positions and the V vectors; a fork
copies its parent's first n entries.  Each step the rotated q must equal the
oracle's bit for bit, and every row's attention must match the oracle fed
the model's stored bits within 1e-5 (f32 KV) / 1e-3 (f16 / q8_0 / q4_0 KV),
max|gpu - oracle| <= tol * max|oracle| per (row, head).  At the end every live
sequence's pages must hold exactly the model's stored bytes."""
import random

import numpy as np
import pytest

from gpu_util import rel_err_rows

pytestmark = pytest.mark.gpu

TOL = {0: 1e-5, 1: 1e-3, 2: 1e-3, 3: 1e-3}


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3], ids=["f32", "f16", "q8_0", "q4_0"])
def test_batch_driver_decode(gi, oracle, dev, kv_type):
    import torch
    H, kvh, hd, P, layers, theta = 8, 2, 128, 16, 2, 500000.0
    kv_dim = kvh * hd
    pages, max_batch, max_blocks = 96, 8, 32
    rng = random.Random(21 + kv_type)
    mgr = gi.PagedKVManager(layers, kv_dim, pages, P)
    mgr.SetFreeList(np.random.default_rng(kv_type).permutation(pages).astype(np.int32))
    pool = gi.PagedKVCache(layers, kvh, hd, P, pages, kv_type)
    pool.SetRoPE(theta, 0, max_blocks * P)
    drv = gi.BatchDecoder(mgr, pool, max_batch, max_blocks)
    model = {}          # sid -> {"K": [layer][list of rows], "V": ...}
    rows = []
    seed = [1000 * kv_type]

    def nrm(shape):
        seed[0] += 1
        return oracle.normal(seed[0], shape)

    def join(n):
        sid = mgr.AllocateSequence()
        model[sid] = {"K": [[] for _ in range(layers)], "V": [[] for _ in range(layers)]}
        if n:
            ids, slots = mgr.AppendTokens(sid, n)
            pos = np.arange(n, dtype=np.int32)
            for l in range(layers):
                k, v = nrm((n, kv_dim)), nrm((n, kv_dim))
                pool.RoPEWrite(l, torch.from_numpy(pos).to(dev), torch.from_numpy(ids).to(dev),
                               torch.from_numpy(slots).to(dev), None, torch.from_numpy(k).to(dev),
                               torch.from_numpy(v).to(dev))
                model[sid]["K"][l] += list(oracle.rope_heads(k, pos, kvh, hd, 0, theta))
                model[sid]["V"][l] += list(v)
        drv.Add(sid)
        rows.append(sid)

    for n in (1, 15, 16, 40, 130):
        join(n)
    worst, forks, steps_checked = 0.0, 0, 0
    for step in range(24):
        if step in (4, 15):
            join(rng.randrange(5, 60))
        if step in (7, 12):                       # fork a running sequence mid-page
            src = rows[rng.randrange(len(rows))]
            n = mgr.Tables[src].NumTokens
            cut = n - 1 - (n % P == 0)
            f = mgr.ForkSequence(src, cut)
            model[f] = {"K": [list(x[:cut]) for x in model[src]["K"]],
                        "V": [list(x[:cut]) for x in model[src]["V"]]}
            drv.Add(f)
            rows.append(f)
            forks += 1
        if step == 10:                            # a sequence finishes
            sid = rows[1]
            drv.Remove(sid)
            rows[1] = rows[-1]
            rows.pop()
            mgr.FreeSequence(sid)
            del model[sid]
        n_rows = drv.Step()
        ids, lens = drv.Rows()
        assert list(ids) == rows and n_rows == len(rows)
        for l in range(layers):
            q, k, v = nrm((n_rows, H * hd)), nrm((n_rows, kv_dim)), nrm((n_rows, kv_dim))
            qd = torch.from_numpy(q).to(dev)
            out = torch.full((n_rows, H * hd), float("nan"), device=dev)
            drv.DecodeLayer(l, H, qd, torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev), out,
                            oracle.attn_scale(hd), rope=True)
            pos = lens.astype(np.int32) - 1
            kr = oracle.rope_heads(k, pos, kvh, hd, 0, theta)
            for r, sid in enumerate(rows):
                model[sid]["K"][l].append(kr[r])
                model[sid]["V"][l].append(v[r])
            pool.synchronize()
            qr = oracle.rope_heads(q, pos, H, hd, 0, theta)
            assert np.array_equal(qd.cpu().numpy().view(np.uint32), qr.view(np.uint32)), (step, l)
            if step % 3 == 0 or step in (7, 8, 12, 13):
                got = out.cpu().numpy()
                for r, sid in enumerate(rows):
                    L = int(lens[r])
                    ks = oracle.store_vectors(kv_type, np.stack(model[sid]["K"][l]))
                    vs = oracle.store_vectors(kv_type, np.stack(model[sid]["V"][l]))
                    assert ks.shape[0] == L
                    want = oracle.attention_decode(qr[r], oracle.widen(kv_type, kv_dim, ks),
                                                   oracle.widen(kv_type, kv_dim, vs), H, kvh, hd, L,
                                                   oracle.attn_scale(hd))
                    worst = max(worst, float(rel_err_rows(got[r], want, H, hd).max()))
                steps_checked += 1
    assert forks == 2 and steps_checked > 8
    print("batch driver max rel err", worst, flush=True)
    assert worst <= TOL[kv_type], worst
    # every live sequence's pages hold the model's bytes, every layer
    ids, lens = drv.Rows()
    for r, sid in enumerate(rows):
        t = torch.from_numpy(drv.RowTable(r)).to(dev)
        assert list(drv.RowTable(r)) == list(mgr.Tables[sid].BlockIDs)
        for l in range(layers):
            ko, vo = pool.Get(l, t, int(lens[r]))
            pool.synchronize()
            assert np.array_equal(ko.cpu().numpy(), oracle.store_vectors(kv_type, np.stack(model[sid]["K"][l])))
            assert np.array_equal(vo.cpu().numpy(), oracle.store_vectors(kv_type, np.stack(model[sid]["V"][l])))
    drv.close()
