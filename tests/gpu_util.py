"""Shared set-up for the GPU parity tests: seeded inputs, pools populated
through the C ABI, and the oracle's view of the same sequences."""
import numpy as np


def seeded(shape, seed, dev, outliers=False):
    """float32 N(0,1) tensor on dev from the oracle's counter-based
    generator (so the CPU side can regenerate it), optionally with 1 %
    outliers at +-8 sigma."""
    import torch
    import oracle
    if outliers:
        x = oracle.normal_with_outliers(seed, shape)
    else:
        x = oracle.normal(seed, shape)
    return torch.from_numpy(x).to(dev), x


def with_specials(x, kv_type, rng):
    """Plants values that exercise the conversion edges: NaN, Inf, huge,
    tiny and subnormal inputs, exact ties."""
    x = x.copy()
    flat = x.reshape(-1)
    n = flat.size
    specials = np.array([np.nan, np.inf, -np.inf, 70000.0, -65519.0, 65504.0, 1e-8, -3e-8,
                         1e-40, -1e-45, 0.0, -0.0, 2.5, 1 + 2**-11 + 2**-12], np.float32)
    idx = rng.choice(n, size=min(n, 4 * specials.size), replace=False)
    flat[idx] = np.resize(specials, idx.size)
    if kv_type in (2, 3):
        # whole Q8_0 / Q4_0 blocks that are all zero, tiny (scale underflow) or huge
        nb = n // 32
        for j, val in zip(rng.choice(nb, size=min(nb, 3), replace=False), (0.0, 1e-7, 1e9)):
            flat[32 * j:32 * j + 32] = val
    return x


class Populated:
    """A pool with several sequences appended through the C ABI.

    Block ids come from the C++ PagedKVManager started from a shuffled free
    list, so tables are fragmented; K/V are appended chunk by chunk in
    token order for every layer."""

    def __init__(self, gi, dev, kv_type, layers, kvh, hd, P, lens, seed, slack_pages=3,
                 specials=False, append_chunk=None, outliers=False):
        import torch
        self.gi, self.dev = gi, dev
        self.kv_type, self.layers, self.kvh, self.hd, self.P = kv_type, layers, kvh, hd, P
        self.kv_dim = kvh * hd
        self.lens = list(lens)
        pages = sum((n + P - 1) // P for n in self.lens) + slack_pages
        rng = np.random.default_rng(seed)
        self.mgr = gi.PagedKVManager(layers, self.kv_dim, pages, P)
        self.mgr.SetFreeList(rng.permutation(pages).astype(np.int32))
        self.pool = gi.PagedKVCache(layers, kvh, hd, P, pages, kv_type)
        self.seqs = [self.mgr.AllocateSequence() for _ in self.lens]
        self.k = {}  # (layer, seq index) -> float32 numpy [n, kv_dim]
        self.v = {}
        ids_all = []
        for i, (sid, n) in enumerate(zip(self.seqs, self.lens)):
            ids, slots = self.mgr.AppendTokens(sid, n)
            ids_all.append((ids, slots))
        for l in range(layers):
            for i, n in enumerate(self.lens):
                if n == 0:
                    self.k[(l, i)] = np.zeros((0, self.kv_dim), np.float32)
                    self.v[(l, i)] = np.zeros((0, self.kv_dim), np.float32)
                    continue
                s0 = seed * 1000003 + l * 7919 + i * 104729
                _, k = seeded((n, self.kv_dim), s0, "cpu", outliers)
                _, v = seeded((n, self.kv_dim), s0 + 1, "cpu", outliers)
                if specials:
                    k = with_specials(k, kv_type, rng)
                    v = with_specials(v, kv_type, rng)
                self.k[(l, i)], self.v[(l, i)] = k, v
                ids, slots = ids_all[i]
                step = append_chunk or n
                for a in range(0, n, step):
                    b = min(n, a + step)
                    self.pool.Write(l, torch.from_numpy(ids[a:b].copy()).to(dev),
                                    torch.from_numpy(slots[a:b].copy()).to(dev),
                                    torch.from_numpy(k[a:b].copy()).to(dev),
                                    torch.from_numpy(v[a:b].copy()).to(dev))
        self.pool.synchronize()
        self.max_blocks = max(1, max((n + P - 1) // P for n in self.lens))

    def table(self, i):
        return np.array(self.mgr.Tables[self.seqs[i]].BlockIDs, np.int32)

    def block_tables(self):
        import torch
        bt = np.zeros((len(self.seqs), self.max_blocks), np.int32)
        for i in range(len(self.seqs)):
            t = self.table(i)
            bt[i, :t.size] = t
        return torch.from_numpy(bt).to(self.dev)

    def stored(self, l, i):
        """Oracle's stored bytes for sequence i, layer l."""
        import oracle
        return (oracle.store_vectors(self.kv_type, self.k[(l, i)]),
                oracle.store_vectors(self.kv_type, self.v[(l, i)]))


def rel_err_rows(got, want, H, hd):
    """max |got - want| / max |want| per (query, head) row; the relative
    error definition the tolerances below use."""
    g = np.asarray(got, np.float64).reshape(-1, hd)
    w = np.asarray(want, np.float64).reshape(-1, hd)
    den = np.maximum(np.abs(w).max(axis=1), 1e-30)
    return np.abs(g - w).max(axis=1) / den
