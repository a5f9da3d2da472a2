"""Writes the golden fixtures of this directory from the oracle.

    python tests/golden/make_golden.py

The reference is Go and cannot run here, and its tests hold no fixture
files, so these vectors come from the oracle (oracle/cpu_ref.c), after it was
pinned against the reference's known-answer tests and the closed forms in
tests/test_oracle*.py.  They freeze its outputs: tests/test_golden.py checks
that the oracle still reproduces them bit for bit, and tests/test_gpu_golden.py
checks the HIP path against them on the GPU.  Inputs come from the oracle's
counter-based generator (SplitMix64 -> Box-Muller), with planted edge values.

Fixtures (numpy .npz, no pickles):
  quant.npz    token vectors with special values -> FP32ToFP16 halves,
               QuantizeQ8_0 and QuantizeQ4_0 blocks and their dequantised
               floats;
  rope.npz     q / k heads at assorted positions -> ApplyRoPE outputs (full and
               partial rotary) and the (cos, sin) rows;
  attn.npz     small decode and chunked-prefill cases per kv type: stored K/V
               bytes and the oracle's attention outputs;
  alloc.npz    a PagedKVManager operation sequence -> block tables and free
               lists after each step.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

SPECIALS = np.array([np.nan, np.inf, -np.inf, 70000.0, -65519.0, 65504.0, 1e-8, -3e-8, 1e-40,
                     -1e-45, 0.0, -0.0, 2.5, 1 + 2 ** -11 + 2 ** -12, 7.0, -7.5], np.float32)


def quant_vectors():
    n_tok, kv_dim = 24, 256
    x = oracle.normal_with_outliers(101, (n_tok, kv_dim))
    flat = x.reshape(-1)
    idx = np.random.default_rng(5).choice(flat.size, 4 * SPECIALS.size, replace=False)
    flat[idx] = np.resize(SPECIALS, idx.size)
    for j, val in zip((3, 17, 40), (0.0, 1e-7, 1e9)):       # whole blocks
        flat[32 * j:32 * j + 32] = val
    x[5] *= 1e-3                                             # small-scale rows
    x[6] *= 300.0
    out = {"x": x}
    for name, kt in (("f16", oracle.KV_F16), ("q8_0", oracle.KV_Q8_0), ("q4_0", oracle.KV_Q4_0)):
        st = oracle.store_vectors(kt, x)
        out["stored_" + name] = st
        out["widened_" + name] = oracle.widen(kt, kv_dim, st)
    return out


def rope_vectors():
    out = {}
    for name, (H, hd, rd, theta) in {"llama8b": (4, 128, 128, 500000.0),
                                     "tinyllama": (4, 64, 64, 10000.0),
                                     "partial": (4, 128, 64, 1000000.0)}.items():
        pos = np.array([0, 1, 2, 15, 16, 255, 4095, 8191, 32767, 131071], np.int32)
        x = oracle.normal(202 + hd + rd, (pos.size, H * hd))
        out[name + "_x"] = x
        out[name + "_pos"] = pos
        out[name + "_shape"] = np.array([H, hd, rd], np.int32)
        out[name + "_theta"] = np.float32(theta)
        out[name + "_y"] = oracle.rope_heads(x, pos, H, hd, rd, theta)
        out[name + "_table"] = np.stack([oracle.rope_table(theta, rd, int(p), 1)[0] for p in pos])
    return out


def attn_vectors():
    """Decode: H=8 q heads over 2 kv heads of 128 (group 4), 40 tokens;
    prefill: a 12-query chunk starting at 28.  One case per kv type (f32
    stored bytes are the inputs' own bits and are not repeated)."""
    H, kvh, hd, L = 8, 2, 128, 40
    kv_dim = kvh * hd
    scale = oracle.attn_scale(hd)
    out = {"shape": np.array([H, kvh, hd, L], np.int32), "scale": np.float32(scale)}
    k = oracle.normal_with_outliers(303, (L, kv_dim))
    v = oracle.normal_with_outliers(304, (L, kv_dim))
    q = oracle.normal(305, (H * hd,))
    qp = oracle.normal(306, (12, H * hd))
    out.update(k=k, v=v, q=q, q_prefill=qp)
    for name, kt in (("f32", 0), ("f16", 1), ("q8_0", 2), ("q4_0", 3)):
        ks = oracle.store_vectors(kt, k)
        vs = oracle.store_vectors(kt, v)
        kw = oracle.widen(kt, kv_dim, ks)
        vw = oracle.widen(kt, kv_dim, vs)
        if kt != 0:
            out["ks_" + name] = ks
            out["vs_" + name] = vs
        out["decode_" + name] = oracle.attention_decode(q, kw, vw, H, kvh, hd, L, scale)
        out["prefill_" + name] = oracle.attention_prefill(qp, kw, vw, H, kvh, hd, L - 12, 12,
                                                          1 << 30, scale)
    return out


def alloc_vectors():
    """PagedKVManager (paged_kv.go:49-148) restated: 6 blocks of 4 tokens;
    allocate two sequences, append, free the first, append to the second
    until the pool is exhausted."""
    m = oracle.PagedKVManager(2, 64, 6, 4)
    a, b = m.AllocateSequence(), m.AllocateSequence()
    ops, tables, frees, results = [], [], [], []

    def snap():
        tables.append([list(m.Tables.get(s, {"BlockIDs": []})["BlockIDs"]) + [-1] * (6 - len(
            m.Tables.get(s, {"BlockIDs": []})["BlockIDs"])) for s in (a, b)])
        frees.append(list(m.FreeBlocks) + [-1] * (6 - len(m.FreeBlocks)))

    for sid, n in ((a, 5), (b, 3)):
        for _ in range(n):
            results.append(m.AppendToken(sid))
            ops.append((0, sid))
            snap()
    m.FreeSequence(a)
    ops.append((1, a))
    results.append((-1, -1))
    snap()
    while True:
        try:
            results.append(m.AppendToken(b))
        except oracle.OutOfPages:
            results.append((-4, -4))
            ops.append((0, b))
            snap()
            break
        ops.append((0, b))
        snap()
    return {"ops": np.array(ops, np.int32), "results": np.array(results, np.int32),
            "tables": np.array(tables, np.int32), "free": np.array(frees, np.int32)}


BUILDERS = {"quant": quant_vectors, "rope": rope_vectors, "attn": attn_vectors,
            "alloc": alloc_vectors}


def main():
    for name, fn in BUILDERS.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
