"""Pins the oracle (oracle/cpu_ref.c) independently of its own code.

Each check is chosen so that a plausible slip in the restatement (round to
nearest instead of truncating, half-to-even instead of half-away, a dropped
scale re-quantisation, a wrong GQA head index, a reordered sum) fails it:
  * the reference's own known-answer tests for this path, restated
    (pkg/quant/quant_test.go:10-19, 129-143; pkg/engine/engine_test.go:
    194-217, 219-249, 251-273; pkg/math/kernels_test.go:23-37;
    pkg/engine/paged_kv_test.go:7-40);
  * closed forms: numpy's IEEE conversions adjusted to round-toward-zero,
    exact float64 textbook attention, exact bit patterns;
  * hand-built special cases with known answers.
"""
import numpy as np
import pytest


def f32bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def d16(b):
    """Little-endian fp16 scale bits of a 34-byte Q8_0 block."""
    return int(b[0]) | (int(b[1]) << 8)


# ---- fp16 conversions (pkg/quant/fp16.go) -----------------------------------

def test_fp16_to_fp32_all_halves(oracle):
    h = np.arange(65536, dtype=np.uint16)
    got = oracle.fp16_to_fp32(h)
    want = h.view(np.float16).astype(np.float32)   # IEEE exact widening
    assert np.array_equal(f32bits(got), f32bits(want))


def rtz_half_closed_form(x):
    """Round-toward-zero float32 -> fp16 bits from numpy's round-to-nearest:
    step one ulp toward zero where rounding went away from zero.  Overflow
    rule of fp16.go:53-57: exponent >= 31 (|x| >= 65536) -> Inf, so
    [65504, 65536) truncates to 65504.  NaN -> sign|0x7E00."""
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        r = x.astype(np.float16)
    rb = r.view(np.uint16).astype(np.uint32)
    sign = (x.view(np.uint32) >> 16) & 0x8000
    ax = np.abs(x.astype(np.float64))
    ar = np.abs(r.astype(np.float64))
    away = np.isfinite(ar) & (ar > ax)
    mag = rb & 0x7FFF
    mag = np.where(away, mag - np.minimum(mag, 1), mag)
    big = np.isinf(ar) & np.isfinite(ax)
    mag = np.where(big & (ax < 65536.0), 0x7BFF, mag)
    mag = np.where(big & (ax >= 65536.0), 0x7C00, mag)
    mag = np.where(np.isnan(x), 0x7E00, mag)
    return (sign | mag).astype(np.uint16)


def test_fp32_to_fp16_closed_form(oracle):
    rng = np.random.default_rng(1)
    parts = [rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)]
    # every half and its float32 neighbours (the truncation boundaries)
    hb = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    for d in (-2, -1, 0, 1, 2):
        parts.append((hb.astype(np.int64) + d).clip(0, 2**32 - 1).astype(np.uint32))
    # overflow / underflow edges and specials
    edges = np.array([65504.0, 65519.0, 65520.0, 65535.99, 65536.0, 1e30, 2.0**-24, 2.0**-25,
                      1.5 * 2.0**-25, 2.0**-26, 0.0, np.inf, np.nan, 1.0], np.float32)
    parts.append(edges.view(np.uint32))
    parts.append((-edges).view(np.uint32))
    bits = np.concatenate(parts)
    x = bits.view(np.float32)
    got = oracle.fp32_to_fp16(x)
    want = rtz_half_closed_form(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(bits[i]), hex(got[i]), hex(want[i])) for i in bad[:5]]


def test_fp16_known_answers(oracle):
    # truncation, not rounding: 1 + 2^-11 + 2^-12 rounds up to 1+2^-10 under
    # round-to-nearest but truncates to 1.0
    assert oracle.fp32_to_fp16(np.float32(1 + 2**-11 + 2**-12)) == 0x3C00
    assert oracle.fp32_to_fp16(np.float32(-(1 + 2**-11 + 2**-12))) == 0xBC00
    assert oracle.fp32_to_fp16(np.float32(65535.0)) == 0x7BFF   # no rounding up to Inf
    assert oracle.fp32_to_fp16(np.float32(65536.0)) == 0x7C00
    assert oracle.fp32_to_fp16(np.float32(np.nan)) == 0x7E00
    assert oracle.fp32_to_fp16(np.float32(2.0**-24)) == 0x0001
    assert oracle.fp32_to_fp16(np.float32(2.0**-25)) == 0x0000


def test_fp16_roundtrip_reference_case(oracle):
    # pkg/quant/quant_test.go:10-19
    for v in [0.0, 1.0, -1.0, 0.5, -0.5, 3.14159, 128.0, -0.001953125]:
        got = oracle.fp16_to_fp32(oracle.fp32_to_fp16(np.float32(v))).item()
        assert abs(got - v) <= 0.01 * abs(v) + 1e-4


# ---- Q8_0 (pkg/quant/quant.go) ----------------------------------------------

def q8_closed_form(x):
    """Q8_0 of one block from numpy IEEE float32 operations (each is
    correctly rounded, as Go's float32 arithmetic is) and the RTZ closed form
    above; rounding half away from zero done exactly in float64."""
    x = np.asarray(x, np.float32)
    ax = np.abs(x)
    ax = np.where(np.isnan(ax), np.float32(0), ax)
    amax = np.float32(ax.max()) if ax.size else np.float32(0)
    scale = np.float32(amax / np.float32(127.0))
    d16 = 0
    if scale > 0:
        d16 = int(rtz_half_closed_form(scale))
        scale = np.uint16(d16).view(np.float16).astype(np.float32)
    inv = np.float32(0)
    if scale > 0:
        with np.errstate(divide="ignore"):
            inv = np.float32(np.float32(1.0) / scale)
    q = np.zeros(32, np.int8)
    if inv > 0:
        with np.errstate(invalid="ignore", over="ignore"):
            v = (x * inv).astype(np.float32)
        v = np.where(v > 127, np.float32(127), np.where(v < -128, np.float32(-128), v))
        v64 = v.astype(np.float64)
        r = np.sign(v64) * np.floor(np.abs(v64) + 0.5)
        r = np.where(np.isnan(r), 0, r)
        q[:x.size] = r.astype(np.int64).astype(np.int8)
    out = np.zeros(34, np.uint8)
    out[0], out[1] = d16 & 0xFF, d16 >> 8
    out[2:] = q.view(np.uint8)
    return out


def test_q8_0_closed_form_random(oracle):
    rng = np.random.default_rng(7)
    for trial in range(300):
        scale = 10.0 ** rng.uniform(-9, 6)
        x = (rng.standard_normal(32) * scale).astype(np.float32)
        if trial % 5 == 0:
            x[rng.integers(0, 32)] *= 8  # outlier
        got = oracle.quantize_q8_0(x)
        assert np.array_equal(got, q8_closed_form(x)), trial


def test_q8_0_max_element_maps_to_127(oracle):
    # The fp16 scale is truncated, so amax/scale >= 127 and the largest
    # magnitude lands on the clamp: +127, or -127 for a negative maximum
    # (the clamp is at -128 but |v| < 127.2 while the scale is a normal half).
    rng = np.random.default_rng(3)
    for _ in range(200):
        x = (rng.standard_normal(32) * 10.0 ** rng.uniform(-2, 3)).astype(np.float32)
        b = oracle.quantize_q8_0(x)
        q = b[2:].view(np.int8)
        i = int(np.argmax(np.abs(x)))
        assert q[i] == (127 if x[i] > 0 else -127)
        assert 0x0400 <= d16(b) < 0x7C00   # normal half


def test_q8_0_special_cases(oracle):
    z = oracle.quantize_q8_0(np.zeros(32, np.float32))
    assert not z.any()
    # amax 127 -> scale exactly 1.0 (0x3C00): ties round away from zero
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2], x[3] = 127.0, 2.5, -2.5, 0.5
    b = oracle.quantize_q8_0(x)
    assert d16(b) == 0x3C00
    assert list(b[2:6].view(np.int8)) == [127, 3, -3, 1]
    # scale truncation: 100/127 = 0.7874016 -> 0x3A4C (round-to-nearest: 0x3A4D)
    x = np.zeros(32, np.float32)
    x[0] = 100.0
    b = oracle.quantize_q8_0(x)
    assert d16(b) == 0x3A4C
    # fp16 underflow of the scale -> d = 0 and every q = 0
    b = oracle.quantize_q8_0(np.full(32, 1e-6, np.float32))
    assert not b.any()
    # overflow -> d = Inf (0x7C00), inverse 0, q = 0
    x = np.ones(32, np.float32)
    x[5] = 1e7
    b = oracle.quantize_q8_0(x)
    assert d16(b) == 0x7C00 and not b[2:].any()
    # subnormal scale truncated from 1.9*2^-24 to 2^-24: -amax clamps at -128
    a = np.float32(127 * 1.9 * 2.0**-24)
    x = np.zeros(32, np.float32)
    x[0], x[1] = a, -a
    b = oracle.quantize_q8_0(x)
    assert d16(b) == 0x0001
    assert list(b[2:4].view(np.int8)) == [127, -128]
    # NaN is skipped by the max and quantises to 0
    x = np.arange(32, dtype=np.float32)
    x[4] = np.nan
    q = oracle.quantize_q8_0(x)[2:].view(np.int8)
    assert q[4] == 0 and q[31] == 127
    # a short final block is zero padded (QuantizeQ8_0 on 40 elements)
    b = oracle.quantize_q8_0(np.arange(1, 41, dtype=np.float32))
    assert b.size == 68 and not b[34 + 2 + 8:].any()


def test_q8_0_reference_tests(oracle):
    # pkg/quant/quant_test.go:129-143
    src = np.arange(64, dtype=np.float32) - 32
    deq = oracle.dequantize_q8_0(oracle.quantize_q8_0(src), 64)
    assert np.all(np.abs(src - deq) <= 0.5)
    # pkg/engine/engine_test.go:251-273 (Q8_0 KV, kvDim 32, k[i] = i)
    k = np.arange(32, dtype=np.float32)
    stored = oracle.store_vectors(oracle.KV_Q8_0, k[None, :])
    kr = oracle.widen(oracle.KV_Q8_0, 32, stored)[0]
    assert abs(kr[10] - 10.0) <= 0.5
    # pkg/quant/quant_test.go:55-83: dequant of hand-built blocks
    blk = np.zeros(34, np.uint8)
    blk[0], blk[1] = 0x00, 0x38          # 0.5
    blk[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    deq = oracle.dequantize_q8_0(blk, 32)
    assert np.array_equal(deq, (np.arange(32) - 16).astype(np.float32) * 0.5)


# ---- DotVecF32 / Softmax / scale ---------------------------------------------

def test_dot_vec_f32_chunk_order(oracle):
    # quant.go:548-567 adds each 8-wide chunk to the running sum; a
    # sequential float32 sum of the same products gives a different answer.
    x = np.zeros(16, np.float32)
    x[0] = 1e8
    x[8:] = 1.0
    w = np.ones(16, np.float32)
    assert oracle.dot_vec_f32(x, w) == np.float32(100000008.0)
    s = np.float32(0)
    for a, b in zip(x, w):
        s = np.float32(s + a * b)
    assert s == np.float32(1e8)
    # scalar tail after the chunks (n = 11)
    x = np.arange(11, dtype=np.float32)
    assert oracle.dot_vec_f32(x, x) == np.float32(385.0)


def test_softmax(oracle):
    # pkg/math/kernels_test.go:23-37
    s = oracle.softmax(np.array([1, 2, 3], np.float32))
    assert abs(float(s.sum()) - 1.0) <= 1e-5 and s[2] > s[1] > s[0]
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(1000) * 4).astype(np.float32)
    e = np.exp(x.astype(np.float64) - x.max())
    assert np.allclose(oracle.softmax(x), e / e.sum(), rtol=2e-6, atol=1e-9)
    assert oracle.softmax(np.array([], np.float32)).size == 0


def test_attn_scale_bits(oracle):
    # forward.go:33 with math_sqrt (forward.go:771-780)
    assert f32bits(oracle.attn_scale(64)) == 0x3E000000
    assert f32bits(oracle.attn_scale(128)) == 0x3DB504F3
    assert oracle.math_sqrt(0) == 0


# ---- attention (forward.go:242-267, 547-577) --------------------------------

def textbook_attention(q, kc, vc, H, KVH, hd, L, scale):
    """softmax(scale * q K^T) V in float64; q-head h reads kv head
    h // (H // KVH)."""
    G = H // KVH
    out = np.zeros((H, hd))
    q = q.reshape(H, hd).astype(np.float64)
    k = kc[:L].reshape(L, KVH, hd).astype(np.float64)
    v = vc[:L].reshape(L, KVH, hd).astype(np.float64)
    for h in range(H):
        s = k[:, h // G, :] @ q[h] * float(scale)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[:, h // G, :]
    return out.reshape(-1)


@pytest.mark.parametrize("H,KVH,hd,L", [(32, 4, 64, 200), (8, 2, 128, 77), (4, 4, 64, 1),
                                        (8, 1, 64, 33)])
def test_attention_decode_vs_textbook(oracle, H, KVH, hd, L):
    q = oracle.normal(11, (H * hd,))
    kc = oracle.normal(12, (L, KVH * hd))
    vc = oracle.normal(13, (L, KVH * hd))
    sc = oracle.attn_scale(hd)
    got = oracle.attention_decode(q, kc, vc, H, KVH, hd, L, sc)
    want = textbook_attention(q, kc, vc, H, KVH, hd, L, sc)
    assert np.max(np.abs(got - want)) <= 2e-6 * np.max(np.abs(want))


def test_prefill_equals_decode_per_token(oracle):
    # engine_test.go:219-249 (batch prefill == sequential decode) restated
    # on the attention step: query b of a chunk starting at start_pos sees
    # the same scores as a decode at position start_pos + b.
    H, KVH, hd, start, chunk = 8, 2, 64, 20, 12
    n = start + chunk
    kc = oracle.normal(21, (n, KVH * hd))
    vc = oracle.normal(22, (n, KVH * hd))
    q = oracle.normal(23, (chunk, H * hd))
    sc = oracle.attn_scale(hd)
    pre = oracle.attention_prefill(q, kc, vc, H, KVH, hd, start, chunk, 8192, sc)
    for b in range(chunk):
        dec = oracle.attention_decode(q[b], kc, vc, H, KVH, hd, start + b + 1, sc)
        assert np.array_equal(pre[b], dec)
    # ring cap of the contiguous cache (forward.go:550-553): max_seq bounds L
    capped = oracle.attention_prefill(q, kc, vc, H, KVH, hd, start, chunk, 25, sc)
    assert np.array_equal(capped[10], oracle.attention_decode(q[10], kc, vc, H, KVH, hd, 25, sc))


@pytest.mark.parametrize("threads", [2, 3, 8])
def test_threaded_oracle_is_bit_identical(oracle, threads):
    """The multi-threaded forms split (query, q-head) rows over threads
    (forward.go:1342-1378 splits heads over goroutines); each row is the
    one-thread computation, so every output bit must match, including the
    empty context and the ring cap."""
    H, KVH, hd = 16, 4, 64
    kc = oracle.normal(31, (300, KVH * hd))
    vc = oracle.normal(32, (300, KVH * hd))
    q = oracle.normal(33, (40, H * hd))
    sc = oracle.attn_scale(hd)
    for L in (0, 1, 17, 300):
        one = oracle.attention_decode(q[0], kc, vc, H, KVH, hd, L, sc)
        assert np.array_equal(one, oracle.attention_decode(q[0], kc, vc, H, KVH, hd, L, sc,
                                                           threads=threads))
    for start, chunk, cap in ((0, 40, 8192), (200, 40, 8192), (250, 40, 270)):
        one = oracle.attention_prefill(q, kc, vc, H, KVH, hd, start, chunk, cap, sc)
        mt = oracle.attention_prefill(q, kc, vc, H, KVH, hd, start, chunk, cap, sc,
                                      threads=threads)
        assert np.array_equal(one, mt)
    # batch decode from stored fp16 / q8_0 vectors, ragged lengths
    lens = np.array([300, 0, 5, 123], np.int32)
    off = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    for kt in (1, 2):
        ks = oracle.store_vectors(kt, oracle.normal(34, (int(lens.sum()), KVH * hd)))
        vs = oracle.store_vectors(kt, oracle.normal(35, (int(lens.sum()), KVH * hd)))
        qb = q[:lens.size]
        one = oracle.decode_batch(kt, qb, ks, vs, off, lens, H, KVH, hd, sc)
        mt, ran = oracle.decode_batch(kt, qb, ks, vs, off, lens, H, KVH, hd, sc, threads=threads)
        assert ran == threads
        assert np.array_equal(one, mt)
        assert not one[1].any()


# ---- KV store / paged pool -----------------------------------------------------

def test_kv_context_wrap(oracle):
    # pkg/engine/engine_test.go:194-217: maxSeq 4, 10 writes, slot 1 = pos 9
    kv_dim, max_seq = 8, 4
    kc = np.zeros((max_seq, 4 * kv_dim), np.uint8)
    vc = np.zeros_like(kc)
    lib = oracle.lib()
    import ctypes
    for pos in range(10):
        k = (pos * 10 + np.arange(kv_dim)).astype(np.float32)
        v = (pos * 100 + np.arange(kv_dim)).astype(np.float32)
        lib.ref_kv_write(0, kv_dim, max_seq, kc.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                         vc.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), pos % max_seq,
                         k.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                         v.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    assert kc[1].view(np.float32)[0] == 90.0 and vc[1].view(np.float32)[0] == 900.0


@pytest.mark.parametrize("kv_type", [0, 1, 2, 3])
def test_paged_store_gather_roundtrip(oracle, kv_type):
    layers, kv_dim, P, nb = 3, 64, 16, 12
    pool = oracle.RefPagedPool(kv_type, layers, kv_dim, nb, P)
    mgr = oracle.PagedKVManager(layers, kv_dim, nb, P)
    s1, s2 = mgr.AllocateSequence(), mgr.AllocateSequence()
    n1, n2 = 35, 50
    k1, v1 = oracle.normal(1, (n1, kv_dim)), oracle.normal(2, (n1, kv_dim))
    k2, v2 = oracle.normal(3, (n2, kv_dim)), oracle.normal(4, (n2, kv_dim))
    for sid, k, v in ((s1, k1, v1), (s2, k2, v2)):
        ids, slots = zip(*[mgr.AppendToken(sid) for _ in range(k.shape[0])])
        pool.store(1, np.array(ids, np.int32), np.array(slots, np.int32), k, v)
    for sid, k, v, n in ((s1, k1, v1, n1), (s2, k2, v2, n2)):
        ko, vo = pool.gather(1, mgr.Tables[sid]["BlockIDs"], n)
        assert np.array_equal(ko, oracle.store_vectors(kv_type, k))
        assert np.array_equal(vo, oracle.store_vectors(kv_type, v))


def test_allocator_reference_test_and_lifo(oracle):
    # pkg/engine/paged_kv_test.go:7-40 plus the LIFO closed form
    mgr = oracle.PagedKVManager(4, 64, 10, 16)
    s = mgr.AllocateSequence()
    assert s == 1
    got = [mgr.AppendToken(s) for _ in range(35)]
    assert [b for b, _ in got[:16]] == [9] * 16 and got[16][0] == 8 and got[32][0] == 7
    assert [sl for _, sl in got] == [i % 16 for i in range(35)]
    assert mgr.Tables[s]["BlockIDs"] == [9, 8, 7] and mgr.Tables[s]["NumTokens"] == 35
    mgr.FreeSequence(s)
    assert len(mgr.FreeBlocks) == 10 and mgr.FreeBlocks[-3:] == [9, 8, 7]
    with pytest.raises(oracle.UnknownSequence):
        mgr.AppendToken(s)
    s2 = mgr.AllocateSequence()
    for _ in range(160):
        mgr.AppendToken(s2)
    with pytest.raises(oracle.OutOfPages):
        mgr.AppendToken(s2)


def test_generator_is_counter_based(oracle):
    a = oracle.normal(99, (1000,))
    b = oracle.normal(99, (500,), offset=500)
    assert np.array_equal(a[500:], b)
    assert abs(float(a.mean())) < 0.1 and abs(float(a.std()) - 1) < 0.1
    x = oracle.normal_with_outliers(5, (100000,))
    frac = float(np.mean(np.abs(x) == 8.0))
    assert 0.008 < frac < 0.012


@pytest.mark.parametrize("kv_type", [0, 2])
def test_kvcache_clone_and_fork_reference_test(oracle, kv_type):
    # pkg/engine/kvcache_test.go:7-71 on the restated KVCache (f32 and q8_0)
    c = oracle.RefKVCache(kv_type, 2, 64, 16)
    c.CurPos = 4
    k = np.arange(1, 65, dtype=np.float32)
    v = k * 2
    c.Write(0, 0, k, v)
    c.Write(1, 1, k, v)
    clone = c.Clone()
    assert clone.CurPos == 4
    got_k = oracle.widen(kv_type, 64, clone.K[0, 0:1])
    want_k = oracle.widen(kv_type, 64, oracle.store_vectors(kv_type, k[None]))
    assert np.array_equal(got_k, want_k)
    if kv_type == 0:
        assert got_k[0, 0] == 1.0 and oracle.widen(0, 64, clone.V[0, 0:1])[0, 0] == 2.0
    forked = c.ForkAt(1)
    assert np.array_equal(forked.K[0, 0], c.K[0, 0])
    assert not forked.K[1, 1].any()  # slot 1 is past maxSlot: not copied
    newk = np.zeros(64, np.float32)
    newk[0] = 999.0
    clone.Write(0, 0, newk, newk)
    assert oracle.widen(kv_type, 64, c.K[0, 0:1])[0, 0] != 999.0
    # out-of-range writes are ignored (kvcache.go:147-149)
    before = c.K.copy()
    c.Write(5, 0, k, v)
    c.Write(0, 16, k, v)
    assert np.array_equal(before, c.K)


def test_prefix_cache_reference_tests(oracle):
    # pkg/engine/prefix_cache_test.go:7-47 on the restated PrefixCache
    pc = oracle.RefPrefixCache(10)
    kv = oracle.RefKVCache(0, 4, 64, 128)
    for l in range(4):
        for t in range(10):
            vals = np.arange(t * 64 + 1, t * 64 + 65, dtype=np.float32)
            kv.Write(l, t, vals, vals + 1)
    pc.Store([101, 202, 303, 404, 505], kv.Clone())
    n, got = pc.FindLongestPrefix([101, 202, 303, 404, 505, 606, 707])
    assert n == 5 and got is not None
    assert np.array_equal(got.K[0, 0], kv.K[0, 0])
    assert pc.FindLongestPrefix([999, 888, 777]) == (0, None)
    # short lists are not stored; a full cache drops one entry first
    pc2 = oracle.RefPrefixCache(2)
    pc2.Store([1, 2, 3], kv)
    assert len(pc2.entries) == 0
    pc2.Store([1, 2, 3, 4], kv)
    pc2.Store([1, 2, 3, 4, 5], kv)
    pc2.Store([5, 6, 7, 8], kv)
    assert len(pc2.entries) == 2 and (1, 2, 3, 4) not in pc2.entries
    # the longest stored prefix wins; a query equal to a key does not match it
    assert pc2.FindLongestPrefix([1, 2, 3, 4, 5, 6])[0] == 5
    assert pc2.FindLongestPrefix([1, 2, 3, 4, 5])[0] == 0
    assert oracle.RefPrefixCache(0).max_size == 32
