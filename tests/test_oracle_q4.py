"""Pins the oracle's Q4_0 (pkg/quant/quant.go:96-116 DequantizeQ4_0,
458-521 QuantizeQ4_0, the KV type of pkg/engine/kvcache.go:99-105, 162-171,
198-206):

  * an independent numpy float32 form of the quantiser on random blocks over
    many decades (numpy's own IEEE division and rounding; the fp16
    truncation is the oracle's FP32ToFP16, pinned exhaustively elsewhere);
  * quant_test.go:21-54 (hand-made blocks, nibble 5 -> -3, 12 -> +4),
    quant_test.go:145-160 (|deq - src| <= 4) and engine_test.go:275-297
    (|deq[10] - 10| <= 3) restated;
  * hand-built cases: ties round away from zero, the max element lands on
    nibble 15 or 1, a zero block, an Inf block, NaN elements, a subnormal
    scale that drives the clamps, a short final block."""
import numpy as np
import pytest


def numpy_q4_0(oracle, x):
    """QuantizeQ4_0 in numpy float32 arithmetic, block by block."""
    x = np.asarray(x, np.float32)
    n = x.size
    nb = (n + 31) // 32
    out = np.zeros(nb * 18, np.uint8)
    for b in range(nb):
        blk = x[32 * b:32 * b + 32]
        a = np.abs(blk)
        a = a[~np.isnan(a)]
        amax = np.float32(a.max()) if a.size else np.float32(0)
        with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
            scale = np.float32(amax / np.float32(7.0))
            d16 = 0
            if scale > 0:
                d16 = int(oracle.fp32_to_fp16(np.array([scale]))[0])
                scale = np.float32(oracle.fp16_to_fp32(np.array([d16], np.uint16))[0])
            inv = np.float32(1.0) / scale if scale > 0 else np.float32(0)
            q = np.full(32, 8, np.int64)
            if inv > 0:
                v = (blk * inv).astype(np.float32)
                r = np.sign(v) * np.floor(np.abs(v.astype(np.float64)) + 0.5)   # half away
                qq = np.where(np.isnan(v), -(2**62), np.nan_to_num(r).astype(np.int64) + 8)
                q[:blk.size] = np.clip(qq, 0, 15)
        out[18 * b] = d16 & 0xFF
        out[18 * b + 1] = d16 >> 8
        out[18 * b + 2:18 * b + 18] = (q[:16] | (q[16:] << 4)).astype(np.uint8)
    return out


def test_q4_0_against_numpy_form(oracle):
    rng = np.random.default_rng(4)
    for e in range(-30, 31, 4):
        x = (rng.standard_normal(32 * 16) * 10.0 ** (e / 2)).astype(np.float32)
        assert np.array_equal(oracle.quantize_q4_0(x), numpy_q4_0(oracle, x)), e
    # mixed magnitudes inside blocks, heavy outliers
    x = rng.standard_normal(32 * 64).astype(np.float32)
    x[rng.choice(x.size, 40, replace=False)] *= 1000
    assert np.array_equal(oracle.quantize_q4_0(x), numpy_q4_0(oracle, x))


def test_q4_0_reference_dequant_dot(oracle):
    # quant_test.go:21-54: two blocks, scale FP32ToFP16(0.25), every byte
    # 5 | 12 << 4 -> elements 0..15 = -3 * 0.25, 16..31 = +4 * 0.25
    d = int(oracle.fp32_to_fp16(np.array([0.25], np.float32))[0])
    blk = np.array([d & 0xFF, d >> 8] + [5 | (12 << 4)] * 16, np.uint8)
    raw = np.concatenate([blk, blk])
    deq = oracle.dequantize_q4_0(raw, 64)
    want = np.tile(np.concatenate([np.full(16, -0.75), np.full(16, 1.0)]), 2).astype(np.float32)
    assert np.array_equal(deq, want)
    x = np.arange(1, 65, dtype=np.float32)
    assert abs(float(np.dot(x.astype(np.float64), deq)) - 708.0) < 1e-4


def test_q4_0_reference_round_trips(oracle):
    # quant_test.go:145-160: src[i] = i - 32, |deq - src| <= 4
    src = np.arange(64, dtype=np.float32) - 32
    deq = oracle.dequantize_q4_0(oracle.quantize_q4_0(src), 64)
    assert np.all(np.abs(deq - src) <= 4.0)
    # engine_test.go:275-297: k[i] = i over kvDim 32, |deq[10] - 10| <= 3
    k = np.arange(32, dtype=np.float32)
    assert abs(oracle.dequantize_q4_0(oracle.quantize_q4_0(k), 32)[10] - 10.0) <= 3.0
    # the KVCache Write/Get path (store_vectors / widen) gives the same
    st = oracle.store_vectors(oracle.KV_Q4_0, k[None, :])
    assert st.shape == (1, 18)
    assert np.array_equal(oracle.widen(oracle.KV_Q4_0, 32, st)[0],
                          oracle.dequantize_q4_0(oracle.quantize_q4_0(k), 32))


def _nibbles(raw, b=0):
    qs = raw[18 * b + 2:18 * b + 18]
    return np.concatenate([qs & 0xF, qs >> 4]).astype(np.int64)


def test_q4_0_special_cases(oracle):
    # amax 7 -> scale 7/7 = 1 exactly: ties go away from zero
    x = np.zeros(32, np.float32)
    x[:6] = [7.0, -7.0, 2.5, -2.5, 0.5, -0.49]
    q = _nibbles(oracle.quantize_q4_0(x))
    assert q[:6].tolist() == [15, 1, 11, 5, 9, 8]
    assert np.all(q[6:] == 8)
    # zero block: d = 0, every nibble 8
    raw = oracle.quantize_q4_0(np.zeros(32, np.float32))
    assert raw[0] == 0 and raw[1] == 0 and np.all(_nibbles(raw) == 8)
    # an Inf in the block: d = Inf (0x7C00), inverse 0 -> every nibble 8
    x = np.ones(32, np.float32)
    x[3] = np.inf
    raw = oracle.quantize_q4_0(x)
    assert (int(raw[0]) | (int(raw[1]) << 8)) == 0x7C00 and np.all(_nibbles(raw) == 8)
    # NaN elements are skipped by the maximum and quantise to nibble 0
    # (int(NaN) is the minimum int64 on amd64, clamped to 0)
    x = np.ones(32, np.float32) * 3.5
    x[5] = np.nan
    q = _nibbles(oracle.quantize_q4_0(x))
    assert q[5] == 0 and q[0] == 15
    # subnormal fp16 scale: amax = 7 * 1.5 * 2^-24 -> scale truncates to
    # 2^-24, inverse 2^24, the max element maps to 10.5 -> 11 + 8 -> clamp 15
    # and its negative to -11 + 8 -> clamp 0
    t = np.float32(7 * 1.5 * 2.0 ** -24)
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2] = t, -t, np.float32(2.0 ** -24)
    raw = oracle.quantize_q4_0(x)
    assert (int(raw[0]) | (int(raw[1]) << 8)) == 0x0001
    q = _nibbles(raw)
    assert q[0] == 15 and q[1] == 0 and q[2] == 9
    # scale below half the smallest subnormal: d = 0, all 8
    raw = oracle.quantize_q4_0(np.full(32, 1e-8, np.float32))
    assert raw[0] == 0 and raw[1] == 0 and np.all(_nibbles(raw) == 8)
    # short final block: elements past the end quantise to 8
    x = np.arange(40, dtype=np.float32)
    raw = oracle.quantize_q4_0(x)
    assert raw.size == 36
    assert np.all(_nibbles(raw, 1)[8:] == 8)
    assert np.array_equal(raw, numpy_q4_0(oracle, x))


@pytest.mark.parametrize("kv_dim", [64, 256, 1024])
def test_q4_0_store_gather_round_trip(oracle, kv_dim):
    """Reference-layout paged pool of Q4_0 token vectors (KVBlock per
    paged_kv.go:13-38, Write/Get per kvcache.go:162-206)."""
    x = oracle.normal(77, (37, kv_dim))
    pool = oracle.RefPagedPool(oracle.KV_Q4_0, 2, kv_dim, 8, 16)
    ids = np.repeat(np.array([5, 2, 7], np.int32), 16)[:37]
    slots = np.arange(37, dtype=np.int32) % 16
    pool.store(1, ids, slots, x, -x)
    k, v = pool.gather(1, np.array([5, 2, 7], np.int32), 37)
    assert np.array_equal(k, oracle.store_vectors(oracle.KV_Q4_0, x))
    assert np.array_equal(v, oracle.store_vectors(oracle.KV_Q4_0, -x))
