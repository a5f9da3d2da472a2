"""Pins the oracle's weight-matrix products (pkg/math/gemv.go MatMulF32 /
F16 / Q4_0 / Q8_0 with DotVecF32 / F16 / Q4_0 / Q8_0 of pkg/quant/quant.go):

  * kernels_test.go:63-80 (identity matrix, y == x exactly) restated;
  * quant_test.go:21-54 (DotVecQ4_0 of hand-made blocks equals the dot with
    the dequantised weights within 1e-4) restated;
  * every type against a float64 product with the dequantised weights
    (DequantizeQ8_0 / Q4_0 and FP16ToFP32 are pinned elsewhere), which fixes
    row/column order, block order and the scale placement;
  * GGUF row sizes (cols*4, cols*2, cols/32*18, cols/32*34)."""
import numpy as np
import pytest


def dequant(oracle, t, raw, rows, cols):
    if t == oracle.GGML_F32:
        return raw.view(np.float32).reshape(rows, cols)
    if t == oracle.GGML_F16:
        return oracle.fp16_to_fp32(raw.view(np.uint16).reshape(rows, cols))
    f = oracle.dequantize_q8_0 if t == oracle.GGML_Q8_0 else oracle.dequantize_q4_0
    return np.stack([f(raw[r], cols) for r in range(rows)])


def test_reference_identity(oracle):
    x = np.array([1, 2, 3, 4], np.float32)
    y = oracle.matmul(oracle.GGML_F32, np.eye(4, dtype=np.float32).view(np.uint8), x, 4, 4)
    assert y[0].tolist() == [1.0, 2.0, 3.0, 4.0]


def test_reference_q4_0_dot_product(oracle):
    d = int(oracle.fp32_to_fp16(np.array([0.25], np.float32))[0])
    blk = np.array([d & 0xFF, d >> 8] + [5 | (12 << 4)] * 16, np.uint8)
    raw = np.concatenate([blk, blk])
    x = np.arange(1, 65, dtype=np.float32)
    deq = oracle.dequantize_q4_0(raw, 64)
    got = oracle.dot_vec_q4_0(x, raw)
    assert abs(float(got) - float(np.dot(x.astype(np.float64), deq))) <= 1e-4
    assert got == np.float32(708.0)
    y = oracle.matmul(oracle.GGML_Q4_0, raw, x, 1, 64)
    assert y[0, 0] == got


@pytest.mark.parametrize("t", [0, 1, 2, 8], ids=["f32", "f16", "q4_0", "q8_0"])
def test_matmul_against_float64(oracle, t):
    rows, cols, batch = 48, 256, 5
    W = oracle.normal_with_outliers(31 + t, (rows, cols))
    W[3] *= 1e-3            # rows at other scales
    W[7] *= 50.0
    x = oracle.normal(41 + t, (batch, cols))
    raw = oracle.quantize_weights(t, W)
    assert raw.shape == (rows, oracle.weight_row_bytes(t, cols))
    assert oracle.weight_row_bytes(t, cols) == {0: cols * 4, 1: cols * 2, 2: cols // 32 * 18,
                                                8: cols // 32 * 34}[t]
    y = oracle.matmul(t, raw, x, rows, cols)
    want = x.astype(np.float64) @ dequant(oracle, t, raw, rows, cols).astype(np.float64).T
    err = np.abs(y - want).max(axis=1) / np.abs(want).max(axis=1)
    assert err.max() <= 1e-5, err.max()     # float32 summation of 256 terms
