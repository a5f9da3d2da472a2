"""GPU parity of the O-projection product (gi_weights_upload +
gi_matmul_batch) against the oracle's MatMul (pkg/math/gemv.go, DotVec* of
pkg/quant/quant.go) on the same GGUF bytes: y = x W^T for F32, F16, Q8_0 and
Q4_0 weights.

Both sides sum in float32, in different orders, so the bars are stated for
float32 dot products of length cols:
  * ill-conditioned inputs (weight rows at 300x and 1e-3x the rest, +-8 sigma
    outliers, a batch row at 1e-4x): per output,
    |y - exact| <= 4 * eps32 * sqrt(cols) * sum_c |W[r][c] x[b][c]|, the
    probabilistic rounding bound of a float32 sum, met by the GPU and by the
    oracle alike (exact = the float64 product of the same dequantised
    weights);
  * well-conditioned inputs (N(0,1)): per batch row,
    max|gpu - oracle| <= 1e-5 * max|oracle| and the same against float64.

The shapes cover both product forms: batches under 128 (and quantised
weights) run the 64 x 64 tiles; F16 / F32 weights at batches of 128 and more
run the split-K tiles, whose cases include rows that are not a multiple of
128, a batch with idle waves in its last tile (130), k-step slices with a
remainder (1056 columns: 33 k-steps) and two batch tiles (384)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def dequant(oracle, t, raw, rows, cols):
    """float32 values of GGUF weights (FP16ToFP32 / DequantizeQ8_0 / Q4_0)."""
    if t == oracle.GGML_F32:
        return raw.view(np.float32).reshape(rows, cols)
    if t == oracle.GGML_F16:
        return oracle.fp16_to_fp32(raw.view(np.uint16).reshape(rows, cols))
    f = oracle.dequantize_q8_0 if t == oracle.GGML_Q8_0 else oracle.dequantize_q4_0
    return np.stack([f(raw[r], cols) for r in range(rows)])


EPS32 = float(np.finfo(np.float32).eps)


def _run(gi, dev, t, rows, cols, raw, x):
    import torch
    pool = gi.PagedKVCache(1, 1, 32, 16, 1, gi.KV_F16)
    wt = gi.Weights(pool, t, rows, cols, raw)
    xd = torch.from_numpy(x).to(dev)
    yd = torch.full((x.shape[0], rows), float("nan"), device=dev)
    wt.MatMulBatch(yd, xd)
    pool.synchronize()
    got = yd.cpu().numpy()
    wt.close()
    pool.close()
    return got


@pytest.mark.parametrize("t", [0, 1, 2, 8], ids=["f32", "f16", "q4_0", "q8_0"])
@pytest.mark.parametrize("rows,cols,batch", [(64, 64, 1), (80, 96, 5), (1024, 4096, 64),
                                             (2048, 512, 130), (4096, 1024, 256), (200, 256, 100), (5, 96, 3),
                                             (200, 1056, 200), (136, 4096, 384)])
def test_matmul_batch(gi, oracle, dev, t, rows, cols, batch):
    W = oracle.normal_with_outliers(7 + t + rows, (rows, cols))
    W[1] *= 1e-3
    W[min(5, rows - 1)] *= 300.0
    x = oracle.normal(9 + t + batch, (batch, cols))
    x[0] *= 1e-4
    raw = oracle.quantize_weights(t, W)
    got = _run(gi, dev, t, rows, cols, raw, x)
    want = oracle.matmul(t, raw, x, rows, cols)
    wd = dequant(oracle, t, raw, rows, cols).astype(np.float64)
    x64 = x.astype(np.float64)
    exact = x64 @ wd.T
    bound = 4 * EPS32 * np.sqrt(cols) * (np.abs(x64) @ np.abs(wd).T) + 1e-30
    r_gpu = float((np.abs(got - exact) / bound).max())
    r_ref = float((np.abs(want - exact) / bound).max())
    print("matmul", t, rows, cols, batch, "error / bound: gpu %.3f, oracle %.3f" % (r_gpu, r_ref),
          flush=True)
    assert r_ref <= 1.0, r_ref          # the bar holds for the reference's own loop
    assert r_gpu <= 1.0, r_gpu


@pytest.mark.parametrize("t", [0, 1, 2, 8], ids=["f32", "f16", "q4_0", "q8_0"])
def test_matmul_well_conditioned(gi, oracle, dev, t):
    rows, cols, batch = 4096, 4096, 32
    W = oracle.normal(71 + t, (rows, cols))
    x = oracle.normal(72 + t, (batch, cols))
    raw = oracle.quantize_weights(t, W)
    got = _run(gi, dev, t, rows, cols, raw, x)
    want = oracle.matmul(t, raw, x, rows, cols)
    exact = x.astype(np.float64) @ dequant(oracle, t, raw, rows, cols).astype(np.float64).T
    den = np.abs(want).max(axis=1)
    e_or = float((np.abs(got - want).max(axis=1) / den).max())
    e_ex = float((np.abs(got - exact).max(axis=1) / den).max())
    print("matmul well-conditioned", t, "gpu vs oracle %.2e, gpu vs f64 %.2e" % (e_or, e_ex), flush=True)
    assert e_or <= 1e-5 and e_ex <= 1e-5, (e_or, e_ex)


@pytest.mark.parametrize("t", [1, 8], ids=["f16", "q8_0"])
def test_matmul_batch_sizes_on_one_weight_set(gi, oracle, dev, t):
    """One weight set called with a growing, then shrinking, batch: the
    activation buffers grow, and the zero padding past each batch is rewritten
    on every call (a smaller batch after a larger one must not see its rows)."""
    import torch
    rows, cols = 192, 256
    W = oracle.normal(81 + t, (rows, cols))
    raw = oracle.quantize_weights(t, W)
    wd = dequant(oracle, t, raw, rows, cols).astype(np.float64)
    pool = gi.PagedKVCache(1, 1, 32, 16, 1, gi.KV_F16)
    wt = gi.Weights(pool, t, rows, cols, raw)
    try:
        for i, batch in enumerate((5, 130, 3, 64, 65)):
            x = oracle.normal(90 + i, (batch, cols))
            yd = torch.full((batch, rows), float("nan"), device=dev)
            wt.MatMulBatch(yd, torch.from_numpy(x).to(dev))
            pool.synchronize()
            got = yd.cpu().numpy()
            exact = x.astype(np.float64) @ wd.T
            err = float((np.abs(got - exact).max(axis=1) / np.abs(exact).max(axis=1)).max())
            assert err <= 1e-5, (batch, err)
    finally:
        wt.close()
        pool.close()


def test_matmul_errors(gi, dev):
    pool = gi.PagedKVCache(1, 1, 32, 16, 1, gi.KV_F16)
    raw = np.zeros((4, 40), np.uint8)
    for t, cols in ((3, 64), (1, 20)):               # unsupported type, cols % 32
        with pytest.raises(gi.GIError) as e:
            gi.Weights(pool, t, 4, cols, raw)
        assert e.value.code == -3
    # weights may outlive their pool: destroy waits for the device itself
    w = gi.Weights(pool, gi.GGML_F16, 16, 32, np.zeros((16, 64), np.uint8))
    pool.close()
    w.close()
