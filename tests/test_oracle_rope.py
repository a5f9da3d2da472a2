"""Pins the oracle's RoPE (ApplyRoPE, pkg/math/kernels.go:22-35) without
restating its formula:

  * kernels_test.go:39-46 (position 0 leaves the vector unchanged);
  * the float32 cos/sin table against a 50-digit evaluation of
    cos / sin(pos * theta^(-2i/d)) (a wrong exponent, index or theta fails);
  * the rotation of a unit vector e_i lands at angle +pos*freq_i in the plane
    (i, i + d/2) (fixes the sign and the half-split pairing);
  * pair norms are kept and q.k depends only on the position difference;
  * a rope dimension below head_dim turns only the first rope_dim dims, at
    rope_dim's frequencies (forward.go:945-977)."""
import math

import mpmath
import numpy as np
import pytest

mpmath.mp.dps = 50


def _exact_f32(x):
    """float32 nearest to the mpmath value x (via a 50-digit decimal string,
    so the only rounding is to float32)."""
    return np.float32(mpmath.nstr(x, 40, strip_zeros=False))


def _ulp_diff(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, np.int64(-2**31) - ia, ia)
    ib = np.where(ib < 0, np.int64(-2**31) - ib, ib)
    return np.abs(ia - ib)


def test_reference_rope_position_zero(oracle):
    # kernels_test.go:39-46: {1, 0, 0, 1} at pos 0, headDim 4, theta 1e4
    out = oracle.apply_rope(np.array([1, 0, 0, 1], np.float32), 0, 4, 10000.0)
    assert out.tolist() == [1.0, 0.0, 0.0, 1.0]


@pytest.mark.parametrize("theta,d", [(10000.0, 64), (500000.0, 128), (1000000.0, 64)])
def test_rope_table_against_50_digit_values(oracle, theta, d):
    rng = np.random.default_rng(7)
    positions = sorted(set([0, 1, 2, 15, 16, 255, 4095, 8191, 32767, 131071] +
                           rng.integers(0, 131072, 40).tolist()))
    half = d // 2
    worst, exact = 0, 0
    total = 0
    th = mpmath.mpf(theta)
    for p in positions:
        tab = oracle.rope_table(theta, d, p, 1)[0]
        for i in range(half):
            ang = mpmath.mpf(p) / th ** (mpmath.mpf(2 * i) / d)
            want = (_exact_f32(mpmath.cos(ang)), _exact_f32(mpmath.sin(ang)))
            du = max(int(_ulp_diff(tab[i, 0], want[0])), int(_ulp_diff(tab[i, 1], want[1])))
            worst = max(worst, du)
            exact += du == 0
            total += 1
    # float64 angles carry ~1e-11 absolute error at 1.3e5 rad: a float32
    # result may sit one ulp off only where the true value is near a tie
    assert worst <= 1, worst
    assert exact >= 0.99 * total, (exact, total)


@pytest.mark.parametrize("d", [8, 64, 128])
def test_rotation_sign_and_pairing(oracle, d):
    theta = 500000.0
    half = d // 2
    for p in (1, 3, 100, 8191):
        for i in range(half):
            e = np.zeros(d, np.float32)
            e[i] = 1.0
            y = oracle.apply_rope(e, p, d, theta)
            # e_i turns inside the (i, i+half) plane only
            others = np.delete(y, [i, i + half])
            assert not others.any()
            ang = float(mpmath.fmod(mpmath.mpf(p) / mpmath.mpf(theta) ** (mpmath.mpf(2 * i) / d),
                                    2 * mpmath.pi))
            got = math.atan2(float(y[i + half]), float(y[i])) % (2 * math.pi)
            diff = abs(got - ang)
            assert min(diff, 2 * math.pi - diff) < 2e-6, (p, i, got, ang)


def test_pair_norms_and_relative_position(oracle):
    d, theta = 128, 500000.0
    half = d // 2
    q = oracle.normal(11, (d,))
    k = oracle.normal(12, (d,))
    for m, n, shift in [(5, 2, 7), (100, 40, 1000), (8000, 8191, 123)]:
        rq = oracle.apply_rope(q, m, d, theta)
        rk = oracle.apply_rope(k, n, d, theta)
        pn_in = np.hypot(q[:half].astype(np.float64), q[half:].astype(np.float64))
        pn_out = np.hypot(rq[:half].astype(np.float64), rq[half:].astype(np.float64))
        assert np.allclose(pn_in, pn_out, rtol=1e-6, atol=1e-6)
        a = float(np.dot(rq.astype(np.float64), rk.astype(np.float64)))
        rq2 = oracle.apply_rope(q, m + shift, d, theta)
        rk2 = oracle.apply_rope(k, n + shift, d, theta)
        b = float(np.dot(rq2.astype(np.float64), rk2.astype(np.float64)))
        assert abs(a - b) <= 1e-4 * (np.linalg.norm(q) * np.linalg.norm(k)), (a, b)


def test_partial_rope_dim_and_per_head(oracle):
    H, hd, rd, theta = 3, 64, 32, 10000.0
    x = oracle.normal(21, (2, H * hd))
    pos = np.array([9, 300], np.int32)
    y = oracle.rope_heads(x, pos, H, hd, rd, theta)
    for t in range(2):
        for h in range(H):
            seg = x[t, h * hd:(h + 1) * hd]
            out = y[t, h * hd:(h + 1) * hd]
            assert np.array_equal(out[rd:], seg[rd:])                     # untouched dims
            want = oracle.apply_rope(seg[:rd], int(pos[t]), rd, theta)   # rope_dim frequencies
            assert np.array_equal(out[:rd], want)
    # rope_dim == head_dim (or <= 0) turns whole heads
    full = oracle.rope_heads(x, pos, H, hd, 0, theta)
    assert np.array_equal(full[1, :hd], oracle.apply_rope(x[1, :hd], 300, hd, theta))
