"""Pins the oracle's convolutions, pooling, FC and L2 (oracle/oracle.c).

The f32 convolution is checked against the f64 brute force on the reference's
own unit-test cases (tests/test_blocked.cpp:107-169, same shapes, U(-1,1) data,
1e-4 max|d| gate); the f64 brute force is pinned by hand-computed answers and
invariants (delta kernel = shift/identity, zero weights = bias, linearity).
"""
import numpy as np

import pyoracle as O


def U(rng, *shape):
    return rng.uniform(-1.0, 1.0, shape).astype(np.float32)


def test_f64_conv_hand_computed():
    x = np.ones((1, 4, 5), dtype=np.float32)
    w = np.ones((1, 1, 3, 3), dtype=np.float32)
    y = O.conv2d(x, w, 1, 1, f64=True)[0]
    # corners see a 2x2 window, edges 2x3 / 3x2, interior 3x3
    assert y[0, 0] == 4 and y[0, 2] == 6 and y[1, 0] == 6 and y[1, 2] == 9 and y[3, 4] == 4
    # stride 2: outputs at input rows 0, 2 and cols 0, 2, 4
    y2 = O.conv2d(x, w, 2, 1, f64=True)[0]
    assert y2.shape == (2, 3)
    assert y2.tolist() == [[4, 6, 4], [6, 9, 6]]
    # a one-hot kernel at (kh, kw) reads x[ih + kh - 1, iw + kw - 1]
    rng = np.random.default_rng(0)
    xr = U(rng, 2, 6, 7)
    for kh in range(3):
        for kw in range(3):
            wk = np.zeros((2, 2, 3, 3), dtype=np.float32)
            wk[0, 1, kh, kw] = 1.0
            wk[1, 0, kh, kw] = 1.0
            yk = O.conv2d(xr, wk, 1, 1, f64=True)
            pad = np.pad(xr, ((0, 0), (1, 1), (1, 1)))
            assert np.array_equal(yk[0], pad[1, kh:kh + 6, kw:kw + 7])
            assert np.array_equal(yk[1], pad[0, kh:kh + 6, kw:kw + 7])


def test_f64_conv_invariants():
    rng = np.random.default_rng(1)
    x, x2 = U(rng, 8, 9, 10), U(rng, 8, 9, 10)
    w, w2 = U(rng, 4, 8, 3, 3), U(rng, 4, 8, 3, 3)
    b = U(rng, 4)
    zero = O.conv2d(x, np.zeros_like(w), 1, 1, bias=b, f64=True)
    assert np.allclose(zero, b[:, None, None].astype(np.float64) * np.ones((4, 9, 10)))
    lin = O.conv2d(x + x2, w, 1, 1, f64=True)
    assert np.allclose(lin, O.conv2d(x, w, 1, 1, f64=True) + O.conv2d(x2, w, 1, 1, f64=True), atol=1e-5)
    lin_w = O.conv2d(x, w + w2, 1, 1, f64=True)
    assert np.allclose(lin_w, O.conv2d(x, w, 1, 1, f64=True) + O.conv2d(x, w2, 1, 1, f64=True), atol=1e-5)
    # residual + relu epilogue
    r = U(rng, 4, 9, 10)
    e = O.conv2d(x, w, 1, 1, bias=b, residual=r, relu=True, f64=True)
    plain = O.conv2d(x, w, 1, 1, f64=True) + b[:, None, None] + r
    assert np.allclose(e, np.maximum(plain, 0.0), atol=1e-12)


def test_f64_conv_matches_numpy_im2col():
    # an independent formulation: explicit im2col + matmul in float64
    rng = np.random.default_rng(2)
    for (IC, OC, H, W, K, s, p) in ((3, 5, 7, 9, 3, 1, 1), (4, 6, 8, 11, 3, 2, 1), (6, 4, 9, 7, 1, 2, 0)):
        x, w = U(rng, IC, H, W), U(rng, OC, IC, K, K)
        xp = np.pad(x.astype(np.float64), ((0, 0), (p, p), (p, p)))
        Ho, Wo = (H + 2 * p - K) // s + 1, (W + 2 * p - K) // s + 1
        cols = np.zeros((IC * K * K, Ho * Wo))
        for ic in range(IC):
            for kh in range(K):
                for kw in range(K):
                    cols[(ic * K + kh) * K + kw] = xp[ic, kh:kh + s * (Ho - 1) + 1:s,
                                                      kw:kw + s * (Wo - 1) + 1:s].reshape(-1)
        ref = (w.reshape(OC, -1).astype(np.float64) @ cols).reshape(OC, Ho, Wo)
        assert np.allclose(O.conv2d(x, w, s, p, f64=True), ref, atol=1e-12)


def test_reference_blocked_cases_f32_vs_f64():
    # tests/test_blocked.cpp:107-169 (3x3 s1/s2, small, fused bias+ReLU, 1x1 s2)
    rng = np.random.default_rng(1234)
    cases = [((20, 11, 32, 64), 3, 1, 1, False), ((20, 11, 64, 128), 3, 2, 1, False),
             ((7, 5, 16, 16), 3, 1, 1, False), ((20, 11, 32, 64), 3, 1, 1, True),
             ((20, 11, 64, 128), 3, 2, 1, True), ((20, 11, 64, 128), 1, 2, 0, False),
             ((15, 9, 32, 64), 1, 2, 0, False)]
    for (W, H, IC, OC), K, s, p, fused in cases:
        x, w = U(rng, IC, H, W), U(rng, OC, IC, K, K)
        b = U(rng, OC) if fused else None
        got = O.conv2d(x, w, s, p, bias=b, relu=fused)
        ref = O.conv2d(x, w, s, p, bias=b, relu=fused, f64=True)
        assert got.shape == ref.shape
        assert np.abs(got - ref).max() <= 1e-4


def test_tstp_closed_form():
    eps = 1e-8
    x = np.full((3, 2, 5), 2.5, dtype=np.float32)
    p = O.tstp(x, eps)
    assert np.allclose(p[:6], 2.5) and np.allclose(p[6:], np.sqrt(eps))
    rng = np.random.default_rng(4)
    x = U(rng, 4, 3, 17)
    p = O.tstp(x, eps)
    mean = x.astype(np.float64).mean(axis=2).reshape(-1)          # C-outer, H-inner
    std = np.sqrt(x.astype(np.float64).var(axis=2, ddof=1) + eps).reshape(-1)
    assert np.allclose(p[:12], mean, atol=1e-6) and np.allclose(p[12:], std, atol=1e-6)
    # two frames: unbiased variance (a-b)^2/2
    y = np.array([[[1.0, 4.0]]], dtype=np.float32)
    assert np.allclose(O.tstp(y, 0.0), [2.5, np.sqrt(4.5)])


def test_linear_and_l2():
    rng = np.random.default_rng(5)
    x, w, b, mv = U(rng, 50), U(rng, 7, 50), U(rng, 7), U(rng, 7)
    y = O.linear(x, w, b, mv)
    assert np.allclose(y, w.astype(np.float64) @ x - mv + b, atol=1e-5)
    e = O.l2norm(y)
    assert abs(np.linalg.norm(e.astype(np.float64)) - 1.0) < 1e-6
    assert np.allclose(e * np.linalg.norm(y), y, atol=1e-5)
    assert np.array_equal(O.l2norm(np.zeros(4, np.float32)), np.zeros(4, np.float32))
