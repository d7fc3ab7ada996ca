"""Pins the int8 Winograd oracle (oracle/wino8.c, restating src/wino.c): the
weight packing's quantization against its closed form on hand-made kernels;
a single-tile case built so that every quantization is exact, against the exact
integer direct convolution; random data against a float64 direct convolution
(signal-to-error above the reference's own 49 dB class)."""
import numpy as np

import pyoracle as O

BT = np.array([[1, 0, -1, 0], [0, 1, 1, 0], [0, -1, 1, 0], [0, 1, 0, -1]], np.float64)


def direct(x, w, b):
    H, W, C = x.shape
    xp = np.pad(x.astype(np.float64), ((1, 1), (1, 1), (0, 0)))
    cols = np.stack([xp[ky:ky + H, kx:kx + W] for ky in range(3) for kx in range(3)], axis=2)
    return (cols.reshape(H * W, -1) @ w.reshape(w.shape[0], -1).T.astype(np.float64) + b).reshape(H, W, -1)


def lut_silu(y16):
    L = O.lib()
    return np.array([L.orc_silu_lut_h(int(v)) for v in y16.reshape(-1).view(np.uint16)], np.uint16).reshape(y16.shape)


def test_pack_closed_form():
    # a kernel with only the centre tap 1 -> U = G e G^T = outer([0, 1/2, -1/2, 0]) (entries 0, +-1/4): sw =
    # (1/4) / 127, q = round(U / sw) = +-127 at the four inner positions
    C, K = 4, 2
    w = np.zeros((K, 3, 3, C), np.float32)
    w[:, 1, 1, :] = 1
    U8, sw, zw = O.wino8_pack(w)
    assert np.allclose(sw, 0.25 / 127)
    Gc = np.array([0, .5, -.5, 0])
    U = np.outer(Gc, Gc).reshape(16)
    assert np.array_equal(U8[:, 0, 0], np.round(U / 0.25 * 127).astype(np.int8))
    # zw[o] = sw * sum_xi coef(o, xi) wsum(xi) with wsum = C q
    AT = np.array([[1, 1, 1, 0], [0, 1, -1, -1]])
    q = U8[:, 0, 0].astype(np.int64).reshape(4, 4) * C
    for o in range(4):
        r, c = divmod(o, 2)
        z = (np.outer(AT[r], AT[c]) * q).sum()
        assert np.isclose(zw[o, 0], sw[0] * z, rtol=1e-6)


def test_exact_single_tile():
    # one 2 x 2 tile, integer inputs whose transformed range is exactly 255 (tile scale 1, zero point exact) and
    # weights whose transform is a multiple of 1/2 with maximum 63.5 (channel scale 1/2): every quantization is
    # exact, so the Winograd result equals the exact direct convolution
    rng = np.random.default_rng(0)
    C, K = 8, 4
    w = np.zeros((K, 3, 3, C), np.float32)
    # centre taps only: U = g outer([0, 1/2, -1/2, 0]) = +-g / 4; one tap of 254 per channel makes max |U| = 63.5,
    # sw = 1/2, and U / sw = +-g / 2: integers for even taps
    w[:, 1, 1, :] = rng.integers(-15, 16, (K, C)) * 4
    w[:, 1, 1, 0] = 254
    U8, sw, zw = O.wino8_pack(w)
    assert np.all(sw == 0.5)
    for seed in range(2000):
        r = np.random.default_rng(seed)
        x = r.integers(-40, 41, (2, 2, C)).astype(np.float32)
        d = np.pad(x, ((1, 1), (1, 1), (0, 0))).astype(np.float64)
        V = np.einsum('ij,jlc,ml->imc', BT, d, BT)
        mn, mx = min(V.min(), 0.0), max(V.max(), 0.0)
        if mx - mn == 255 and float(mn).is_integer():
            break
    else:
        raise AssertionError("no exact case found")
    b = np.zeros(K, np.float32)
    got = O.wino8(x, (U8, sw, zw), b)
    exact = direct(x, w, b)
    assert np.abs(exact).max() < 2 ** 24     # exact in fp32: both sides round it to fp16 once
    want = lut_silu(exact.astype(np.float16))
    assert np.array_equal(got.view(np.uint16), want)


def test_random_against_direct_conv():
    rng = np.random.default_rng(3)
    H, W, C, K = 9, 14, 32, 16          # odd height: a partial last tile row
    x = (rng.standard_normal((H, W, C)) / (1 + np.exp(-rng.standard_normal((H, W, C))))).astype(np.float32)
    w = (rng.standard_normal((K, 3, 3, C)) * np.sqrt(2 / (9 * C))).astype(np.float32)
    b = (rng.standard_normal(K) * 0.1).astype(np.float32)
    got = O.wino8(x, O.wino8_pack(w), b).astype(np.float64)
    y = direct(x, w, b)
    ref = y / (1 + np.exp(-y))
    snr = 10 * np.log10((ref ** 2).sum() / ((got - ref) ** 2).sum())
    assert snr > 35, snr
