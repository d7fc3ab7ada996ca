"""GPU parity of the fp16 Winograd F(2x2,3x3) convolution against a float64
direct convolution (the oracle the configuration names: the reference has no
64-channel kernel).

Stated tolerance, per output before the activation (u = 2^-11, the fp16 unit
roundoff): |y_gpu - y_direct| <= 4 u E + u |y_direct| + 2^-24, with
E = sum_ci |A|^T (|U| o |V|) |A| evaluated in float64 on the exact transforms:
every product U_p V_p carries the fp16 roundings of U (one) and of V (two levels
of adds), the matrix core sums in fp32, and the result is rounded to fp16 once.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BT = np.array([[1, 0, -1, 0], [0, 1, 1, 0], [0, -1, 1, 0], [0, 1, 0, -1]], np.float64)
G = np.array([[1, 0, 0], [.5, .5, .5], [.5, -.5, .5], [0, 0, 1]], np.float64)
AT = np.array([[1, 1, 1, 0], [0, 1, -1, -1]], np.float64)


def say(*a):
    print(*a, flush=True)


def direct(xp, w, b):
    """float64 3x3 'same' conv: xp [H+2][W+2][C] (zero halo), w [K][3][3][C] -> [H][W][K]."""
    Hp, Wp, C = xp.shape
    H, W = Hp - 2, Wp - 2
    cols = np.stack([xp[ky:ky + H, kx:kx + W] for ky in range(3) for kx in range(3)], axis=2)  # H W 9 C
    return cols.reshape(H * W, 9 * C) @ w.reshape(w.shape[0], -1).T.astype(np.float64) + b


def bound(xp, w):
    """E per output (H, W, K): the first-order error magnitude of the transformed products."""
    Hp, Wp, C = xp.shape
    H, W = Hp - 2, Wp - 2
    K = w.shape[0]
    U = np.abs(np.einsum('ij,kjlc,ml->kimc', G, w.astype(np.float64), G))       # K 4 4 C
    E = np.zeros((H, W, K))
    for ty in range(H // 2):
        for tx in range(W // 2):
            d = xp[2 * ty:2 * ty + 4, 2 * tx:2 * tx + 4].astype(np.float64)       # 4 4 C
            V = np.abs(np.einsum('ij,jlc,ml->imc', BT, d, BT))                    # 4 4 C
            Mabs = np.einsum('kimc,imc->kim', U, V)                               # K 4 4
            E[2 * ty:2 * ty + 2, 2 * tx:2 * tx + 2] = np.einsum('ai,kim,bm->abk', np.abs(AT), Mabs, np.abs(AT))
    return E


def run(hip, xp, w, b, act=0, opad=0, res=None, rpad=0):
    H_ = hip
    B, Hp, Wp, C = xp.shape
    H, W = Hp - 2, Wp - 2
    K = w.shape[0]
    P = H_.lib().bnh_wino16_new(C, K, np.ascontiguousarray(w, np.float32).ctypes.data,
                                np.ascontiguousarray(b, np.float32).ctypes.data)
    if not P:
        H_.check(None, "bnh_wino16_new")
    try:
        x_ws = Hp * Wp * C + 32
        xs = np.zeros((B, x_ws), np.float16)
        xs[:, :Hp * Wp * C] = xp.reshape(B, -1)
        rows = (H + 2 * opad) * (W + 2 * opad)
        o_ws = rows * K + 16
        dx = H_.DeviceArray.from_host(xs)
        do = H_.DeviceArray.from_host(np.full((B, o_ws), np.float16(3.0)))
        dr, r_ws, ldr = None, 0, 0
        if res is not None:
            dr = H_.DeviceArray.from_host(np.ascontiguousarray(res).reshape(B, -1))
            r_ws, ldr = (H + 2 * rpad) * (W + 2 * rpad) * K, K
        H_.check(H_.lib().bnh_wino_f16(dx.ptr, x_ws, H, W, C, P, act, do.ptr, o_ws, K, opad,
                                       dr.ptr if dr else None, r_ws, ldr, rpad, B, None), "wino_f16")
        H_.sync()
        return do.numpy()[:, :rows * K].reshape(B, H + 2 * opad, W + 2 * opad, K)
    finally:
        H_.lib().bnh_wino16_free(P)


def silu(y):
    return y / (1 + np.exp(-y))


def make(rng, B, H, W, C, K):
    xp = np.zeros((B, H + 2, W + 2, C), np.float16)
    xp[:, 1:-1, 1:-1] = rng.standard_normal((B, H, W, C))
    w = (rng.standard_normal((K, 3, 3, C)) * np.sqrt(2.0 / (9 * C))).astype(np.float16).astype(np.float32)
    b = (rng.standard_normal(K) * 0.1).astype(np.float32)
    return xp, w, b


@pytest.mark.parametrize("H,W,C,K", [(6, 10, 24, 24), (8, 66, 64, 64), (4, 4, 8, 40), (10, 34, 60, 16)])
def test_within_stated_tolerance(hip, H, W, C, K):
    rng = np.random.default_rng(H * 100 + W + C)
    B = 2
    xp, w, b = make(rng, B, H, W, C, K)
    say("wino", H, W, C, K)
    out = run(hip, xp, w, b).astype(np.float64)
    u = 2.0 ** -11
    for i in range(B):
        ref = direct(xp[i].astype(np.float64), w, b).reshape(H, W, K)
        tol = 4 * u * bound(xp[i], w) + u * np.abs(ref) + 2.0 ** -24
        err = np.abs(out[i] - ref)
        assert (err <= tol).all(), float(np.max(err / tol))


def test_epilogue_forms(hip):
    rng = np.random.default_rng(3)
    B, H, W, C, K = 2, 6, 8, 16, 32
    xp, w, b = make(rng, B, H, W, C, K)
    res = rng.standard_normal((B, H, W, K)).astype(np.float16)
    plain = run(hip, xp, w, b).astype(np.float32)
    say("wino epilogue")
    s = run(hip, xp, w, b, act=1, opad=1, res=res)
    assert not s[:, 0].any() and not s[:, -1].any() and not s[:, :, 0].any() and not s[:, :, -1].any()
    inner = s[:, 1:-1, 1:-1].astype(np.float64)
    # SiLU of (about) the same pre-activations, then one fp16 residual add
    want = (silu(plain.astype(np.float64)) + res.astype(np.float64))
    assert np.abs(inner - want).max() < 0.02
    r = run(hip, xp, w, b, act=2).astype(np.float32)
    assert (r >= 0).all() and np.array_equal(r[plain > 0.01], plain[plain > 0.01])


def test_config2_full_size(hip):
    """64 -> 64 channels over 96 x 256, two windows, against float64 direct convolution."""
    rng = np.random.default_rng(22)
    B, H, W, C, K = 2, 96, 256, 64, 64
    xp, w, b = make(rng, B, H, W, C, K)
    say("wino config2")
    out = run(hip, xp, w, b).astype(np.float64)
    u = 2.0 ** -11
    for i in range(B):
        ref = direct(xp[i].astype(np.float64), w, b).reshape(H, W, K)
        err = np.abs(out[i] - ref)
        # the bound at full size, on a band of rows (the python bound is slow): rows 40..47
        tol = 4 * u * bound(xp[i, 40:50], w) + u * np.abs(ref[40:48]) + 2.0 ** -24
        assert (err[40:48] <= tol).all()
        # everywhere: relative to the output scale
        assert err.max() <= 8 * u * np.abs(ref).max()


@pytest.mark.parametrize("H,W", [(8, 12), (24, 64)])
def test_conv3c24_against_oracle(hip, H, W):
    """The CONV3C24 form (24 -> 24 channels, SiLU, residual = the op's own zero-haloed input, zero-haloed output)
    against the oracle's restatement of src/wino_s0.c. Both sides are held to float64 truth
    t = SiLU(direct conv + b) + x:
      GPU:    |gpu - t| <= 1.1 (4 u E + u |y|) + 2 u |t| + 2^-20 |y| + 2^-24
      oracle: |orc - t| <= 1.1 (40 u E) + 2e-3 max(1, |SiLU(y)|) + 2 u |t|
    (fp16 chain over 24 input channels, fp16 output transform and bias, the fp16 polynomial SiLU's accuracy),
    and |gpu - orc| within the sum of the two."""
    import pyoracle as O
    rng = np.random.default_rng(H + W)
    B, C = 2, 24
    xp, w, b = make(rng, B, H, W, C, C)
    say("wino conv3c24", H, W)
    g = run(hip, xp, w, b, act=1, opad=1, res=xp, rpad=1).astype(np.float64)
    u = 2.0 ** -11
    for i in range(B):
        assert not g[i, 0].any() and not g[i, -1].any() and not g[i, :, 0].any() and not g[i, :, -1].any()
        o = O.wino_s0(xp[i], w, b).astype(np.float64)
        assert np.array_equal(o[0], g[i, 0]) and np.array_equal(o[:, 0], g[i, :, 0])
        y = direct(xp[i].astype(np.float64), w, b).reshape(H, W, C)
        sy = silu(y)
        t = sy + xp[i, 1:-1, 1:-1].astype(np.float64)
        E = bound(xp[i], w)
        tg = 1.1 * (4 * u * E + u * np.abs(y)) + 2 * u * np.abs(t) + 2.0 ** -20 * np.abs(y) + 2.0 ** -24
        to = 1.1 * 40 * u * E + 2e-3 * np.maximum(1.0, np.abs(sy)) + 2 * u * np.abs(t)
        gi, oi = g[i, 1:-1, 1:-1], o[1:-1, 1:-1]
        assert (np.abs(gi - t) <= tg).all(), float(np.max(np.abs(gi - t) / tg))
        assert (np.abs(oi - t) <= to).all(), float(np.max(np.abs(oi - t) / to))
        assert (np.abs(gi - oi) <= tg + to).all()


def test_bad_shapes_refused(hip):
    H_ = hip
    w = np.zeros((8, 3, 3, 6), np.float32)
    assert not H_.lib().bnh_wino16_new(6, 8, w.ctypes.data, None)
    assert b"C % 4 == 0" in H_.lib().bnh_last_error()
