"""GPU parity of the int8 Winograd F(2x2,3x3) convolution (libbnneon's WINO_S8,
src/wino.c) against the oracle: bit-identical fp16 outputs, for odd and even
image sizes (partial last tiles), channel counts past one MFMA step, several
windows at padded strides, and inputs with a constant or all-zero tile."""
import numpy as np
import pytest

import pyoracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def run(hip, x, w, b, slack=24):
    H_ = hip
    B, H, W, C = x.shape
    K = w.shape[0]
    P = H_.lib().bnh_wino8_new(C, K, np.ascontiguousarray(w, np.float32).ctypes.data,
                               np.ascontiguousarray(b, np.float32).ctypes.data)
    if not P:
        H_.check(None, "bnh_wino8_new")
    try:
        x_ws = H * W * C + slack
        xs = np.zeros((B, x_ws), np.float32)
        xs[:, :H * W * C] = x.reshape(B, -1)
        o_ws = H * W * K + 8
        dx = H_.DeviceArray.from_host(xs)
        do = H_.DeviceArray.from_host(np.full((B, o_ws), np.float16(5.0)))
        nb = H_.lib().bnh_wino8_work_bytes(H, W, C, B)
        dw = H_.DeviceArray(nb, np.uint8)
        H_.check(H_.lib().bnh_wino_s8(dx.ptr, x_ws, H, W, P, do.ptr, o_ws, B, dw.ptr, nb, None), "wino_s8")
        H_.sync()
        got = do.numpy()
        assert (got[:, H * W * K:] == np.float16(5.0)).all()   # nothing written past a window's output
        return got[:, :H * W * K].reshape(B, H, W, K)
    finally:
        H_.lib().bnh_wino8_free(P)


def same16(a, b):
    an, bn = np.isnan(a), np.isnan(b)
    return np.array_equal(an, bn) and np.array_equal(a.view(np.uint16)[~an], b.view(np.uint16)[~bn])


@pytest.mark.parametrize("H,W,C,K", [(8, 8, 8, 16), (9, 14, 32, 16), (15, 7, 72, 48), (24, 32, 128, 80), (1, 1, 16, 32)])
def test_bit_exact(hip, H, W, C, K):
    rng = np.random.default_rng(H * 1000 + W * 10 + C)
    B = 3
    x = rng.standard_normal((B, H, W, C)).astype(np.float32)
    x = x / (1 + np.exp(-x))                                   # SiLU-distributed activations
    w = (rng.standard_normal((K, 3, 3, C)) * np.sqrt(2 / (9 * C))).astype(np.float32)
    b = (rng.standard_normal(K) * 0.1).astype(np.float32)
    say("wino8", H, W, C, K)
    got = run(hip, x, w, b)
    pk = O.wino8_pack(w)
    for i in range(B):
        assert same16(got[i], O.wino8(x[i], pk, b)), i


def test_flat_and_zero_tiles(hip):
    rng = np.random.default_rng(9)
    B, H, W, C, K = 2, 6, 6, 16, 16
    x = rng.standard_normal((B, H, W, C)).astype(np.float32)
    x[0, :2, :2] = 0.0            # an all-zero tile (range 0: scale 1)
    x[1, 2:4, 2:4] = 0.75         # a locally constant patch
    x[1, 4:, 4:] = 1e-33          # a tiny-range tile (scale floored at 1e-30)
    w = (rng.standard_normal((K, 3, 3, C)) * 0.2).astype(np.float32)
    b = np.zeros(K, np.float32)
    say("wino8 flat tiles")
    got = run(hip, x, w, b)
    pk = O.wino8_pack(w)
    for i in range(B):
        assert same16(got[i], O.wino8(x[i], pk, b)), i


def test_bad_params(hip):
    H_ = hip
    w = np.zeros((20, 3, 3, 8), np.float32)
    b = np.zeros(20, np.float32)
    assert not H_.lib().bnh_wino8_new(8, 20, w.ctypes.data, b.ctypes.data)
    assert b"K % 16 == 0" in H_.lib().bnh_last_error()
