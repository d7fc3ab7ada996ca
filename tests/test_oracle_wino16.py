"""Pins the fp16 Winograd (CONV3C24) oracle (oracle/wino16.c, restating
src/wino_s0.c): the half-precision FRECPE against the fp32 estimate (pinned
exhaustively elsewhere) on every normal and near-normal half, its special cases,
FRECPS against a fused 2 - a b, the polynomial SiLU within its fp16 accuracy of
the exact function, and the whole convolution against a float64 direct
convolution + SiLU + residual within the fp16 accumulation bound."""
import math

import numpy as np

import pyoracle as O


def hb(v):
    return int(np.array([v], np.float16).view(np.uint16)[0])


def hv(b):
    return float(np.array([b], np.uint16).view(np.float16)[0])


def test_frecpe_h_matches_fp32_estimate():
    L = O.lib()
    for b in range(0x0100, 0x7c00):          # every positive normal half and the denormals >= 2^-16
        for s in (0, 0x8000):
            h = b | s
            f32 = L.orc_frecpe(hv(h))
            want = L.orc_f2h(f32)
            assert L.orc_frecpe_h(h) == want, hex(h)
    assert L.orc_frecpe_h(0x0000) == 0x7c00 and L.orc_frecpe_h(0x8000) == 0xfc00
    assert L.orc_frecpe_h(0x00ff) == 0x7c00    # below 2^-16: overflow to infinity
    assert L.orc_frecpe_h(0x7c00) == 0x0000 and L.orc_frecpe_h(0xfc00) == 0x8000
    assert L.orc_frecpe_h(hb(1.0)) == hb(511 / 512)


def test_frecps_h():
    L = O.lib()
    assert L.orc_frecps_h(0x7c00, 0) == hb(2.0) and L.orc_frecps_h(0, 0xfc00) == hb(2.0)
    rng = np.random.default_rng(0)
    for a, b in rng.standard_normal((2000, 2)).astype(np.float16):
        assert L.orc_frecps_h(hb(a), hb(b)) == L.orc_h_fma(hb(-a), hb(b), hb(2.0))


def test_silu_poly_accuracy():
    L = O.lib()
    worst = 0.0
    for x in np.arange(-16, 16, 1 / 256).astype(np.float16):
        y = hv(L.orc_silu_poly_h(hb(x)))
        ex = float(x) / (1 + math.exp(-float(x)))
        worst = max(worst, abs(y - ex) / max(1.0, abs(ex)))
    assert worst < 2e-3, worst


def test_conv_against_direct():
    rng = np.random.default_rng(1)
    H, W = 8, 12
    xp = np.zeros((H + 2, W + 2, 24), np.float16)
    xp[1:-1, 1:-1] = rng.standard_normal((H, W, 24))
    w = (rng.standard_normal((24, 3, 3, 24)) * math.sqrt(2 / 216)).astype(np.float32)
    b = (rng.standard_normal(24) * 0.1).astype(np.float32)
    out = O.wino_s0(xp, w, b).astype(np.float64)
    x64 = xp.astype(np.float64)
    cols = np.stack([x64[ky:ky + H, kx:kx + W] for ky in range(3) for kx in range(3)], axis=2)
    y = cols.reshape(H * W, -1) @ w.reshape(24, -1).T.astype(np.float64) + b
    ref = (y / (1 + np.exp(-y))).reshape(H, W, 24) + x64[1:-1, 1:-1]
    assert not out[0].any() and not out[-1].any()
    err = np.abs(out[1:-1, 1:-1] - ref)
    assert err.max() < 0.05 * max(1.0, np.abs(ref).max()), err.max()
