"""Pins the oracle's restatement of the dotprod family's STEM3 (oracle/dot.c, stem_conv_f32_h of
src/kern_f16.c:15-71) without re-typing it:
  * index layout: a single unit weight at tap (ky, kx, ci) of channel co moves exactly that input value, rounded
    to fp16 and through the table SiLU (pinned on all inputs in test_oracle_s8n / the fp16 tests), to (oy, ox, co);
  * the edge rule: taps past the bottom / right edge are skipped, so the last row / column of outputs sees only
    the bias where the weights sit on ky = 2 / kx = 2;
  * the chain order: on operands chosen so that the fp32 roundings depend on the order, the result equals a
    sequential FMA chain over (ky, kx, ci) from the bias, computed here with exact rationals and one round to
    nearest even per step; a chain in another order gives a different value;
  * magnitude: random inputs against a float64 direct convolution within fp16 rounding."""
from fractions import Fraction

import numpy as np

import pyoracle as O


def f32_rne(q):
    """The fp32 nearest-even rounding of a rational (normal range)."""
    if q == 0:
        return 0.0
    s = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    scale = Fraction(2) ** (23 - e)
    m = a * scale
    f = m.numerator // m.denominator
    r = m - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2):
        f += 1
    return s * float(Fraction(f) / scale)


def h(x):
    return np.float16(x)


def silu_h(v):
    return O.lib().orc_silu_lut_h(int(np.array([v], np.float16).view(np.uint16)[0]))


def test_stem3_layout_one_tap_at_a_time():
    rng = np.random.default_rng(1)
    H, W = 6, 8
    img = rng.standard_normal((H, W, 3)).astype(np.float32)
    for (ky, kx, ci, co) in ((0, 0, 0, 0), (1, 2, 1, 7), (2, 1, 2, 23), (2, 2, 0, 12)):
        w = np.zeros((24, 3, 3, 3), np.float32)
        w[co, ky, kx, ci] = 1.0
        out = O.stem3(img, w, np.zeros(24, np.float32))
        for oy in range(H // 2):
            for ox in range(W // 2):
                iy, ix = 2 * oy + ky, 2 * ox + kx
                v = img[iy, ix, ci] if iy < H and ix < W else 0.0
                want = silu_h(h(v))
                assert int(out[oy + 1, ox + 1, co].view(np.uint16)) == want, (ky, kx, ci, co, oy, ox)
        assert not out[0].any() and not out[-1].any() and not out[:, 0].any() and not out[:, -1].any()


def test_stem3_edges_skip_taps():
    """Weights on ky = 2 only: the last output row (its ky = 2 taps past the image) is the bias alone; likewise
    kx = 2 and the last column."""
    rng = np.random.default_rng(2)
    H, W = 8, 10
    img = (rng.standard_normal((H, W, 3)) + 3).astype(np.float32)
    b = rng.standard_normal(24).astype(np.float32)
    for axis in (0, 1):
        w = np.zeros((24, 3, 3, 3), np.float32)
        if axis == 0:
            w[:, 2, :, :] = 1.0
        else:
            w[:, :, 2, :] = 1.0
        out = O.stem3(img, w, b)[1:-1, 1:-1]
        edge = out[-1] if axis == 0 else out[:, -1]
        for co in range(24):
            assert (edge[..., co].view(np.uint16) == silu_h(h(b[co]))).all()
        inner = out[0] if axis == 0 else out[:, 0]
        assert not (inner.view(np.uint16) == np.array([silu_h(h(x)) for x in b], np.uint16)).all()


def test_stem3_chain_order():
    """Cancelling operands: a 2 x 2 image of ones (output (0, 0) reads 12 taps, the products are the weights),
    +2^16 on tap (0, 0, 0), -2^16 on tap (1, 1, 0), small values elsewhere. The oracle equals the sequential
    (ky, kx, ci) FMA chain from the bias computed with exact rationals (the small terms between the two large ones
    rounded at 2^16's scale); the (ci, ky, kx) order, where -2^16 comes fourth, gives other fp16 results."""
    rng = np.random.default_rng(3)
    H, W = 2, 2
    img = np.ones((H, W, 3), np.float32)
    w = np.zeros((24, 3, 3, 3), np.float32)
    w[:, :2, :2, :] = rng.uniform(0.1, 1.0, (24, 2, 2, 3)).astype(np.float32)
    w[:, 0, 0, 0] = 2.0 ** 16
    w[:, 1, 1, 0] = -(2.0 ** 16)
    b = rng.uniform(-0.5, 0.5, 24).astype(np.float32)
    out = O.stem3(img, w, b)
    taps = [(ky, kx, ci) for ky in range(2) for kx in range(2) for ci in range(3)]

    def chain(co, order):
        acc = Fraction(float(b[co]))
        for (ky, kx, ci) in order:
            acc = Fraction(f32_rne(Fraction(float(w[co, ky, kx, ci])) + acc))
        return np.float32(float(acc))
    differ = 0
    for co in range(24):
        want = chain(co, taps)
        other = chain(co, sorted(taps, key=lambda t: (t[2], t[0], t[1])))
        assert int(out[1, 1, co].view(np.uint16)) == silu_h(h(want)), co
        differ += silu_h(h(want)) != silu_h(h(other))
    assert differ >= 12  # a chain in the other order fails most channels


def test_stem3_against_float64():
    rng = np.random.default_rng(4)
    H, W = 10, 14
    img = rng.standard_normal((H, W, 3)).astype(np.float32)
    w = (rng.standard_normal((24, 3, 3, 3)) * 0.5).astype(np.float32)
    b = (rng.standard_normal(24) * 0.1).astype(np.float32)
    out = O.stem3(img, w, b)[1:-1, 1:-1].astype(np.float64)
    xp = np.zeros((H + 2, W + 2, 3))
    xp[:H, :W] = img
    y = np.zeros((H // 2, W // 2, 24))
    for ky in range(3):
        for kx in range(3):
            y += np.einsum("hwc,oc->hwo", xp[ky:ky + H:2, kx:kx + W:2], w[:, ky, kx, :].astype(np.float64))
    y += b
    s = y / (1 + np.exp(-y))
    assert np.abs(out - s).max() <= 2e-3 * max(1.0, np.abs(s).max())
