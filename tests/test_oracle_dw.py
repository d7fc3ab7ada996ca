"""Pins the depthwise oracle (oracle/dw.c): its exact fp16 arithmetic against
independent implementations (numpy's float16 add / multiply, which round a
float32 result that is exact or double-rounding-safe; Fraction arithmetic for
the fused multiply-add), the fp16 LUT SiLU against the exact function within
the reference's stated error, and the depthwise convolutions against closed
forms (identity taps, constant inputs) and a float64 direct convolution."""
import math
from fractions import Fraction

import numpy as np
import pytest

import pyoracle as O


def hbits(x):
    return int(np.array([x], np.float16).view(np.uint16)[0])


def hval(b):
    return np.array([b], np.uint16).view(np.float16)[0]


def random_halves(rng, n):
    b = rng.integers(0, 1 << 16, n).astype(np.uint16)
    v = b.view(np.float16)
    return b[np.isfinite(v)]


def test_fp16_add_mul_match_numpy():
    L = O.lib()
    rng = np.random.default_rng(0)
    a, b = random_halves(rng, 20000), random_halves(rng, 20000)
    n = min(len(a), len(b))
    for x, y in zip(a[:n], b[:n]):
        hx, hy = hval(x), hval(y)
        with np.errstate(all="ignore"):
            s, p = np.float16(hx + hy), np.float16(hx * hy)
        gs, gp = hval(L.orc_h_add(int(x), int(y))), hval(L.orc_h_mul(int(x), int(y)))
        assert (np.isnan(s) and np.isnan(gs)) or s.view(np.uint16) == gs.view(np.uint16), (hx, hy)
        assert (np.isnan(p) and np.isnan(gp)) or p.view(np.uint16) == gp.view(np.uint16), (hx, hy)


def round_fp16(q):
    """The fp16 value nearest to the Fraction q (ties to even), as bits."""
    if q == 0:
        return 0
    guess = np.float16(float(q))
    best = None
    b0 = int(guess.view(np.uint16))
    for b in (b0 - 1, b0, b0 + 1):
        if b < 0 or b > 0xffff:
            continue
        v = hval(b)
        if not np.isfinite(v):
            continue
        d = abs(Fraction(float(v)) - q)
        key = (d, int(b) & 1)
        if best is None or key < best[0]:
            best = (key, b)
    return best[1]


def test_fp16_fma_exact_rounding():
    L = O.lib()
    rng = np.random.default_rng(1)
    # moderate exponents so that nothing overflows: fractions stay exact
    vals = (rng.standard_normal(6000) * rng.choice([1e-4, 1e-2, 1, 30], 6000)).astype(np.float16)
    vals = vals.view(np.uint16)
    for i in range(0, len(vals) - 2, 3):
        a, b, c = (int(v) for v in vals[i:i + 3])
        q = Fraction(float(hval(a))) * Fraction(float(hval(b))) + Fraction(float(hval(c)))
        if abs(q) > 65000:
            continue
        got = L.orc_h_fma(a, b, c)
        want = round_fp16(q)
        if q == 0:
            assert got & 0x7fff == 0
        else:
            assert got == want, (hval(a), hval(b), hval(c))
    # denormal products and a tie that rounds to even
    assert L.orc_h_fma(hbits(2 ** -14), hbits(2 ** -6), 0) == 1 << 4   # 2^-20: denormal, exact
    assert L.orc_h_fma(hbits(1.0), hbits(1.0), hbits(2 ** -11)) == hbits(1.0)  # 1 + 2^-11: tie -> even (1.0)


def test_silu_lut_accuracy_and_closed_forms():
    L = O.lib()
    xs = np.linspace(-8, 8, 3201).astype(np.float16)
    err = 0.0
    for x in xs:
        y = float(hval(L.orc_silu_lut_h(hbits(x))))
        ex = float(x) / (1 + math.exp(-float(x)))
        err = max(err, abs(y - ex))
    assert err < 5e-3    # the reference states 4.2e-3 max abs error on [-8, 8] (src/silu_lut.h:7-8)
    assert L.orc_silu_lut_h(0) == 0
    big = hbits(100.0)
    assert hval(L.orc_silu_lut_h(big)) == np.float16(100.0)  # |x| q(15.4) is below half an ulp of 100


def make_dw(rng, H, W, C, k, dtype):
    h = (k - 1) // 2
    xp = np.zeros((H + 2 * h, W + 2 * h, C), dtype)
    xp[h:h + H, h:h + W] = rng.standard_normal((H, W, C)).astype(dtype)
    w = (rng.standard_normal((k * k, C)) * math.sqrt(2 / (k * k))).astype(dtype)
    b = rng.standard_normal(C).astype(dtype) * 0.1
    return xp, w, b.astype(dtype)


@pytest.mark.parametrize("k,s", [(3, 1), (3, 2), (5, 1), (5, 2), (7, 1)])
def test_dwk_f32_identity_and_direct(k, s):
    rng = np.random.default_rng(k * 10 + s)
    H, W, C = 9, 11, 16
    h = (k - 1) // 2
    pt = pl = h if s == 1 else h - 1 if h else 0
    Ho, Wo = (H + pt + h - k) // s + 1, (W + pl + h - k) // s + 1
    xp, w, b = make_dw(rng, H, W, C, k, np.float32)
    ident = np.zeros_like(w)
    ident[(k * k) // 2] = 1
    out, cs = O.dwk_f32(xp, H, W, C, k, s, h, h, ident, np.zeros(C, np.float32), 0, (H - 1) // s + 1, (W - 1) // s + 1)
    assert np.array_equal(out, xp[h:h + H:s, h:h + W:s])
    out, cs = O.dwk_f32(xp, H, W, C, k, s, pt, pl, w, b, 1, Ho, Wo)
    ref = np.zeros((Ho, Wo, C))
    for oy in range(Ho):
        for ox in range(Wo):
            patch = xp[oy * s - pt + h:oy * s - pt + h + k, ox * s - pl + h:ox * s - pl + h + k].reshape(k * k, C)
            ref[oy, ox] = (patch.astype(np.float64) * w).sum(0) + b
    ref = ref / (1 + np.exp(-ref))
    assert np.abs(out - ref).max() < 1e-4 * np.abs(ref).max() + 1e-5
    assert np.allclose(cs, out.reshape(-1, C).sum(0), rtol=1e-5, atol=1e-4)


def test_dwk_f32_chsum_grouping_closed_form():
    # constant outputs 2^-3 everywhere (zero input, bias 0.125, no act): every partial sum is exact
    H, W, C, k = 4, 7, 8, 3
    xp = np.zeros((H + 2, W + 2, C), np.float32)
    out, cs = O.dwk_f32(xp, H, W, C, k, 1, 1, 1, np.ones((9, C), np.float32), np.full(C, 0.125, np.float32), 0, H, W)
    assert (out == 0.125).all() and (cs == 0.125 * H * W).all()


def test_dw3_f32_identity_is_silu():
    rng = np.random.default_rng(5)
    H, W, C = 6, 10, 8
    xp, _, _ = make_dw(rng, H, W, C, 3, np.float32)
    w = np.zeros((9, C), np.float32)
    w[4] = 1
    out, cs = O.dw3_f32(xp, H, W, C, 1, w, np.zeros(C, np.float32), H, W)
    inner = xp[1:1 + H, 1:1 + W]
    assert np.array_equal(out, O.eval_f32(1, inner).reshape(out.shape))
    seq = np.zeros(C, np.float32)
    for v in out.reshape(-1, C):
        seq = (seq + v).astype(np.float32)
    assert np.array_equal(cs, seq)


@pytest.mark.parametrize("k,s", [(3, 1), (5, 2)])
def test_dwk_f16_close_to_f32(k, s):
    rng = np.random.default_rng(k + s)
    H, W, C = 8, 13, 16
    h = (k - 1) // 2
    Ho, Wo = (H - 1) // s + 1, (W - 1) // s + 1
    xp, w, b = make_dw(rng, H, W, C, k, np.float32)
    o32, cs32 = O.dwk_f32(xp, H, W, C, k, s, h, h, w, b, 1, Ho, Wo)
    o16, cs16 = O.dwk_f16(xp.astype(np.float16), H, W, C, k, s, h, h, w.astype(np.float16), b.astype(np.float16), 1,
                          Ho, Wo)
    assert np.abs(o16.astype(np.float32) - o32).max() < 3e-2
    assert np.abs(cs16 - cs32).max() < 0.05 * np.abs(cs32).max() + 0.1


def test_dw3_f16_identity_is_lut_silu():
    rng = np.random.default_rng(6)
    H, W, C = 5, 9, 8
    xp, _, _ = make_dw(rng, H, W, C, 3, np.float16)
    w = np.zeros((9, C), np.float16)
    w[4] = 1
    out, cs = O.dw3_f16(xp, H, W, C, 1, 1, 1, w, np.zeros(C, np.float16), H, W)
    L = O.lib()
    inner = xp[1:1 + H, 1:1 + W].reshape(-1)
    want = np.array([L.orc_silu_lut_h(int(v)) for v in inner.view(np.uint16)], np.uint16).view(np.float16)
    assert np.array_equal(out.reshape(-1).view(np.uint16), want.view(np.uint16))


def test_dw_s8_brute_force():
    rng = np.random.default_rng(7)
    H, W, C, k, s, pt, pl = 6, 7, 8, 5, 2, 1, 2
    Ho, Wo = (H + pt + 2 - k) // s + 1, (W + pl + 2 - k) // s + 1
    x = rng.integers(-128, 128, (H, W, C)).astype(np.int8)
    w = rng.integers(-127, 128, (k * k, C)).astype(np.int8)
    bias = rng.integers(-5000, 5000, C).astype(np.int32)
    mult = rng.integers(2 ** 30, 2 ** 31, C).astype(np.int32)
    shift = rng.integers(4, 9, C).astype(np.int32)
    lut = rng.integers(-128, 128, 256).astype(np.int8)
    out = O.dw_s8(x, k, s, pt, pl, w, bias, mult, shift, -128, -3, -128, 127, lut, Ho, Wo)
    plain = O.dw_s8(x, k, s, pt, pl, w, bias, mult, shift, -128, -3, -128, 127, None, Ho, Wo)
    L = O.lib()
    for oy in range(Ho):
        for ox in range(Wo):
            for c in range(C):
                acc = int(bias[c])
                for ky in range(k):
                    for kx in range(k):
                        iy, ix = oy * s - pt + ky, ox * s - pl + kx
                        if 0 <= iy < H and 0 <= ix < W:
                            acc += int(w[ky * k + kx, c]) * (int(x[iy, ix, c]) + 128)
                y = L.orc_requant(acc, int(mult[c]), int(shift[c]), -3, -128, 127)
                assert plain[oy, ox, c] == y and out[oy, ox, c] == lut[y + 128]
