"""Pins the CPU oracle of the int8 GEMM path (oracle/s8n.c) before it is
trusted as the checker: Arm ARM known answers for FRECPE, closed forms of the
SiLU and of per-row quantization, brute-force integer GEMMs and the gemmlowp
fixed-point identities of the Q31 requant specification.
"""
import math
import struct

import numpy as np
import pytest

import pyoracle as O
from bnneon import s8pack


def f32(x):
    return float(np.float32(x))


def bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


# ------------------------------------------------------------------ FRECPE
def test_frecpe_known_answers():
    L = O.lib()
    # FRECPE(1.0) = 511/512 (the largest 9-bit estimate of [1, 2))
    assert L.orc_frecpe(1.0) == 0.998046875
    assert L.orc_frecpe(2.0) == 0.998046875 / 2
    assert L.orc_frecpe(-4.0) == -0.998046875 / 4
    # 1.5: a = 2*384+1 = 769, 2^19 // 769 = 681, (681+1)//2 = 341 -> 1.33203125 / 2
    assert L.orc_frecpe(1.5) == 0.666015625
    assert L.orc_frecpe(0.0) == math.inf
    assert L.orc_frecpe(-0.0) == -math.inf
    assert L.orc_frecpe(math.inf) == 0.0
    assert math.isnan(L.orc_frecpe(math.nan))
    # below 2^-128 the reciprocal overflows: infinity (round to nearest)
    assert L.orc_frecpe(2.0 ** -129) == math.inf


def test_frecpe_estimate_bounds_every_index():
    """Every one of the 256 significand indices: 9-bit estimate of 1/x,
    relative error below 2^-8, and monotone non-increasing in x."""
    L = O.lib()
    prev = None
    for i in range(256):
        x = f32(1.0 + (i + 0.5) / 256)  # middle of interval i
        r = L.orc_frecpe(x)
        assert abs(r * x - 1) < 2 ** -8, (i, x, r)
        # the result carries 8 fraction bits only
        assert bits(r) & 0x7fff == 0
        if prev is not None:
            assert r <= prev
        prev = r


def test_frecpe_exponent_scaling():
    L = O.lib()
    rng = np.random.default_rng(0)
    for m in rng.uniform(1, 2, 64).astype(np.float32):
        base = L.orc_frecpe(float(m))
        for e in range(-100, 100, 7):
            x = float(np.float32(m) * np.float32(2.0 ** e))
            assert L.orc_frecpe(x) == f32(base * 2.0 ** -e)


def test_frecpe_denormal_results_and_operands():
    L = O.lib()
    # operand 2^126 * 1.0: result exponent 253 - 253 = 0 -> denormal 0.998046875 * 2^-126
    x = 2.0 ** 126
    assert L.orc_frecpe(x) == f32(0.998046875 * 2.0 ** -126)
    # denormal operand 2^-127 (exp field 0, top fraction bit set): 1/x ~ 2^127
    assert L.orc_frecpe(2.0 ** -127) == f32(0.998046875 * 2.0 ** 127)


# ------------------------------------------------------------------ SiLU
def test_silu_closed_forms():
    L = O.lib()
    assert L.orc_silu_f32(0.0) == 0.0
    # t <= -60: 2^t + 1 rounds to 1; FRECPE(1) = 511/512, one Newton step gives
    # 511/512 * 513/512 = 1 - 2^-18 exactly: silu(x) = x * (1 - 2^-18)
    for x in (41.6, 100.0, 1e6, 3e38):
        assert L.orc_silu_f32(x) == f32(np.float32(x) * np.float32(1 - 2 ** -18))
    # t >= 60: d = 1 + 2^60; the product underflows towards 0 (x / 2^60)
    assert abs(L.orc_silu_f32(-100.0)) < 1e-15
    assert math.isnan(L.orc_silu_f32(math.nan))


def test_silu_accuracy_against_exact():
    """FRECPE + one Newton step: relative error of the gate ~ (2^-9)^2."""
    L = O.lib()
    xs = np.linspace(-30, 30, 4001).astype(np.float32)
    for x in xs:
        y = L.orc_silu_f32(float(x))
        ex = float(x) / (1 + math.exp(-float(x)))
        assert abs(y - ex) <= 2e-5 * abs(ex) + 1e-30, (x, y, ex)


# ------------------------------------------------------------------ conversions
def test_conversions_saturate_like_aarch64():
    L = O.lib()
    assert L.orc_cvtn_s32(2.5) == 2 and L.orc_cvtn_s32(3.5) == 4
    assert L.orc_cvtn_s32(-2.5) == -2
    assert L.orc_cvta_s32(2.5) == 3 and L.orc_cvta_s32(-2.5) == -3
    assert L.orc_cvtn_s32(3e9) == 2 ** 31 - 1 and L.orc_cvtn_s32(-3e9) == -2 ** 31
    assert L.orc_cvtn_s32(math.nan) == 0
    # lrintf: 64-bit saturating conversion, low 32 bits kept
    assert L.orc_lrintf_s32(3e9) == 3000000000 - 2 ** 32
    assert L.orc_lrintf_s32(1e20) == -1
    assert L.orc_lrintf_s32(-1e20) == 0
    assert L.orc_fmax(-0.0, 0.0) == 0.0 and math.copysign(1, L.orc_fmax(-0.0, 0.0)) > 0
    assert math.isnan(L.orc_fmax(math.nan, 1.0)) and math.isnan(L.orc_fmin(1.0, math.nan))


# ------------------------------------------------------------------ quantization
def test_quant_rows_hand_example():
    # row [0 1 2 3] (K = 4: min/max from the 4-lane loop, values from the
    # lrintf tail): inv = 254/3, z = -127, q = [-127 -42 42 127], pad = z
    q, sa, za = O.quant_rows(np.array([[0, 1, 2, 3]], np.float32), 4, 16)
    assert q[0, :4].tolist() == [-127, -42, 42, 127]
    assert q[0, 4:].tolist() == [-127] * 12
    assert za[0] == -127 and sa[0] == np.float32(3) / np.float32(254)


def test_quant_rows_constant_row():
    x = np.full((2, 24), -0.75, np.float32)
    x[1] = 0
    q, sa, za = O.quant_rows(x, 24, 32)
    assert (q[0, :24] == -127).all() and za[0] == 0
    assert sa[0] == np.float32(0.75) / np.float32(127)
    # an all-zero row: a = 1e-30, every byte 0
    assert (q[1] == 0).all() and za[1] == 0 and sa[1] == np.float32(1e-30) / np.float32(127)


def test_quant_rows_extremes_and_roundtrip():
    rng = np.random.default_rng(1)
    for K in (1, 3, 7, 8, 13, 40, 144, 1152):
        Kp = s8pack.r16(K)
        x = (rng.standard_normal((16, K)) * rng.uniform(0.01, 100, (16, 1))
             + rng.uniform(-5, 5, (16, 1))).astype(np.float32)
        q, sa, za = O.quant_rows(x, K, Kp)
        assert q.min() >= -127
        for m in range(16):
            if K < 2:
                continue
            lo, hi = int(np.argmin(x[m])), int(np.argmax(x[m]))
            assert q[m, lo] == -127 and q[m, hi] == 127
            deq = (q[m, :K].astype(np.float64) - za[m]) * float(sa[m])
            assert np.abs(deq - x[m]).max() <= 0.5001 * float(sa[m]) + 1e-6 * np.abs(x[m]).max()
            assert (q[m, K:] == np.int8(np.uint8(za[m] & 0xff))).all()


def test_quant_rows_gate_equals_gating_first():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((8, 64)).astype(np.float32)
    g = rng.uniform(0, 1, 64).astype(np.float32)
    a = O.quant_rows(x, 64, 64, gate=g)
    b = O.quant_rows(x * g, 64, 64)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


# ------------------------------------------------------------------ GEMM + epilogue
def _tiny_case(rng, M, K, N):
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((N, K)).astype(np.float32) * 0.1
    b = rng.standard_normal(N).astype(np.float32)
    return x, w, b, s8pack.pack_s8(w, b)


def test_gemm_int_sums_brute_force():
    """The oracle's y equals an independent numpy restatement built from the
    unpacked weights (pins the panel layout and the epilogue's op order)."""
    rng = np.random.default_rng(3)
    for M, K, N in ((5, 7, 3), (9, 40, 24), (17, 144, 33)):
        x, w, b, pk = _tiny_case(rng, M, K, N)
        _, K_, Kp, Np = pk["shape"]
        out, q, sa, za = O.pw_s8(x, pk)
        wq = s8pack.unpack_panels(pk["q"], Np, Kp).astype(np.int64)
        acc = q[:M].astype(np.int64) @ wq.T
        c = (acc - za[:M, None].astype(np.int64) * pk["cs"][None, :Np]).astype(np.int32)
        s = (pk["sw"][None, :Np] * sa[:M, None]).astype(np.float32)
        y = (c.astype(np.float32) * s).astype(np.float32) + pk["b"][None, :Np]
        assert np.array_equal(out[:, :Np], y.astype(np.float32))


def test_gemm_zero_weights_give_bias():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((6, 32)).astype(np.float32)
    b = rng.standard_normal(8).astype(np.float32)
    pk = s8pack.pack_s8(np.zeros((8, 32), np.float32), b)
    out, *_ = O.pw_s8(x, pk)
    assert np.array_equal(out, np.broadcast_to(b, out.shape))
    out, *_ = O.pw_s8(x, pk, act=2)
    assert np.array_equal(out, np.broadcast_to(np.maximum(b, 0), out.shape))


def test_gemm_dequant_approximates_float_gemm():
    rng = np.random.default_rng(5)
    x, w, b, pk = _tiny_case(rng, 64, 96, 40)
    out, *_ = O.pw_s8(x, pk)
    ref = x.astype(np.float64) @ w.T.astype(np.float64) + b
    err = np.abs(out[:, :40] - ref).max()
    assert err < 0.05 * np.abs(ref).max()


def test_epilogue_residual_and_padded_store():
    rng = np.random.default_rng(6)
    H, W = 3, 4
    x, w, b, pk = _tiny_case(rng, H * W, 24, 16)
    res = rng.standard_normal((H * W, 16)).astype(np.float32)
    plain, *_ = O.pw_s8(x, pk, act=1)
    with_res, *_ = O.pw_s8(x, pk, act=1, res=res, ldr=16)
    assert np.array_equal(with_res, (plain + res).astype(np.float32))
    padded, *_ = O.pw_s8(x, pk, act=1, ow=W, opad=2)
    img = padded.reshape(H + 4, W + 4, 16)
    assert np.array_equal(img[2:2 + H, 2:2 + W].reshape(H * W, 16), plain)
    img[2:2 + H, 2:2 + W] = 0
    assert not img.any()


# ------------------------------------------------------------------ Q31 requant spec
def _srdhm_exact(a, b):
    """(2ab + 2^31 rounding) / 2^32 by Python integers, ties away from zero."""
    if a == b == -2 ** 31:
        return 2 ** 31 - 1
    ab = a * b
    nudge = 2 ** 30 if ab >= 0 else 1 - 2 ** 30
    v = ab + nudge
    return int(v / 2 ** 31) if abs(v) < 2 ** 52 else (abs(v) // 2 ** 31) * (1 if v >= 0 else -1)


def test_requant_fixed_point_identities():
    L = O.lib()
    assert L.orc_srdhm(-2 ** 31, -2 ** 31) == 2 ** 31 - 1
    assert L.orc_srdhm(2 ** 30, 2 ** 30) == 2 ** 29
    # x * 0.5 in Q31 doubling-high-mul is x / 2 rounded to nearest, ties
    # upwards (gemmlowp's nudge 1 - 2^30 for negative products: -2.5 -> -2)
    for x in (-5, -3, -1, 1, 3, 5, 1001):
        assert L.orc_srdhm(x, 2 ** 30) == math.floor(x / 2 + 0.5)
    # RoundingDivideByPOT rounds half away from zero
    for x, e, want in ((5, 1, 3), (-5, 1, -3), (4, 1, 2), (-3, 1, -2), (6, 2, 2), (-6, 2, -2), (7, 3, 1)):
        assert L.orc_rdbypot(x, e) == want, (x, e)
    rng = np.random.default_rng(7)
    for _ in range(2000):
        a = int(rng.integers(-2 ** 31, 2 ** 31))
        m = int(rng.integers(2 ** 30, 2 ** 31))
        s = int(rng.integers(0, 12))
        exact = a * m / 2 ** (31 + s)
        v = L.orc_rdbypot(L.orc_srdhm(a, m), s)
        assert abs(v - exact) <= 1.0  # two roundings: within one unit
        assert L.orc_srdhm(a, m) == _srdhm_exact(a, m)


def test_requant_gemm_brute_force():
    rng = np.random.default_rng(8)
    N, K, M = 6, 48, 12
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    x = rng.integers(-128, 128, (K, M)).astype(np.int8)
    bias = rng.integers(-2 ** 14, 2 ** 14, N).astype(np.int32)
    mult = rng.integers(2 ** 30, 2 ** 31, N).astype(np.int32)
    shift = rng.integers(6, 11, N).astype(np.int32)
    out = O.gemm_s8_requant(w, x, bias, mult, shift, -128, -128)
    acc = w.astype(np.int64) @ (x.astype(np.int64) + 128) + bias[:, None]
    L = O.lib()
    for n in range(N):
        for m in range(M):
            y = L.orc_rdbypot(_srdhm_exact(int(acc[n, m]), int(mult[n])), int(shift[n])) - 128
            assert out[n, m] == max(-128, min(127, y))


# ------------------------------------------------------------------ discriminating closed forms (exact arithmetic)
def _f32_rne(fr):
    """The fp32 nearest to a Fraction (ties to even), normal and subnormal range, computed in integers."""
    from fractions import Fraction
    fr = Fraction(fr)
    if fr == 0:
        return 0.0
    sign, a = (-1 if fr < 0 else 1), abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    quantum = Fraction(2) ** (max(e, -126) - 23)          # one ulp at this exponent (2^-149 for subnormals)
    q, r = divmod(a, quantum)
    if r * 2 > quantum or (r * 2 == quantum and q % 2 == 1):
        q += 1
    return float(np.float32(sign * float(q * quantum)))


def test_f32_rne_helper_against_numpy():
    from fractions import Fraction
    rng = np.random.default_rng(0)
    for _ in range(2000):
        a, b = rng.standard_normal(2).astype(np.float32)
        assert _f32_rne(Fraction(float(a)) * Fraction(float(b))) == float(np.float32(a) * np.float32(b))
        assert _f32_rne(Fraction(float(a)) + Fraction(float(b))) == float(np.float32(a) + np.float32(b))


def _integer_t_inputs():
    """fp32 x where t = fl(x * -1.44269504f) is an exact integer n (then the exp2 split has f = 0, p = 1)."""
    c = np.float32(-1.44269504)
    out = []
    for n in list(range(-23, -8)) + list(range(9, 60)):
        x0 = np.float32(n / float(c))
        for k in range(-64, 65):
            x = np.nextafter(x0, np.float32(np.inf) if k > 0 else np.float32(-np.inf)) if k else x0
            for _ in range(abs(k) - 1):
                x = np.nextafter(x, np.float32(np.inf) if k > 0 else np.float32(-np.inf))
            if float(np.float32(x) * c) == float(n):
                out.append((float(x), n))
                break
    return out


def test_silu_where_t_is_an_integer():
    """SiLU(x) = x * r with d = 1 + 2^n exactly rounded, r0 = FRECPE(d) = 511/512 * 2^-E (the published FRECPE(1.0),
    scaled by d's binary exponent E: for these n the top 8 fraction bits of d are 0), and one Newton step
    r = r0 * fl(2 - d r0). A slip in the magic-number split, the exponent shift, the clamp or the step shows here."""
    from fractions import Fraction
    L = O.lib()
    cases = _integer_t_inputs()
    assert len(cases) >= 40, len(cases)
    for x, n in cases:
        d = _f32_rne(1 + Fraction(2) ** n)
        E = math.frexp(d)[1] - 1
        r0 = Fraction(511, 512) / Fraction(2) ** E
        s = _f32_rne(2 - Fraction(d) * r0)
        r = _f32_rne(r0 * Fraction(s))
        want = _f32_rne(Fraction(x) * Fraction(r))
        assert L.orc_silu_f32(x) == want, (x, n)


def test_frecps_is_one_fused_rounding():
    """FRECPS(d, r) = fl(2 - d r) with one rounding (FPRecipStepFused), not fl(2 - fl(d r)): on random operands of
    the SiLU's range the two differ, and the oracle gives the fused value every time."""
    from fractions import Fraction
    L = O.lib()
    rng = np.random.default_rng(12)
    d = (1 + rng.uniform(0, 2 ** 20, 3000)).astype(np.float32)
    r = np.array([L.orc_frecpe(float(v)) for v in d], np.float32)
    differ = 0
    for dv, rv in zip(d, r):
        fused = _f32_rne(2 - Fraction(float(dv)) * Fraction(float(rv)))
        assert L.orc_frecps(float(dv), float(rv)) == fused
        differ += _f32_rne(2 - Fraction(_f32_rne(Fraction(float(dv)) * Fraction(float(rv))))) != fused
    assert differ > 100, differ


def test_dequant_order_discriminated():
    """y = fl(fl(f * fl(sw * sa)) + b) (src/gemm_s8n.c:105-114: vmulq(vcvtq(acc), vmulq(sw, sa)), then + b, three
    roundings, no fusion), checked in exact arithmetic on entries where the other orders give other floats."""
    from fractions import Fraction
    rng = np.random.default_rng(8)
    M, K, N = 48, 72, 40
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 30, (M, 1))).astype(np.float32)
    w = (rng.standard_normal((N, K)) * rng.uniform(0.01, 3, (N, 1))).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) * 5
    pk = s8pack.pack_s8(w, b)
    _, _, Kp, Np = pk["shape"]
    out, q, sa, za = O.pw_s8(x, pk)
    wq = s8pack.unpack_panels(pk["q"], Np, Kp).astype(np.int64)
    acc = q[:M].astype(np.int64) @ wq.T - za[:M, None].astype(np.int64) * pk["cs"][None, :Np]
    F = Fraction
    decisive = 0
    for m in range(M):
        for n in range(N):
            f = _f32_rne(F(int(acc[m, n])))
            sw_, sa_, bb = float(pk["sw"][n]), float(sa[m]), float(pk["b"][n])
            ref = _f32_rne(F(_f32_rne(F(f) * F(_f32_rne(F(sw_) * F(sa_))))) + F(bb))
            others = {
                _f32_rne(F(_f32_rne(F(_f32_rne(F(f) * F(sw_))) * F(sa_))) + F(bb)),
                _f32_rne(F(_f32_rne(F(_f32_rne(F(f) * F(sa_))) * F(sw_))) + F(bb)),
                _f32_rne(F(f) * F(_f32_rne(F(sw_) * F(sa_))) + F(bb)),
            }
            assert float(out[m, n]) == ref, (m, n)
            decisive += ref not in others
    assert decisive >= 100, decisive
