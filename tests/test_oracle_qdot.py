"""Pins the CPU oracle of the dotprod family's int8 arithmetic (oracle/qdot.c) before it is trusted as the checker:
the weight packing and quantisation parameters against hand examples and an independent numpy statement, the
fp16 quantisation's single fp16 rounding against numpy's float16, the GEMM epilogue's operation order against exact
rational arithmetic (where the other orders give other floats), the polynomials' closed forms (integer exponents,
powers of two) and accuracy bounds, the 3 x 3 conv's geometry against a direct integer convolution, and the SED
heads, SE gate and generalised mean against float64 statements of their mathematics within quantisation bounds."""
import math
from fractions import Fraction

import numpy as np
import pytest

import pyoracle as O


def f32(x):
    return float(np.float32(x))


def rne32(q):
    """Fraction -> nearest float32 (ties to even), for normal results."""
    if q == 0:
        return 0.0
    s = -1 if q < 0 else 1
    a = abs(q)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    scale = Fraction(2) ** (23 - e)
    m = a * scale
    f = math.floor(m)
    r = m - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2):
        f += 1
    return s * float(Fraction(f) / scale)


def fma32(a, b, c):
    return rne32(Fraction(a) * Fraction(b) + Fraction(c))


# ------------------------------------------------------------------ packing and parameters
def test_wpack_against_numpy_statement():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((20, 37)).astype(np.float32)
    w[4] = 0.0
    b = rng.standard_normal(20).astype(np.float32)
    pk = O.qd_wpack(w, b, 32)
    s = np.where(np.abs(w).max(1) > 0, np.abs(w).max(1) / np.float32(127), np.float32(1)).astype(np.float32)
    q = np.clip(np.rint(w / s[:, None]), -127, 127).astype(np.int32)
    assert np.array_equal(pk["scale"][:20], s)
    assert np.array_equal(pk["q"][:20, :37], q)
    assert not pk["q"][:, 37:].any() and not pk["q"][20:].any()
    assert np.array_equal(pk["swsum"][:20], (s * q.sum(1).astype(np.float32)).astype(np.float32))
    assert (pk["scale"][20:] == 1).all() and not pk["swsum"][20:].any() and not pk["b"][20:].any()
    # the largest magnitude of each non-zero row quantises to +-127
    assert (np.abs(q[np.arange(20) != 4]).max(1) == 127).all()


def test_params_hand_examples():
    # range [0, 255]: scale 1, zp = rint(0) + 128
    assert O.qd_params(0.0, 255.0) == (1.0, 128.0, 1.0)
    # range [-255, 0]: scale 1, zp = -255 + 128 = -127
    assert O.qd_params(-255.0, 0.0) == (1.0, -127.0, 1.0)
    # an empty range (all zeros): scale 1, zp 128
    assert O.qd_params(0.0, 0.0) == (1.0, 128.0, 1.0)
    # the range always holds 0: a positive minimum counts as 0
    s, zp, inv = O.qd_params(3.0, 5.1)
    assert s == f32(np.float32(5.1) / np.float32(255)) and zp == 128.0
    # [-1, 1]: s = 2/255, zp = rint(-127.5) + 128 = -128 + 128 = 0 (ties to even)
    s, zp, inv = O.qd_params(-1.0, 1.0)
    assert s == f32(np.float32(2) / np.float32(255)) and inv == f32(np.float32(1) / np.float32(s))
    assert zp == float(np.rint(np.float32(-1) * np.float32(inv))) + 128


def test_quant_rows_f32_hand_row_and_roundtrip():
    x = np.array([[0.0, 1.0, 2.0, 255.0, 128.4, 128.6, 3.5, 4.5, 7.0]], np.float32)  # K = 9: an 8-wide part + tail
    a, rq = O.qd_quant_rows(x, 9)
    assert rq.tolist() == [[1.0, 128.0]]
    # q = rint(x) - 128 (ties to even in both the magic-number part and the rint tail)
    assert a[0, :9].tolist() == [-128, -127, -126, 127, 0, 1, -124, -124, -121]
    assert not a[0, 9:].any() and a.shape[1] == 16
    rng = np.random.default_rng(1)
    x = rng.standard_normal((50, 44)).astype(np.float32) * 5
    a, rq = O.qd_quant_rows(x, 44)
    deq = rq[:, :1] * (a[:, :44].astype(np.float32) + rq[:, 1:])
    assert (np.abs(deq - x) <= rq[:, :1] * 0.5001).all()


def test_quant_rows_f16_single_fp16_rounding():
    """codes below K & ~15 come from fma(h, (fp16)inv, 1536) rounded once to fp16 (numpy's float16 rounds the exact
    value); the tail from rint(h g inv) in fp32 with the unrounded inv"""
    rng = np.random.default_rng(2)
    K = 44  # K & ~15 = 32 (fp16 codes), K & ~7 = 40 (fp16 range), then the fp32 tails
    x = (rng.standard_normal((30, K)) * 4).astype(np.float16)
    g = rng.uniform(0, 1.5, K).astype(np.float16)
    a, rq = O.qd_quant_rows(x, K, g)
    for m in range(30):
        h = (x[m].astype(np.float64) * g.astype(np.float64)).astype(np.float16)  # gated product, one fp16 rounding
        h32 = x[m].astype(np.float32) * g.astype(np.float32)                      # the fp32 tail's exact product
        mn = min(0.0, float(h[:K & ~7].min()), float(h32[K & ~7:].min(initial=0)))
        mx = max(0.0, float(h[:K & ~7].max()), float(h32[K & ~7:].max(initial=0)))
        s, zp, inv = O.qd_params(mn, mx)
        assert rq[m].tolist() == [s, zp]
        hinv = float(np.float16(inv))
        for c in range(K):
            if c < (K & ~15):
                v = float(np.float16(float(h[c]) * hinv + 1536.0))  # exact in float64, one rounding
                q = int(v) - 1536 - int(zp)
            else:
                q = int(np.rint(np.float32(h32[c]) * np.float32(inv))) - int(zp)
            assert a[m, c] == max(-128, min(127, q)), (m, c)


# ------------------------------------------------------------------ the epilogue's operation order
def test_epilogue_order_against_exact_arithmetic():
    """v = fma(swsum, sa zp, fma(acc sw, sa, b)): each rounding checked with Fraction; the values are chosen so that
    (acc sa) sw, one fused (acc sw sa + b) and the unfused forms give other floats"""
    rng = np.random.default_rng(3)
    found = 0
    for trial in range(400):
        K = 16
        x = rng.standard_normal((1, K)).astype(np.float32) * rng.uniform(0.1, 50)
        w = rng.standard_normal((1, K)).astype(np.float32)
        b = rng.standard_normal(1).astype(np.float32)
        pk = O.qd_wpack(w, b, 16)
        a, rq = O.qd_quant_rows(x, K)
        out = O.qd_gemm(a, rq, pk)[0, 0]
        acc = int((a[0, :K].astype(np.int64) * pk["q"][0, :K].astype(np.int64)).sum())
        sa, zp, sw, ss, bb = float(rq[0, 0]), float(rq[0, 1]), float(pk["scale"][0]), float(pk["swsum"][0]), float(b[0])
        zs = rne32(Fraction(sa) * Fraction(zp))
        v0 = rne32(Fraction(acc) * Fraction(sw))
        want = fma32(ss, zs, fma32(v0, sa, bb))
        assert out == want, trial
        alt = [fma32(ss, zs, fma32(rne32(Fraction(acc) * Fraction(sa)), sw, bb)),
               rne32(Fraction(rne32(Fraction(v0) * Fraction(sa) + Fraction(bb))) + Fraction(ss) * Fraction(zs)),
               rne32(Fraction(acc) * Fraction(sw) * Fraction(sa) + Fraction(bb) + Fraction(ss) * Fraction(zs))]
        found += any(v != want for v in alt)
    assert found >= 20, found


def test_gemm_sums_brute_force():
    rng = np.random.default_rng(4)
    M, K, N = 7, 100, 32
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((N, K)).astype(np.float32)
    pk = O.qd_wpack(w, None)
    a, rq = O.qd_quant_rows(x, K)
    # with sw = 1 / (sum scale) stripped: the ReLU form of a zero-bias GEMM is max(v, 0) of the same v
    lin = O.qd_gemm(a, rq, pk)
    relu = O.qd_gemm(a, rq, pk, act=2)
    assert np.array_equal(relu, np.maximum(lin, 0))
    deq_x = rq[:, :1] * (a[:, :K].astype(np.float64) + rq[:, 1:])
    deq_w = pk["q"][:, :K] * pk["scale"][:, None].astype(np.float64)
    assert np.allclose(lin, deq_x @ deq_w.T, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------ polynomials
def test_exp2_p5_closed_forms():
    L = O.lib()
    for n in range(-126, 127):
        assert L.orc_exp2_p5(float(n)) == 2.0 ** n  # f = 0: p = 1, n added to the exponent
    xs = np.linspace(-20, 20, 4001).astype(np.float32)
    for t in xs:
        y = L.orc_exp2_p5(float(t))
        assert abs(y - 2.0 ** float(t)) <= 4e-6 * 2.0 ** float(t)  # Taylor terms to f^5, |f| <= 1/2: (ln 2 / 2)^6 / 720 / 2^-0.5


def test_silu_f32_a_closed_forms_and_accuracy():
    L = O.lib()
    # x with -x log2e rounding to an integer n: d = 2^n + 1 exactly (n <= 23); two Newton steps from FRECPE
    hit = 0
    for n in (-3, -1, 0, 1, 2, 5, 10):
        x = np.float32(-n / 1.44269504)
        for _ in range(8):
            t = np.float32(x) * np.float32(-1.44269504)
            if t == n:
                break
            x = np.nextafter(x, np.float32(np.inf) if t > n else np.float32(-np.inf))
        if np.float32(x) * np.float32(-1.44269504) != n:
            continue
        d = f32(2.0 ** n + 1.0)
        r = L.orc_frecpe(d)
        r = f32(np.float32(r) * np.float32(fma32(-d, r, 2.0)))
        r = f32(np.float32(r) * np.float32(fma32(-d, r, 2.0)))
        assert L.orc_silu_f32_a(float(x)) == f32(np.float32(x) * np.float32(r)), n
        hit += 1
    assert hit >= 5, hit
    for x in np.linspace(-40, 40, 8001).astype(np.float32):
        y = L.orc_silu_f32_a(float(x))
        ex = float(x) / (1 + math.exp(-float(x)))
        assert abs(y - ex) <= 5e-6 * abs(ex) + 1e-30, (x, y, ex)  # exp2_p5's 4e-6 carried by 1 / d


def test_log2_dot_closed_forms_and_accuracy():
    L = O.lib()
    for k in range(-125, 127):
        assert L.orc_log2_dot(2.0 ** k) == float(k)
    for x in np.exp(np.linspace(-60, 60, 6001)).astype(np.float32):
        assert abs(L.orc_log2_dot(float(x)) - math.log2(float(x))) <= 4e-6 * max(1.0, abs(math.log2(float(x))))


# ------------------------------------------------------------------ conv geometry, heads, SE gate, GeM
@pytest.mark.parametrize("H,W,C,K,s", [(8, 12, 16, 32, 2), (7, 9, 8, 16, 2), (6, 5, 8, 16, 1)])
def test_qconv3_against_direct_integer_conv(H, W, C, K, s):
    rng = np.random.default_rng(H + W + s)
    x = rng.standard_normal((H, W, C)).astype(np.float32)
    w = rng.standard_normal((K, 3, 3, C)).astype(np.float32)
    b = rng.standard_normal(K).astype(np.float32)
    pk = O.qd_wpack(w.reshape(K, 9 * C), b)
    out = O.qconv3(x, pk, s).astype(np.float32)
    xp, rq = O.qd_quant_tensor_pad(x)
    assert (xp[0] == -int(rq[1])).all() and (xp[:, -1] == -int(rq[1])).all()
    Ho, pt = O.tf_same(H, 3, s)
    Wo, pl = O.tf_same(W, 3, s)
    # the conv of the dequantised input over TF-same padding, from the float64 statement
    deq = np.zeros((H + 2, W + 2, C))
    deq[:] = rq[0] * (xp.astype(np.float64) + rq[1])
    q = pk["q"][:, :9 * C].reshape(K, 3, 3, C).astype(np.float64) * pk["scale"][:, None, None, None]
    ref = np.zeros((Ho, Wo, K))
    for oy in range(Ho):
        for ox in range(Wo):
            y0, x0 = oy * s - pt + 1, ox * s - pl + 1
            ref[oy, ox] = np.einsum("yxc,kyxc->k", deq[y0:y0 + 3, x0:x0 + 3], q) + b
    ref = ref / (1 + np.exp(-ref))
    assert np.allclose(out.reshape(Ho, Wo, K), ref, rtol=2e-2, atol=2e-2)


def test_heads_against_float_statement():
    rng = np.random.default_rng(5)
    H, W, C, hid, nc = 5, 7, 32, 48, 20
    ncp = 32
    shapes = [(nc, C)] + [(hid, C), (nc, hid), (nc, hid)] * 2
    ws_ = [(rng.standard_normal(s) / np.sqrt(s[1])).astype(np.float32) for s in shapes]
    bs_ = [(rng.standard_normal(s[0]) * 0.1).astype(np.float32) for s in shapes]
    packs = [O.qd_wpack(w, b, ncp if i == 0 or i % 3 != 1 else None) for i, (w, b) in enumerate(zip(ws_, bs_))]
    F = rng.standard_normal((H * W, C)).astype(np.float32)
    emb = rng.standard_normal(C).astype(np.float32)
    got = O.heads_s8(F, emb, H, W, packs)
    ref = ws_[0].astype(np.float64) @ emb + bs_[0]
    Fi = F.reshape(H, W, C).astype(np.float64)
    for i in range(2):
        s = Fi.mean(1) if i == 0 else Fi.mean(0)
        Lt = s.shape[0]
        pad = np.concatenate([np.full((1, C), -np.inf), s, np.full((1, C), -np.inf)])
        padz = np.concatenate([np.zeros((1, C)), s, np.zeros((1, C))])
        pooled = np.max([pad[t:t + Lt] for t in range(3)], 0) + sum(padz[t:t + Lt] for t in range(3)) / 3
        j = 1 + 3 * i
        h = np.maximum(pooled @ ws_[j].T + bs_[j], 0)
        att = np.clip(h @ ws_[j + 1].T + bs_[j + 1], -10, 10)
        cla = h @ ws_[j + 2].T + bs_[j + 2]
        ev = np.exp(att - att.max(0))
        ref = ref + (ev * cla).sum(0) / ev.sum(0)
    assert np.allclose(got[:nc], ref, rtol=0.05, atol=0.05)
    assert not got[nc:].any()


def test_se_gate16_against_float_statement():
    rng = np.random.default_rng(6)
    C, rd, P_ = 64, 8, 50
    w1 = (rng.standard_normal((rd, C)) / 8).astype(np.float32)
    b1 = (rng.standard_normal(rd) * 0.1).astype(np.float32)
    w2 = (rng.standard_normal((C, rd)) / 3).astype(np.float32)
    b2 = (rng.standard_normal(C) * 0.1).astype(np.float32)
    cs = (rng.standard_normal(C) * 20).astype(np.float32)
    m, g = O.se_gate16(cs, P_, w1, b1, w2, b2)
    assert np.array_equal(m, (cs * np.float32(1 / np.float32(P_))).astype(np.float32))
    v = w1.astype(np.float64) @ (cs / P_) + b1
    t = v / (1 + np.exp(-v))
    ref = 1 / (1 + np.exp(-(w2.astype(np.float64) @ t + b2)))
    assert np.allclose(g.astype(np.float64), ref, atol=2e-3)


def test_gem_a_against_float_statement():
    rng = np.random.default_rng(7)
    F = np.abs(rng.standard_normal((40, 24))).astype(np.float32)
    F[0, 0] = -3.0
    e = O.gem_a(F, 1e-6, 3.0)
    ref = (np.maximum(F.astype(np.float64), 1e-6) ** 3).mean(0) ** (1 / 3)
    assert np.allclose(e, ref, rtol=3e-6)


# ------------------------------------------------------------------ the dotprod prototype head (PROTO variant 2)
def pack_c12(q):
    """prototype rows q [Np][K] -> panels [Np/12][K/4][12][4]"""
    Np, K = q.shape
    return np.ascontiguousarray(q.reshape(Np // 12, 12, K // 4, 4).transpose(0, 2, 1, 3))


def pack_c4(q, Kp):
    """prototype rows q [Np][K] -> the no-dotprod head's panels [Np/4][Kp/16][4][16]"""
    Np, K = q.shape
    qp = np.zeros((Np, Kp), np.int8)
    qp[:, :K] = q
    return np.ascontiguousarray(qp.reshape(Np // 4, 4, Kp // 16, 16).transpose(0, 2, 1, 3))


@pytest.mark.parametrize("P,C,Np", [(24, 40, 36), (64, 64, 24)])
def test_proto_dot_against_the_no_dotprod_head(P, C, Np):
    """fp16 cells widened give the fp32 head's sums and scales (its -127 floor is unreachable: |x| <= max|x|), and
    the 12-prototype panels hold the same prototypes as the 4-prototype ones: colmax and logits agree bit for bit"""
    rng = np.random.default_rng(P + C)
    x = (rng.standard_normal((P, C + 8)) * 2).astype(np.float16)
    q = rng.integers(-127, 128, (Np, C)).astype(np.int8)
    sw = rng.uniform(0.001, 0.01, Np).astype(np.float32)
    nc, ppc = Np // 3, 3
    clsw = rng.standard_normal((nc, ppc)).astype(np.float32)
    clsb = rng.standard_normal(nc).astype(np.float32)
    rc, lg, cm = O.proto_s8_dot(x, C, 1e-5, pack_c12(q), sw, Np, clsw, clsb, nc, ppc)
    Kp = (C + 15) // 16 * 16
    rc0, lg0, cm0, _ = O.proto_s8(x.astype(np.float32), C, 1e-5, pack_c4(q, Kp), sw, Np, Kp, clsw, clsb, nc, ppc)
    assert rc == rc0 == 0
    assert np.array_equal(cm, cm0) and np.array_equal(lg, lg0)
