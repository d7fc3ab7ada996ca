"""Pins the bit-level operation orders of the oracle that no golden vector covers: the log-mel front end's FFT
butterflies (src/fft_tab.h:22-80), the SE gate's first FC (src/v24_f32.c:164-179; the fp16-weight form of
SE_GATE16, src/rt_ops_dot.c:381-420), the depthwise convolutions' channel sums (src/pc_kern_f32.c:174-334,
src/gemm_f32.c:303-441, src/pc_kern_f16.c:16-96, src/kern_f16.c:83-155) and HEADS_S8's pooling and attention
soft-max (src/rt_ops_dot.c:531-570).

Each expected value is computed here in exact arithmetic (Fraction), rounded to float32 (or fp16) once per operation
of the reference's order; inputs are chosen, or drawn in numbers, so that the plausible other orders (another
association, a fused or an unfused multiply-add, another lane pairing, another block split) round to other floats
on many of them, and the test counts those decisive cases. A wrong order in the oracle fails here."""
from fractions import Fraction as Fr

import numpy as np

import pyoracle as O

f32, f16 = np.float32, np.float16


def rne32(q):
    """A rational rounded once to float32, nearest even (exact: through the float32 neighbours)."""
    q = Fr(q)
    if q == 0:
        return f32(0)
    lo = f32(float(q))                     # within one float32 step of q
    cands = {lo, np.nextafter(lo, f32(np.inf)), np.nextafter(lo, f32(-np.inf))}
    best = min(cands, key=lambda c: (abs(Fr(float(c)) - q), int(np.asarray(c).view(np.uint32)) & 1))
    return f32(best)


def rne16(q):
    q = Fr(q)
    if q == 0:
        return f16(0)
    lo = f16(float(q))
    cands = {lo, np.nextafter(lo, f16(np.inf)), np.nextafter(lo, f16(-np.inf))}
    return f16(min(cands, key=lambda c: (abs(Fr(float(c)) - q), int(np.asarray(c).view(np.uint16)) & 1)))


def F(x):
    return Fr(float(x))


def add(a, b):
    if isinstance(a, Fr) or isinstance(b, Fr) or (np.isfinite(a) and np.isfinite(b)):
        return rne32(F(a) + F(b))
    return f32(a) + f32(b)       # infinities: IEEE addition


def fma(a, b, c):
    return rne32(F(a) * F(b) + F(c))


def mul(a, b):
    return rne32(F(a) * F(b))


# ---------------------------------------------------------------- FFT (fft_dit_x4, src/fft_tab.h:25-80)
def cmul_ref(br, bi, wr, wi):
    """vfmsq_n_f32(vmulq_n_f32(b, wr), bi, wi), vfmaq_n_f32(vmulq_n_f32(b, wi), bi, wr): the first product rounded,
    the second fused into the subtraction / addition"""
    return fma(-F(bi), F(wi), mul(br, wr)), fma(bi, wr, mul(br, wi))


def cmul_unfused(br, bi, wr, wi):
    return add(mul(br, wr), -F(mul(bi, wi))), add(mul(br, wi), mul(bi, wr))


def cmul_swapped(br, bi, wr, wi):
    return rne32(F(br) * F(wr) - F(mul(bi, wi))), rne32(F(br) * F(wi) + F(mul(bi, wr)))


def fft8(re, im, cmul, first_fold=False):
    """The 8-point transform in the reference's pass structure: the fused first two stages (no twiddle products,
    d1 (-i) as a swap), then the last radix-2 level with twiddles of fft_twiddles(8)"""
    re, im = [f32(v) for v in re], [f32(v) for v in im]
    twr, twi = O.fft_twiddles(8)
    for i in (0, 4):
        ar, ai, br, bi, cr, ci, dr, di = re[i], im[i], re[i + 1], im[i + 1], re[i + 2], im[i + 2], re[i + 3], im[i + 3]
        s0r, s0i, d0r, d0i = add(ar, br), add(ai, bi), add(ar, -F(br)), add(ai, -F(bi))
        s1r, s1i, d1r, d1i = add(cr, dr), add(ci, di), add(cr, -F(dr)), add(ci, -F(di))
        if first_fold:   # ((a + b) + c) + d: a restatement that sums the four points in turn
            re[i], im[i] = add(add(s0r, cr), dr), add(add(s0i, ci), di)
        else:
            re[i], im[i] = add(s0r, s1r), add(s0i, s1i)
        re[i + 2], im[i + 2] = add(s0r, -F(s1r)), add(s0i, -F(s1i))
        re[i + 1], im[i + 1] = add(d0r, d1i), add(d0i, -F(d1r))
        re[i + 3], im[i + 3] = add(d0r, -F(d1i)), add(d0i, d1r)
    for j in range(4):
        vr, vi = cmul(re[j + 4], im[j + 4], twr[j], twi[j])
        ur, ui = re[j], im[j]
        re[j], im[j] = add(ur, vr), add(ui, vi)
        re[j + 4], im[j + 4] = add(ur, -F(vr)), add(ui, -F(vi))
    return np.array(re, f32), np.array(im, f32)


def test_fft_first_stages_sum_in_pairs():
    # points (2^24, 1, 1, 1): (a + b) + (c + d) = 2^24 + 2 (2^24 + 1 ties to even 2^24); the four summed in turn
    # lose every 1 (2^24)
    re = np.array([2 ** 24, 1, 1, 1, 0, 0, 0, 0], f32)
    R, I = O.fft_dit(re, np.zeros(8, f32))
    assert R[0] == 2 ** 24 + 2 and R[4] == 2 ** 24 + 2
    assert fft8(re, np.zeros(8), cmul_ref, first_fold=True)[0][0] == 2 ** 24


def test_fft8_in_exact_arithmetic():
    """random 8-point frames: every output equals the exact-arithmetic transform in the reference's order; the
    unfused and the other fused complex products give other floats on many outputs"""
    rng = np.random.default_rng(4)
    decisive = 0
    for _ in range(300):
        re = (rng.standard_normal(8) * rng.uniform(0.01, 100)).astype(f32)
        im = (rng.standard_normal(8) * rng.uniform(0.01, 100)).astype(f32)
        R, I = O.fft_dit(re, im)
        wr, wi = fft8(re, im, cmul_ref)
        assert np.array_equal(R, wr) and np.array_equal(I, wi)
        for alt in (cmul_unfused, cmul_swapped):
            ar, ai = fft8(re, im, alt)
            decisive += int(np.sum(ar != wr) + np.sum(ai != wi))
    assert decisive >= 200, decisive


def test_fft_radix4_pass_products():
    """32 points: an impulse (v, u) at position 12 (the 'd' slot of the first radix-2^2 group) is spread by the
    first stage over positions 12..15; the radix-2^2 pass (len 8) multiplies it by w1 = W32^(4j), then by
    w2 = W32^(2j), each product in the fused form: outputs t2 = (v, u) w1 w2 at positions j, -t2 at j + 8,
    (-t2i, t2r) at j + 4 and (t2i, -t2r) at j + 12; the last level copies positions 0..15 to 16..31"""
    twr, twi = O.fft_twiddles(32)
    v, u = f32(1.2126465), f32(1.0795898)
    re, im = np.zeros(32, f32), np.zeros(32, f32)
    re[12], im[12] = v, u
    R, I = O.fft_dit(re, im)
    decisive = 0
    for j in range(4):
        t = cmul_ref(v, u, twr[4 * j], twi[4 * j])
        t2 = cmul_ref(t[0], t[1], twr[2 * j], twi[2 * j])
        assert (R[j], I[j]) == t2, j
        assert (R[j + 8], I[j + 8]) == (-t2[0], -t2[1])
        assert (R[j + 4], I[j + 4]) == (-t2[1], t2[0]) and (R[j + 12], I[j + 12]) == (t2[1], -t2[0])
        for alt in (cmul_unfused, cmul_swapped):
            a = alt(v, u, twr[4 * j], twi[4 * j])
            decisive += alt(a[0], a[1], twr[2 * j], twi[2 * j]) != t2
    assert np.array_equal(R[16:], R[:16]) and np.array_equal(I[16:], I[:16])
    assert decisive >= 2, decisive


# ---------------------------------------------------------------- SE first FC (v24k32_se_fc1)
def fc1_ref(mean, w, b, h16=False, pairing="lanes"):
    """one output of the first FC: eight lane chains (channel c into chain c % 8, fused), combined as
    ((a0 + a4) + (a1 + a5)) + ((a2 + a6) + (a3 + a7)) ('lanes'; 'adjacent': pairs (2j, 2j+1); 'one': a single
    chain), + b, then SiLU x / (1 + expf(-x))"""
    C = len(mean)
    ww = [f32(f16(x)) if h16 else f32(x) for x in w]
    if pairing == "one":
        v = f32(0)
        for c in range(C):
            v = fma(ww[c], mean[c], v)
    else:
        a = [f32(0)] * 8
        for c in range(C):
            a[c % 8] = fma(ww[c], mean[c], a[c % 8])
        if pairing == "lanes":
            t = [add(a[j], a[j + 4]) for j in range(4)]
        else:
            t = [add(a[2 * j], a[2 * j + 1]) for j in range(4)]
        v = add(add(t[0], t[1]), add(t[2], t[3]))
    x = add(v, b)
    e = O.expf(np.array([-x], f32))[0]
    return f32(x) / add(f32(1), e)     # one IEEE division (numpy's float32 division is correctly rounded)


def test_se_fc1_lane_order():
    for h16 in (False, True):
        # designed: chains [2^24 + seven lost 1s, 1, 0, 1, 0, 1 + 8 steps, 0, 1]: (t0 + t1) + (t2 + t3) keeps the
        # small chains together; s1 = x exactly (expf(-x) = 0 for x near 2^24)
        C = 64
        mean = np.zeros(C, f32)
        w = np.ones(C, f32)
        mean[0] = 2 ** 24
        mean[8::8] = 1
        mean[[1, 3, 5, 7]] = 1
        s1 = O.se_fc1(mean, w[None, :], np.zeros(1, f32), h16=h16)[0]
        want = fc1_ref(mean, w, 0, h16)
        assert s1 == want and want == 2 ** 24 + 4
        assert fc1_ref(mean, w, 0, h16, "adjacent") != want and fc1_ref(mean, w, 0, h16, "one") != want
        # random rows: exact arithmetic agrees everywhere; the other lane orders differ on many
        rng = np.random.default_rng(9 + h16)
        C, rd = 48, 40
        mean = (rng.standard_normal(C) * rng.uniform(0.1, 10, C)).astype(f32)
        w = rng.standard_normal((rd, C)).astype(f32)
        b = rng.standard_normal(rd).astype(f32)
        s1 = O.se_fc1(mean, w, b, h16=h16)
        decisive = 0
        for r in range(rd):
            want = fc1_ref(mean, w[r], b[r], h16)
            assert s1[r] == want, (h16, r)
            decisive += (fc1_ref(mean, w[r], b[r], h16, "adjacent") != want) + (fc1_ref(mean, w[r], b[r], h16, "one")
                                                                                  != want)
        assert decisive >= 10, (h16, decisive)


# ---------------------------------------------------------------- depthwise channel sums
def identity_taps(k, C, dt):
    w = np.zeros((k * k, C), dt)
    w[(k * k) // 2] = 1
    return w, np.zeros(C, dt)


def chsum_expected(out, form):
    """the channel sums of the outputs out [Ho][Wo][C] in the reference's order:
    'dwk32': per row, 4-pixel groups add ((v0 + v1) + (v2 + v3)), the rest one by one (pc_dwk_f32_cr);
    'dw332': every pixel in turn (dw3x3_f32_cr / silu_rows_f32);
    'dwk16': 4-pixel groups as fp16 ((v0 + v1) + (v2 + v3)), then pairs as fp16 v0 + v1, then singles, each widened
             and added to the fp32 sum (pc_dwk_f16_cr);
    'dw316': per row an fp16 running sum of every pixel in turn, widened and added at the row's end (dw3x3_f16_cr);
    'seq32': every pixel in turn (a planted alternative of the grouped forms)"""
    Ho, Wo, C = out.shape
    cs = [f32(0)] * C
    for c in range(C):
        s = f32(0)
        for y in range(Ho):
            v = [out[y, x, c] for x in range(Wo)]
            if form in ("dw332", "seq32"):
                for a in v:
                    s = add(s, a)
            elif form == "dwk32":
                x = 0
                while x + 4 <= Wo:
                    s = add(s, add(add(v[x], v[x + 1]), add(v[x + 2], v[x + 3])))
                    x += 4
                for a in v[x:]:
                    s = add(s, a)
            elif form == "dwk16":
                x = 0
                h = lambda a, b: rne16(F(a) + F(b))
                while x + 4 <= Wo:
                    s = add(s, f32(h(h(v[x], v[x + 1]), h(v[x + 2], v[x + 3]))))
                    x += 4
                while x + 2 <= Wo:
                    s = add(s, f32(h(v[x], v[x + 1])))
                    x += 2
                for a in v[x:]:
                    s = add(s, f32(a))
            elif form == "dw316":
                r = f16(0)
                for a in v:
                    r = rne16(F(r) + F(a))
                s = add(s, f32(r))
        cs[c] = s
    return np.array(cs, f32)


def test_channel_sums_fp32():
    # identity taps: the outputs are the inputs (DWK without activation) or their SiLU (DW3, fixed)
    rng = np.random.default_rng(21)
    H, W, C = 3, 7, 8
    x = (rng.standard_normal((H, W, C)) * 300).astype(f32)
    x[0, 0, :] = 2 ** 24
    x[0, 1:, :] = 1
    xp = np.zeros((H + 2, W + 2, C), f32)
    xp[1:-1, 1:-1] = x
    w, b = identity_taps(3, C, f32)
    out, cs = O.dwk_f32(xp, H, W, C, 3, 1, 1, 1, w, b, 0, H, W)
    assert np.array_equal(out, x)
    want = chsum_expected(out, "dwk32")
    assert np.array_equal(cs, want)
    assert cs[0] == chsum_expected(out[:, :, :1], "dwk32")[0]
    assert int(np.sum(chsum_expected(out, "seq32") != want)) >= 4
    out3, cs3 = O.dw3_f32(xp, H, W, C, 1, w, b, H, W)
    assert np.array_equal(cs3, chsum_expected(out3, "dw332"))
    assert int(np.sum(chsum_expected(out3, "dwk32") != cs3)) >= 4


def test_channel_sums_fp16():
    rng = np.random.default_rng(22)
    H, W, C = 3, 7, 16
    x = (rng.standard_normal((H, W, C)) * 40).astype(f16)
    x[0, 0, :] = 2048
    x[0, 1:, :] = 1
    xp = np.zeros((H + 2, W + 2, C), f16)
    xp[1:-1, 1:-1] = x
    w, b = identity_taps(3, C, f16)
    out, cs = O.dwk_f16(xp, H, W, C, 3, 1, 1, 1, w, b, 0, H, W)
    assert np.array_equal(out, x)
    want = chsum_expected(out, "dwk16")
    assert np.array_equal(cs, want)
    assert int(np.sum(chsum_expected(out, "seq32") != want)) >= 4
    out3, cs3 = O.dw3_f16(xp, H, W, C, 1, 1, 1, w, b, H, W)
    want3 = chsum_expected(out3, "dw316")
    assert np.array_equal(cs3, want3)
    assert int(np.sum(chsum_expected(out3, "dwk16") != want3)) >= 4


# ---------------------------------------------------------------- HEADS_S8 pooling and soft-max
def test_heads_pool_order():
    """time means: a sum from 0 in order of the other axis, then / length; pooling: fmaxf of the 3 neighbours +
    (the sum from 0 of v * 0.33333334f, each product rounded, in order t - 1, t, t + 1)"""
    rng = np.random.default_rng(23)
    H, W, C = 5, 6, 16
    Fm = (rng.standard_normal((H * W, C)) * rng.uniform(0.5, 50, C)).astype(f32)
    Fm[0:4, 0] = [2 ** 24, 1, 1, 1]
    third = f32(0.33333334)
    decisive = 0
    for i in (0, 1):
        L, n = (H, W) if i == 0 else (W, H)
        s, pooled = O.heads_pool(Fm, H, W, i)
        for t in range(L):
            for c in range(C):
                seq = f32(0)
                vals = [Fm[t * W + u, c] if i == 0 else Fm[u * W + t, c] for u in range(n)]
                for v in vals:
                    seq = add(seq, v)
                mean = rne32(F(seq) / n)
                assert s[t, c] == mean, (i, t, c)
                pair = add(add(vals[0], vals[1]), add(vals[2], vals[3])) if n == 4 else None
                decisive += pair is not None and rne32(F(pair) / n) != mean
        for t in range(L):
            for c in range(C):
                nb = [s[u, c] for u in (t - 1, t, t + 1) if 0 <= u < L]
                sm = f32(0)
                for v in nb:
                    sm = add(sm, mul(v, third))
                want = add(max(nb), sm)
                assert pooled[t, c] == want, (i, t, c)
                fused = f32(0)
                for v in nb:
                    fused = fma(v, third, fused)
                sumfirst = mul(add(add(nb[0], nb[1]), nb[2]) if len(nb) == 3 else add(nb[0], nb[1]), third)
                decisive += (add(max(nb), fused) != want) + (add(max(nb), sumfirst) != want)
    assert decisive >= 30, decisive


def test_heads_softmax_order():
    """per class: att clipped to [-10, 10], mx = fmaxf, then in order of t: ev = expf(att - mx) (C library),
    z += ev, acc += ev * cla (product rounded); logit += acc / z. Designed column: att = 10 then 31 x -10, so every
    ev but the first is expf(-20) ~ 2e-9 < 2^-25 and is lost against 1 in z; the reversed order keeps them."""
    L, ncp, nc = 32, 16, 3
    rng = np.random.default_rng(24)
    att = rng.uniform(-14, 14, (L, ncp)).astype(f32)
    cla = rng.standard_normal((L, ncp)).astype(f32)
    att[:, 0] = -10
    att[0, 0] = 10
    cla[:, 0] = 1
    cla[0, 0] = 0
    lg0 = rng.standard_normal(ncp).astype(f32)
    lg0[0] = 0
    lg = O.heads_softmax(att, cla, nc, lg0)
    decisive = 0
    for k in range(ncp):
        a = np.clip(att[:, k], -10, 10).astype(f32)
        if k >= nc:
            assert lg[k] == lg0[k]
            continue
        mx = f32(a.max())
        ev = O.expf((a - mx).astype(f32))
        assert np.array_equal((a - mx).astype(f32), np.array([add(v, -F(mx)) for v in a], f32))
        z = acc = f32(0)
        for t in range(L):
            z = add(z, ev[t])
            acc = add(acc, mul(ev[t], cla[t, k]))
        want = add(lg0[k], rne32(F(acc) / F(z)))
        assert lg[k] == want, k
        zr = accr = f32(0)
        for t in reversed(range(L)):
            zr = add(zr, ev[t])
            accr = add(accr, mul(ev[t], cla[t, k]))
        decisive += add(lg0[k], rne32(F(accr) / F(zr))) != want
    assert decisive >= 2, decisive
    # the designed column: z = 1 exactly in the reference's order (each expf(-20) is lost against 1), so the logit is
    # acc = the sum of the 31 small terms; summed backwards z keeps them (1 + 2^-23) and the logit is another float
    e = O.expf(np.array([-20], f32))[0]
    assert e < 2 ** -25
    acc = f32(0)
    for _ in range(31):
        acc = add(acc, e)
    assert lg[0] == acc
    assert rne32(F(acc) / F(add(acc, 1))) != acc
