"""Pins the oracle of the fp32 / fp16 prototype heads (oracle/proto.c: orc_l2norm_f32 / _f16, orc_colmax_f32,
orc_colmax_f32h, orc_colmax_f16; PROTO variant 0 src/rt_ops_f32.c:548-570, PROTO_F32H :572-591, PROTO variant 1
src/rt_ops_f16.c:227-250).

The summation orders are pinned on inputs where the reference's order and the plausible other orders round to
different floats. Each expected value is derived by hand in the comment beside it (powers of two, absorption of small
terms by 2^24 or by fp16's 2048); each plausible other order is computed here as a planted mistake and must give a
different float, so a wrong order in the oracle fails the test. Layouts are pinned by integer data, on which every
order is exact, against a float64 product.
"""
from fractions import Fraction as Fr

import numpy as np

import pyoracle as O
from bnneon import netbuild

f32, f16 = np.float32, np.float16


def rnd32(q):
    """A rational rounded once to float32 (nearest even), through float64 only when that is exact."""
    d = float(q)
    assert Fr(d) == q, "test values must be exact in float64"
    return f32(d)


def fma32(a, b, c):
    return rnd32(Fr(float(a)) * Fr(float(b)) + Fr(float(c)))


def fma16(a, b, c):
    q = Fr(float(a)) * Fr(float(b)) + Fr(float(c))
    d = float(q)
    assert Fr(d) == q
    return f16(d)


# ---------------------------------------------------------------- L2 normalisation (pc_l2norm_f32 / _f16)
def sumsq_alternatives(x):
    """Sums of squares of x in orders a restatement could plausibly use instead of the reference's."""
    def chains(rev=False):
        ch = [f32(0)] * 8
        for c in (reversed(range(len(x))) if rev else range(len(x))):
            ch[c % 8] = fma32(x[c], x[c], ch[c % 8])
        return ch

    def ref_comb(ch):
        t = [f32(ch[j] + ch[j + 4]) for j in range(4)]
        return f32(f32(t[0] + t[1]) + f32(t[2] + t[3]))

    def adj_comb(ch):   # lane pairs (2j, 2j + 1)
        t = [f32(ch[2 * j] + ch[2 * j + 1]) for j in range(4)]
        return f32(f32(t[0] + t[1]) + f32(t[2] + t[3]))

    def seq_comb(ch):   # lanes added one after another
        s = f32(0)
        for v in ch:
            s = f32(s + v)
        return s

    one = f32(0)
    for v in x:         # one chain over every channel
        one = fma32(v, v, one)
    exact = rnd32(sum(Fr(float(v)) ** 2 for v in x))
    return {"adjacent lanes": adj_comb(chains()), "sequential lanes": seq_comb(chains()),
            "channels reversed": ref_comb(chains(True)), "one chain": one, "exact": exact}


def den_of(S):
    return f32(np.sqrt(np.float64(S)))   # sqrt of a float32 via float64 is correctly rounded


def check_l2_cell(x, S_ref, must_differ):
    a = O.l2norm(x.reshape(1, -1), x.size, 0.0)
    den = den_of(f32(S_ref))
    big = int(np.argmax(x))
    assert a[0, big] == f32(x[big]) / den, (a[0, big], f32(x[big]) / den)
    assert np.array_equal(a[0], x / den)
    alts = sumsq_alternatives(x)
    for name in must_differ:
        assert den_of(alts[name]) != den, name   # the planted mistake would change the output


def test_l2norm_chain_order():
    # 64 channels: channel c feeds chain c % 8 in order of c. Chain 0: 4096^2 = 2^24, then seven 1s, each lost to
    # the tie at 2^24 + 1 (ties to even); chain 4: eight 1s = 8. t0 = 2^24 + 8, t1 = t2 = t3 = 0: S = 2^24 + 8,
    # den = sqrtf(2^24 + 8) = 4096 + 2^-10. One chain over every channel loses all fifteen 1s (den 4096); the chains
    # walked backwards and the exact sum give 2^24 + 16 (den 4096 + 2^-9).
    x = np.zeros(64, f32)
    x[0] = 4096
    x[8::8] = 1
    x[4::8] = 1
    check_l2_cell(x, 2 ** 24 + 8, ("one chain", "channels reversed", "exact"))


def test_l2norm_lane_pairing():
    # chains c = [2^24, 1, 0, 1, 0, 1, 0, 1] (channels 0..7 only): t_j = c_j + c_{j+4} = [2^24, 2, 0, 2];
    # (t0 + t1) + (t2 + t3) = (2^24 + 2) + 2 = 2^24 + 4, den = 4096 + 2^-11. Lane pairs (2j, 2j + 1) give
    # ((2^24 + 1) + (0 + 1)) + ((0 + 1) + (0 + 1)) = 2^24 + 2 (den 4096), lanes added in turn lose every 1.
    x = np.array([4096, 1, 0, 1, 0, 1, 0, 1], f32)
    check_l2_cell(x, 2 ** 24 + 4, ("adjacent lanes", "sequential lanes"))


def test_l2norm_eps_and_rows():
    # a 3-4-5 cell: den = 5 + eps exactly as float32 adds it; rows past C (ld > C) are not read
    x = np.zeros((2, 24), f32)
    x[0, 0], x[0, 9] = 3, 4
    x[1, 5] = -2
    x[:, 16:] = 7   # beyond C = 16
    a = O.l2norm(x, 16, 0.25)
    assert a.shape == (2, 16)
    assert a[0, 0] == f32(3) / f32(5.25) and a[0, 9] == f32(4) / f32(5.25)
    assert a[1, 5] == f32(-2) / f32(2.25)
    assert np.count_nonzero(a) == 3


def test_l2norm_f16_rounds_the_fp32_quotient():
    # pc_l2norm_f16: a = fp16(fp32(x) / den), den in fp32. Cells (3, 5) and (5, 1): the quotient computed in fp16
    # from an fp16 den gives another fp16 value.
    for x0, x1 in ((3, 5), (5, 1), (13, 3)):
        x = np.zeros((1, 8), f16)
        x[0, 0], x[0, 5] = x0, x1
        a = O.l2norm(x, 8, 0.0, f16=True).view(f16)
        den = f32(np.sqrt(f32(x0 * x0 + x1 * x1)))
        assert a[0, 0] == f16(f32(x0) / den) and a[0, 5] == f16(f32(x1) / den)
        assert f16(f16(x0) / f16(den)) != a[0, 0] or f16(f16(x1) / f16(den)) != a[0, 5]


# ---------------------------------------------------------------- fp32 column maxima (gemm_f32_colmax, f32h)
def chain_row_and_proto():
    """A row and a prototype whose products, in order of k, are 2^24, seven 1s, -2^24, -1, then
    (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24. The chain from +0: 2^24 (the 1s are lost to ties at 2^24 + 1), 0, -1, then
    one fused rounding of -1 + 1 + 2^-11 + 2^-24 = 2^-11 + 2^-24 (exact)."""
    K = 16
    a = np.zeros(K, f32)
    w = np.zeros(K, f32)
    a[0], w[0] = 4096, 4096
    a[1:8], w[1:8] = 1, 1
    a[8], w[8] = -4096, 4096
    a[9], w[9] = 1, -1
    a[10] = w[10] = f32(1 + 2 ** -12)
    return a, w, f32(2 ** -11 + 2 ** -24)


def chain_alternatives(a, w):
    prods = [Fr(float(x)) * Fr(float(y)) for x, y in zip(a, w)]
    out = {}
    s = f32(0)
    for x, y in zip(a[::-1], w[::-1]):
        s = fma32(x, y, s)
    out["reversed"] = s
    s = f32(0)
    for p in prods:     # multiply, round, then add
        s = f32(s + rnd32(p))
    out["unfused"] = s
    out["exact"] = rnd32(sum(prods))
    lanes = [f32(0)] * 4
    for k, (x, y) in enumerate(zip(a, w)):
        lanes[k % 4] = fma32(x, y, lanes[k % 4])
    out["4 lanes"] = f32(f32(lanes[0] + lanes[1]) + f32(lanes[2] + lanes[3]))
    return out


def test_colmax_f32_chain_order():
    a, w, want = chain_row_and_proto()
    K, P, N = a.size, 8, 8
    A = np.full((P, K), -1.0, f32)      # other cells: the chain ends below want
    A[3] = a
    W = np.zeros((N, K), f32)
    W[5] = w
    panels, _, (_, _, Kp, Np) = netbuild.Net.fpack(W, np.zeros(N, f32), K_pad=8)
    cm = O.colmax_f32(A, panels, Kp, Np)
    assert cm[5] == want
    for name, v in chain_alternatives(a, w).items():
        assert v != want, name
    # prototypes of zeros: every chain is +0
    assert all(cm[n] == 0 and not np.signbit(cm[n]) for n in range(N) if n != 5)


def test_colmax_f32h_chain_order():
    # the same chain with fp16-representable weights: 4096, 1, 4096, -1, then a = 1 + 2^-14, w = 1 + 2^-10:
    # (1 + 2^-10)(1 + 2^-14) = 1 + 2^-10 + 2^-14 + 2^-24, fused onto -1 exactly; a rounded product loses 2^-24
    a, w, _ = chain_row_and_proto()
    a[10], w[10] = f32(1 + 2 ** -14), f32(1 + 2 ** -10)
    want = f32(2 ** -10 + 2 ** -14 + 2 ** -24)
    K, P, N = a.size, 8, 16
    A = np.full((P, K), -1.0, f32)
    A[6] = a
    W = np.zeros((N, K), f16)
    W[9] = w.astype(f16)
    assert np.array_equal(W[9].astype(f32), w)
    wp = np.ascontiguousarray(W.reshape(N // 8, 8, K).transpose(0, 2, 1))
    cm = O.colmax_f32h(A, wp, N)
    assert cm[9] == want
    for name, v in chain_alternatives(a, w).items():
        assert v != want, name


def test_colmax_f32_layouts_exact():
    rng = np.random.default_rng(3)
    for P, K, N in ((8, 24, 20), (24, 40, 33), (16, 8, 8)):
        A = rng.integers(-3, 4, (P, K)).astype(f32)
        W = rng.integers(-3, 4, (N, K)).astype(f32)
        want = (A.astype(np.float64) @ W.T.astype(np.float64)).max(0)
        panels, _, (_, _, Kp, Np) = netbuild.Net.fpack(W, np.zeros(N, f32), K_pad=8)
        cm = O.colmax_f32(A, panels, Kp, Np)
        assert np.array_equal(cm[:N], want)
        assert not cm[N:].any()
        Wh = np.zeros((Np, K), f16)
        Wh[:N] = W
        wp = np.ascontiguousarray(Wh.reshape(Np // 8, 8, K).transpose(0, 2, 1))
        assert np.array_equal(O.colmax_f32h(A, wp, Np)[:N], want)


def test_colmax_nan_propagates():
    A = np.ones((8, 8), f32)
    A[2, 3] = np.nan
    W = np.ones((8, 8), f32)
    panels, _, (_, _, Kp, Np) = netbuild.Net.fpack(W, np.zeros(8, f32), K_pad=8)
    assert np.isnan(O.colmax_f32(A, panels, Kp, Np)).all()   # FMAX keeps the NaN whatever the other cells hold


# ---------------------------------------------------------------- fp16 column maxima (gemm_f16_colmax)
def hpack(W16):
    N, K = W16.shape
    w, _, _, (_, _, Kp, Np) = netbuild.Net.pack_h16(W16.astype(f32), np.zeros(N, f32), K)
    return w, Kp, Np


def test_colmax_f16_blocks():
    # K = 264: three balanced K blocks of 88 (kblocks: 3 blocks <= 128 steps, a multiple of 8), each an fp16 chain
    # from +0, the blocks' results summed in fp32 from +0. Row of ones; weights 2048 at k 0, 1 at k 87 (block 0:
    # 2048 + 1 ties to even 2048 in fp16), 1 at k 88 and k 127 (block 1: 2): 2048 + 2 + 0 = 2050.
    # Blocks of 128 lose all three 1s (2048); one fp16 chain gives 2048; an fp32 chain or the exact sum 2051.
    K = 264
    A = np.zeros((8, K), f16)
    A[4] = 1
    W = np.zeros((24, K), f16)
    W[17, 0], W[17, 87], W[17, 88], W[17, 127] = 2048, 1, 1, 1
    # prototype 2: a fused fp16 product: -1, then (1 + 2^-6)^2 = 1 + 2^-5 + 2^-12 onto it exactly
    A[6, 0], A[6, 1] = 1, 1 + 2 ** -6
    W[2, 0], W[2, 1] = -1, 1 + 2 ** -6
    w, Kp, Np = hpack(W)
    cm = O.colmax_f16(A, w, Kp, Np)
    assert cm[17] == 2050
    assert cm[2] == f32(2 ** -5 + 2 ** -12)

    def blocks(a, w, bounds):
        fb = f32(0)
        for lo, hi in bounds:
            acc = f16(0)
            for k in range(lo, hi):
                acc = fma16(w[k], a[k], acc)
            fb = f32(fb + f32(acc))
        return fb
    a4, w17 = A[4], W[17]
    assert blocks(a4, w17, ((0, 128), (128, 256), (256, 264))) == 2048        # fixed 128-step blocks
    assert blocks(a4, w17, ((0, K),)) == 2048                                  # one fp16 chain
    s = f32(0)
    for k in range(K):
        s = fma32(w17[k], a4[k], s)
    assert s == 2051                                                           # an fp32 chain
    unfused = f16(f16(-1) + f16(f16(1 + 2 ** -6) * f16(1 + 2 ** -6)))
    assert unfused != f16(2 ** -5 + 2 ** -12)                                  # a rounded product


def test_colmax_f16_single_block_and_layout():
    rng = np.random.default_rng(5)
    for P, K, N in ((8, 64, 24), (16, 128, 40), (8, 136, 16)):   # one block, one block, two blocks of 72 and 64
        A = rng.integers(-3, 4, (P, K)).astype(f16)
        W = rng.integers(-3, 4, (N, K)).astype(f16)
        want = (A.astype(np.float64) @ W.T.astype(np.float64)).max(0)
        w, Kp, Np = hpack(W)
        cm = O.colmax_f16(A, w, Kp, Np)
        assert np.array_equal(cm[:N], want), (P, K, N)


# ---------------------------------------------------------------- whole ops
def test_proto_ops_compose():
    rng = np.random.default_rng(11)
    P, C, ld, N, nc = 16, 32, 40, 24, 6
    x = rng.standard_normal((P, ld)).astype(f32)
    protos = rng.standard_normal((N, C)).astype(f32)
    clsw = rng.uniform(0.5, 1.5, N).astype(f32)
    clsb = rng.standard_normal(nc).astype(f32)
    a = O.l2norm(x, C, 1e-5)
    panels, _, (_, _, Kp, Np) = netbuild.Net.fpack(protos, np.zeros(N, f32), K_pad=8)
    rc, lg, cm, a2 = O.proto_fp("f32", x, C, 1e-5, panels, Np, clsw, clsb, nc, N // nc)
    assert rc == 0 and np.array_equal(a, a2)
    assert np.array_equal(cm, O.colmax_f32(a, panels, Kp, Np))
    ref = np.zeros(nc, f32)
    for c in range(nc):
        s = f32(0)
        for q in range(N // nc):
            s = f32(s + f32(cm[c * (N // nc) + q] * clsw[c * (N // nc) + q]))
        ref[c] = f32(s + clsb[c])
    assert np.array_equal(lg, ref)
    # fp16 head: cells as fp16, the normalised cells rounded to fp16
    xh = x.astype(f16)
    rc, lg16, cm16, ah = O.proto_fp("f16", xh, C, 1e-5, hpack(protos.astype(f16))[0], Np, clsw, clsb, nc, N // nc)
    assert rc == 0 and np.array_equal(ah, O.l2norm(xh, C, 1e-5, f16=True))
    assert np.allclose(lg16, lg, rtol=0.05, atol=0.05)
