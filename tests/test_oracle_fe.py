"""Pins the oracle's fp32 ops around the int8 GEMMs (oracle/fe.c): the
log2 / exp2 / sigmoid approximations against the exact functions within their
stated accuracy and at their exact points, the log-mel front end against a
float64 real FFT of the same frames, the fp32 GEMM and the stem exactly on
integer-valued data (where every fp32 operation is exact, so any index, layout
or operand slip shows) and within fp32 error on random data, the SE gate
against its float64 formula, the mean exactly on integers and the halo copy
exactly."""
import math

import numpy as np

import pyoracle as O


def test_log2_exp2_sigmoid():
    L = O.lib()
    for e in range(-20, 21):
        assert L.orc_log2_acc(2.0 ** e) == e
        assert L.orc_exp2_f32(float(e)) == 2.0 ** e
    assert L.orc_exp2_f32(200.0) == 2.0 ** 126 and L.orc_exp2_f32(-200.0) == 2.0 ** -126
    rng = np.random.default_rng(0)
    x = np.exp(rng.uniform(-30, 30, 5000)).astype(np.float32)
    got = np.array([L.orc_log2_acc(float(v)) for v in x])
    assert np.abs(got - np.log2(x.astype(np.float64))).max() < 1e-5
    t = rng.uniform(-100, 100, 5000).astype(np.float32)
    got = np.array([L.orc_exp2_f32(float(v)) for v in t])
    ex = np.exp2(t.astype(np.float64))
    assert (np.abs(got - ex) / ex).max() < 5e-7
    s = rng.uniform(-30, 30, 5000).astype(np.float32)
    got = np.array([L.orc_sigmoid_f32(float(v)) for v in s])
    assert np.abs(got - 1 / (1 + np.exp(-s.astype(np.float64)))).max() < 1e-6
    assert L.orc_sigmoid_f32(0.0) == 0.5


def mel_bank(nmel, nfft, sr, fmin=60.0, fmax=None):
    """triangular filters on the mel scale (a synthetic front end's filter bank)."""
    fmax = fmax or sr / 2
    bins = nfft // 2 + 1
    hz = np.linspace(0, sr / 2, bins)
    m = lambda f: 2595 * np.log10(1 + f / 700)
    pts = 700 * (10 ** (np.linspace(m(fmin), m(fmax), nmel + 2) / 2595) - 1)
    W = np.zeros((nmel, bins), np.float32)
    for j in range(nmel):
        lo, c, hi = pts[j], pts[j + 1], pts[j + 2]
        W[j] = np.maximum(0, np.minimum((hz - lo) / (c - lo), (hi - hz) / (hi - c)))
    return W


def close_logmel(spec, pcm, frame, hop, pad, nfft, window, mel, floor_, scale):
    """spec against float64 in the energy domain: the fp32 FFT's error is relative to the frame's energy, so
    |exp(spec / scale) - max(E64, floor)| <= 1e-5 max_j E64 + 1e-5 E64 per frame."""
    E = ref_logmel64(pcm, frame, hop, pad, nfft, window, mel, floor_, None)
    got = np.exp(spec.astype(np.float64) / scale)
    tol = 1e-5 * E.max(1, keepdims=True) + 1e-5 * E
    return (np.abs(got - np.maximum(E, floor_)) <= tol).all(), float(np.max(np.abs(got - np.maximum(E, floor_)) / tol))


def ref_logmel64(pcm, frame, hop, pad, nfft, window, mel, floor_, scale):
    y = np.concatenate([np.zeros(pad), pcm.astype(np.float64), np.zeros(nfft + hop)])
    nfr = (pcm.size + 2 * pad - frame) // hop + 1
    out = np.zeros((nfr, mel.shape[0]))
    w = np.zeros(nfft)
    w[:frame] = window
    for t in range(nfr):
        X = np.fft.rfft(y[t * hop:t * hop + nfft] * w)
        E = mel.astype(np.float64) @ np.abs(X)
        out[t] = E if scale is None else np.log(np.maximum(E, floor_)) * scale
    return out


def test_logmel_against_float64_fft():
    rng = np.random.default_rng(1)
    sr, nsamp, frame, hop, pad, nfft = 32000, 6400, 640, 320, 160, 1024
    t = np.arange(nsamp) / sr
    pcm = (0.03 * rng.standard_normal(nsamp) + 0.5 * np.sin(2 * np.pi * 3000 * t)).astype(np.float32)
    window = (0.5 - 0.5 * np.cos(2 * np.pi * np.arange(frame) / frame)).astype(np.float32)
    mel = mel_bank(128, nfft, sr)
    spec = O.logmel(pcm, frame, hop, pad, nfft, window, mel, 1e-3, 0.5)
    assert spec.shape == (20, 128)
    ok, worst = close_logmel(spec, pcm, frame, hop, pad, nfft, window, mel, 1e-3, 0.5)
    assert ok, worst


def test_logmel_sine_peak_and_odd_frame():
    """a sine on bin 96 of a 256-point FFT peaks in the filter covering bin 96; an odd frame length (the last sample
    pairs with a zero window tap) and a frame shorter than nfft agree with float64 too."""
    sr, nfft, frame, hop, pad = 8000, 256, 201, 100, 50
    nsamp = 2000
    pcm = np.sin(2 * np.pi * 96 * sr / nfft * np.arange(nsamp) / sr).astype(np.float32)
    window = np.hanning(frame + 2)[1:-1].astype(np.float32)
    bins = nfft // 2 + 1
    mel = np.zeros((8, bins), np.float32)
    for j in range(8):
        mel[j, 16 * j:16 * j + 16] = 1.0
    spec = O.logmel(pcm, frame, hop, pad, nfft, window, mel, 1e-6, 1.0)
    assert (spec[2:-2].argmax(1) == 6).all()
    ok, worst = close_logmel(spec, pcm, frame, hop, pad, nfft, window, mel, 1e-6, 1.0)
    assert ok, worst


def test_gemm_f32_exact_on_integers():
    rng = np.random.default_rng(2)
    M, N, K = 37, 21, 13
    A = rng.integers(-8, 9, (M, 20)).astype(np.float32)
    w = rng.integers(-8, 9, (N, K)).astype(np.float32)
    b = rng.integers(-50, 50, N).astype(np.float32)
    panels, bb, (N_, K_, Kp, Np) = O.fpack(w, b)
    assert (Kp, Np) == (16, 24)
    out = O.gemm_f32(A, panels, bb, Kp, Np)
    want = A[:, :K] @ w.T + b
    assert np.array_equal(out[:, :N], want) and not out[:, N:].any()
    g = rng.integers(-2, 3, Kp).astype(np.float32)
    out = O.gemm_f32(A, panels, bb, Kp, Np, gate=g)
    assert np.array_equal(out[:, :N], (A[:, :K] * g[:K]) @ w.T + b)
    res = rng.integers(-9, 9, (M, Np)).astype(np.float32)
    out = O.gemm_f32(A, panels, bb, Kp, Np, act=2, res=res, ldr=Np)
    assert np.array_equal(out[:, :N], np.maximum(A[:, :K] @ w.T + b, 0) + res[:, :N])
    silu = O.gemm_f32(A, panels, bb, Kp, Np, act=1)
    assert np.array_equal(silu, O.eval_f32(1, O.gemm_f32(A, panels, bb, Kp, Np)))
    # padded store: M = 37 rows as 37 x 1 pixels... use 36 rows as 6 x 6 with halo 2
    out = O.gemm_f32(A[:36], panels, bb, Kp, Np, ow=6, opad=2).reshape(10, 10, Np)
    assert not out[:2].any() and not out[:, :2].any() and not out[-2:].any() and not out[:, -2:].any()
    assert np.array_equal(out[2:8, 2:8, :N].reshape(36, N), A[:36, :K] @ w.T + b)


def test_gemm_f32_random_within_fp32_bound():
    rng = np.random.default_rng(3)
    M, N, K = 50, 40, 100
    A = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((N, K)).astype(np.float32)
    panels, bb, (_, _, Kp, Np) = O.fpack(w, np.zeros(N))
    out = O.gemm_f32(A, panels, bb, Kp, Np)[:, :N]
    ex = A.astype(np.float64) @ w.T.astype(np.float64)
    bound = K * 2.0 ** -24 * (np.abs(A).astype(np.float64) @ np.abs(w).T.astype(np.float64))
    assert (np.abs(out - ex) <= bound).all()


def test_stem_exact_on_integers():
    rng = np.random.default_rng(4)
    H, W, k, s = 11, 9, 3, 2
    img = rng.integers(-5, 6, (H, W)).astype(np.float32)
    w = rng.integers(-3, 4, (40, k * k)).astype(np.float32)
    b = rng.integers(-5, 6, 40).astype(np.float32)
    panels, bb, (N, K, Kp, Np) = O.fpack(w, b)
    assert Kp == 12
    out = O.stem_f32(img, k, s, panels, bb, Kp, Np, act=0, opad=1)
    Ho, Wo = (H - k) // s + 1, (W - k) // s + 1
    out = out.reshape(Ho + 2, Wo + 2, Np)
    cols = np.stack([img[ky:ky + s * (Ho - 1) + 1:s, kx:kx + s * (Wo - 1) + 1:s]
                     for ky in range(k) for kx in range(k)], -1)
    want = cols.reshape(-1, k * k) @ w.T + b
    assert np.array_equal(out[1:-1, 1:-1].reshape(-1, Np), want)
    assert not out[0].any() and not out[:, 0].any() and not out[-1].any() and not out[:, -1].any()


def test_se_gate_against_float64():
    rng = np.random.default_rng(5)
    for Cc, rd in ((40, 10), (36, 9), (576, 24)):
        P_ = 63
        chsum = (rng.standard_normal(Cc) * 20).astype(np.float32)
        w1 = (rng.standard_normal((rd, Cc)) * 0.2).astype(np.float32)
        b1 = rng.standard_normal(rd).astype(np.float32)
        w2t = (rng.standard_normal((rd, Cc)) * 0.3).astype(np.float32)
        b2 = rng.standard_normal(Cc).astype(np.float32)
        g = O.se_gate_f32(chsum, P_, w1, b1, w2t, b2)
        m = chsum.astype(np.float64) / P_
        h = w1.astype(np.float64) @ m + b1
        s1 = h / (1 + np.exp(-h))
        ex = 1 / (1 + np.exp(-(w2t.T.astype(np.float64) @ s1 + b2)))
        assert np.abs(g - ex).max() < 2e-5


def test_mean_and_pad():
    rng = np.random.default_rng(6)
    x = rng.integers(-100, 100, (64, 24)).astype(np.float32)
    m = O.mean_f32(x, 20)
    assert np.array_equal(m, (x[:, :20].sum(0) / np.float32(64)).astype(np.float32))
    x = rng.standard_normal((6 * 5, 16)).astype(np.float32)
    p = O.pad(x, 6, 5, 12, 2).reshape(10, 9, 12)
    assert np.array_equal(p[2:8, 2:7], x[:, :12].reshape(6, 5, 12))
    assert not p[:2].any() and not p[-2:].any() and not p[:, :2].any() and not p[:, -2:].any()


# ---------------------------------------------------------------- the fp16 path's ops (oracle/fe.c)
def test_stem_f32to16_is_the_fp32_stem_rounded():
    rng = np.random.default_rng(7)
    H, W, k, s, co = 13, 12, 3, 2, 20
    img = (rng.standard_normal((H, W)) * 4).astype(np.float32)
    img[0, 0] = 1e6   # past the fp16 range: +inf after the rounding
    w = rng.standard_normal((co, k * k)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32)
    panels, bb, (N, K, Kp, Np) = O.fpack(w, b)
    ref32 = O.stem_f32(img, k, s, panels, bb, Kp, Np, act=1, opad=0)
    got = O.stem_f32to16(img, k, s, panels, bb, Kp, co, Np, act=1, opad=1, ldo=Np, fill=3.0)
    Ho, Wo = (H - k) // s + 1, (W - k) // s + 1
    got = got.reshape(Ho + 2, Wo + 2, Np)
    inner = got[1:-1, 1:-1].reshape(-1, Np)
    want = ref32[:, :co].astype(np.float16)   # numpy's float32 -> float16 is round to nearest even
    assert np.array_equal(inner[:, :co].view(np.uint16), want.view(np.uint16))
    assert (inner[:, co:] == 3.0).all()        # channels past N untouched
    assert np.isinf(inner).any()
    assert not got[0].any() and not got[-1].any() and not got[:, 0].any() and not got[:, -1].any()


def test_se_f16_gate_and_product():
    rng = np.random.default_rng(8)
    P_, Cc, rd = 40, 48, 6
    D = rng.standard_normal((P_, Cc)).astype(np.float16)
    chsum = (rng.standard_normal(Cc) * 10).astype(np.float32)
    w1 = (rng.standard_normal((rd, Cc)) * 0.2).astype(np.float32)
    b1 = rng.standard_normal(rd).astype(np.float32)
    w2t = (rng.standard_normal((rd, Cc)) * 0.3).astype(np.float32)
    b2 = rng.standard_normal(Cc).astype(np.float32)
    got = O.se_f16(D, chsum, w1, b1, w2t, b2)
    g16 = O.se_f16(np.ones((P_, Cc), np.float16), chsum, w1, b1, w2t, b2)[0]   # 1 x g is g itself
    # the gate: the float64 formula, then one rounding to fp16 (the fp32 steps differ by ~1e-6 relative)
    m = chsum.astype(np.float64) / P_
    h = w1.astype(np.float64) @ m + b1
    ex = 1 / (1 + np.exp(-(w2t.T.astype(np.float64) @ (h / (1 + np.exp(-h))) + b2)))
    assert np.abs(g16.astype(np.float64) - ex).max() <= 2.0 ** -11 * ex.max() + 1e-6
    # the product: one fp16 multiply per element (numpy's float16 multiply rounds the exact product once)
    assert np.array_equal(got.view(np.uint16), (D * g16[None, :]).view(np.uint16))


def test_mean_f16_is_the_sequential_fp32_sum():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((300, 24)) * 100).astype(np.float16)
    m = O.mean_f16(x, 20)
    seq = np.add.accumulate(x[:, :20].astype(np.float32), axis=0, dtype=np.float32)[-1]
    assert np.array_equal(m, (seq / np.float32(300)).astype(np.float32))
    # the order shows: 60000, then 1e-4 terms each lost against it (ulp 2^-8 there), then -60000: the sequential
    # fp32 sum is 0 where the exact sum is 100 x 1e-4
    col = np.concatenate([[60000.0], np.full(100, 1e-4), [-60000.0]]).astype(np.float16)[:, None]
    assert O.mean_f16(col, 1)[0] == 0.0


def test_gemv_lane_order_and_exactness():
    rng = np.random.default_rng(10)
    # integer data: every fp32 operation exact, both weight forms, K with 8-lane, 4-lane and scalar parts
    for K in (16, 20, 23, 3):
        w = rng.integers(-4, 5, (7, K)).astype(np.float32)
        x = rng.integers(-9, 10, K).astype(np.float32)
        b = rng.integers(-5, 6, 7).astype(np.float32)
        want = w.astype(np.float64) @ x + b
        assert np.array_equal(O.gemv(w, b, x), want.astype(np.float32))
        assert np.array_equal(O.gemv(w.astype(np.float16), b, x), want.astype(np.float32))
        assert np.array_equal(O.gemv(w, b, x, act=2), np.maximum(want, 0).astype(np.float32))
    # the lane pairing ((l0 + l4) + (l1 + l5)) + ((l2 + l6) + (l3 + l7)): with 2^25 in lane 0 and 1 in lane 4 the 1
    # is lost (ulp 4 at 2^25) before lane 2's -2^25 cancels it; a sequential sum would keep both ones
    x = np.array([2.0 ** 25, 0, -2.0 ** 25, 0, 1, 0, 1, 0], np.float32)
    w = np.ones((1, 8), np.float32)
    assert O.gemv(w, np.zeros(1, np.float32), x)[0] == 0.0
    # the K % 4 tail: product and sum rounded apart (no fused multiply-add). The tail product is
    # 2^-24 (1 + 2^-36), which rounds to 2^-24; 1 + 2^-24 is then a tie that rounds to even, 1.0 (one fused
    # operation would see a value above the tie and give 1 + 2^-23)
    x = np.zeros(9, np.float32)
    w = np.zeros((1, 9), np.float32)
    x[0], w[0, 0] = 1.0, 1.0
    w[0, 8] = np.float32(1 + 2.0 ** -12)
    x[8] = np.float32(2.0 ** -24 * (1 - 2.0 ** -12 + 2.0 ** -24))
    assert float(w[0, 8]) * float(x[8]) == 2.0 ** -24 * (1 + 2.0 ** -36)
    assert O.gemv(w, np.zeros(1, np.float32), x)[0] == np.float32(1.0)
