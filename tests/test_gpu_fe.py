"""GPU parity of the fp32 ops around the int8 GEMMs against the CPU oracle
(oracle/fe.c), all bit-identical: the device expf against the C library's
expf, the log-mel front end (Perch geometry, an odd frame length, a frame
shorter than the FFT, a signal with a click and silence), the stem, the
squeeze-excitation gate and in-place SE, the spatial mean and the halo copy,
each on several windows per launch with padded per-window strides."""
import numpy as np
import pytest

import pyoracle as O
from bnneon import perchnet

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.dtype == b.dtype and a.shape == b.shape, (a.dtype, b.dtype, a.shape, b.shape)
    an, bn = np.isnan(a), np.isnan(b)
    u = np.uint16 if a.dtype == np.float16 else np.uint32
    return bool(np.array_equal(an, bn) and np.array_equal(a.view(u)[~an], b.view(u)[~bn]))


def strided(a, slack):
    B = a.shape[0]
    n = a[0].size
    out = np.zeros((B, n + slack), a.dtype)
    out[:, :n] = a.reshape(B, n)
    return out, n + slack


def test_expf_matches_c_library(hip):
    H = hip
    rng = np.random.default_rng(0)
    bits = np.concatenate([rng.integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32),
                           np.arange(0xc2d00000, 0xc2d80000, dtype=np.uint32),   # around -104 (underflow edge)
                           np.arange(0x42b00000, 0x42b20000, dtype=np.uint32),   # around 88 (overflow edge)
                           np.arange(0x3f000000, 0x3f100000, dtype=np.uint32)])  # [0.5, 0.56)
    x = bits.view(np.float32)
    say("expf", x.size)
    dx = H.DeviceArray.from_host(x)
    dy = H.DeviceArray(x.shape, np.float32)
    H.check(H.lib().bnh_eval_expf(dx.ptr, dy.ptr, x.size, None), "eval_expf")
    H.sync()
    assert same_bits(dy.numpy(), O.expf(x))


def test_powf_matches_c_library(hip):
    """the device powf (GEM_A's final power) against the C library's on GEM_A's arguments (means over [2^-130, 2^8)
    with y = 1/p), on random finite pairs and on the special cases"""
    H = hip
    rng = np.random.default_rng(1)
    n = 1 << 21
    xb = rng.integers(0x00400000, 0x43800000, n, dtype=np.uint64).astype(np.uint32)
    ys = (np.float32(1) / np.array([1, 1.5, 2, 2.5, 3, 3.5, 4, 5, 6, 8, 10], np.float32)).astype(np.float32)
    x = np.concatenate([xb.view(np.float32), rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
                        .view(np.float32)])
    y = np.concatenate([ys[rng.integers(0, ys.size, n)], (rng.standard_normal(n) * 8).astype(np.float32)])
    sp = np.array([0, -0.0, 1, -1, 2, -2, 0.5, np.inf, -np.inf, np.nan, 1e-45, 3e38, -3], np.float32)
    sy = np.array([0, -0.0, 1, -1, 2, 3, -3, 0.5, np.inf, -np.inf, np.nan, 1.5, 200], np.float32)
    gx, gy = np.meshgrid(sp, sy)
    x = np.concatenate([x, gx.ravel()]).astype(np.float32)
    y = np.concatenate([y, gy.ravel()]).astype(np.float32)
    say("powf", x.size)
    dx, dy = H.DeviceArray.from_host(x), H.DeviceArray.from_host(y)
    dz = H.DeviceArray(x.shape, np.float32)
    H.check(H.lib().bnh_eval_powf(dx.ptr, dy.ptr, dz.ptr, x.size, None), "eval_powf")
    H.sync()
    assert same_bits(dz.numpy(), O.powf(x, y))


def run_logmel(H, pcm, frame, hop, pad, nfft, window, mel, floor_, scale, slack=5):
    B, nsamp = pcm.shape
    nmel = mel.shape[0]
    F = H.lib().bnh_logmel_new(nsamp, frame, hop, pad, nfft, nmel, np.ascontiguousarray(window, np.float32).ctypes.data,
                               np.ascontiguousarray(mel, np.float32).ctypes.data, floor_, scale)
    if not F:
        H.check(None, "bnh_logmel_new")
    try:
        nfr = H.lib().bnh_logmel_frames(F)
        xs, x_ws = strided(pcm.astype(np.float32), slack)
        dx = H.DeviceArray.from_host(xs)
        s_ws = nfr * nmel + 3
        do = H.DeviceArray.from_host(np.full((B, s_ws), np.nan, np.float32))
        H.check(H.lib().bnh_logmel_run(F, dx.ptr, x_ws, do.ptr, s_ws, B, None), "logmel")
        H.sync()
        return do.numpy()[:, :nfr * nmel].reshape(B, nfr, nmel)
    finally:
        H.lib().bnh_logmel_free(F)


def test_logmel_perch_geometry(hip):
    rng = np.random.default_rng(1)
    B = 3
    pcm = np.stack([perchnet.signal(rng) for _ in range(B)])
    pcm[1, 5000] = 1.0          # a click
    pcm[2, 40000:80000] = 0.0   # silence: the floor
    window = (0.5 - 0.5 * np.cos(2 * np.pi * np.arange(640) / 640)).astype(np.float32)
    mel = perchnet.mel_bank()
    say("logmel perch", B)
    got = run_logmel(hip, pcm, 640, 320, 160, 1024, window, mel, 1e-3, 1.0)
    assert got.shape == (B, 500, 128)
    for i in range(B):
        assert same_bits(got[i], O.logmel(pcm[i], 640, 320, 160, 1024, window, mel, 1e-3, 1.0)), i


@pytest.mark.parametrize("nsamp,frame,hop,pad,nfft,nmel", [(2000, 201, 100, 50, 256, 8), (3000, 64, 48, 0, 64, 5),
                                                           (1500, 400, 160, 200, 512, 40), (900, 16, 16, 7, 16, 3)])
def test_logmel_geometries(hip, nsamp, frame, hop, pad, nfft, nmel):
    rng = np.random.default_rng(nsamp + nfft)
    pcm = rng.standard_normal((2, nsamp)).astype(np.float32) * 0.3
    window = rng.uniform(-0.2, 1.0, frame).astype(np.float32)   # negative taps: -0 products in the pad
    bins = nfft // 2 + 1
    mel = np.where(rng.uniform(0, 1, (nmel, bins)) < 0.3, rng.uniform(0, 1, (nmel, bins)), 0).astype(np.float32)
    mel[:, 0] = 0
    mel[0, 0] = 0.5      # DC and Nyquist bins in use
    mel[-1, -1] = 0.25
    say("logmel", nsamp, frame, hop, pad, nfft, nmel)
    got = run_logmel(hip, pcm, frame, hop, pad, nfft, window, mel, 1e-4, 0.7)
    for i in range(2):
        assert same_bits(got[i], O.logmel(pcm[i], frame, hop, pad, nfft, window, mel, 1e-4, 0.7)), i


@pytest.mark.parametrize("Hh,W,k,s,co,act,opad", [(500, 128, 3, 2, 40, 1, 1), (33, 20, 5, 1, 12, 2, 0),
                                                   (17, 19, 1, 1, 8, 0, 2), (40, 30, 7, 3, 16, 1, 0),
                                                   (33, 20, 3, 1, 24, 1, 0)])
def test_stem(hip, Hh, W, k, s, co, act, opad):
    H = hip
    rng = np.random.default_rng(Hh + k)
    B = 3
    img = (rng.standard_normal((B, Hh, W)) * 3).astype(np.float32)
    w = (rng.standard_normal((co, k * k)) * np.sqrt(2 / (k * k))).astype(np.float32)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    panels, bb, (N, K, Kp, Np) = O.fpack(w, b)
    Ho, Wo = (Hh - k) // s + 1, (W - k) // s + 1
    ldo = Np + 4
    xs, x_ws = strided(img, 7)
    dx = H.DeviceArray.from_host(xs)
    dw = H.DeviceArray.from_host(panels)
    db = H.DeviceArray.from_host(bb)
    rows = (Ho + 2 * opad) * (Wo + 2 * opad)
    o_ws = rows * ldo + 8
    do = H.DeviceArray.from_host(np.full((B, o_ws), 5.0, np.float32))
    say("stem", Hh, W, k, s, co)
    H.check(H.lib().bnh_stem_f32(dx.ptr, x_ws, Hh, W, k, s, Ho, Wo, dw.ptr, db.ptr, Kp, Np, act, do.ptr, o_ws, ldo,
                                 opad, B, None), "stem")
    H.sync()
    got = do.numpy()[:, :rows * ldo].reshape(B, rows, ldo)
    for i in range(B):
        want = O.stem_f32(img[i], k, s, panels, bb, Kp, Np, act=act, opad=opad, ldo=ldo)
        assert same_bits(got[i][:, :Np], want[:, :Np]), i
        if not opad:
            assert (got[i][:, Np:] == 5.0).all()   # channels past Np untouched


@pytest.mark.parametrize("C,rd,P,inplace,ws", [(40, 10, 15687, False, True), (2304, 96, 64, False, True),
                                               (2304, 96, 64, False, False), (36, 9, 100, True, True),
                                               (4096, 512, 8, False, True), (816, 34, 256, True, True),
                                               (816, 34, 256, True, False), (1392, 58, 5, False, True)])
def test_se(hip, C, rd, P, inplace, ws):
    """ws: with the FC workspace (two kernels over all windows) or without (one kernel per group of windows)."""
    H = hip
    rng = np.random.default_rng(C + rd)
    B = 3
    chsum = (rng.standard_normal((B, C)) * np.sqrt(P) * 0.5).astype(np.float32)
    chsum[0, :4] = [np.inf, -np.inf, 0.0, -0.0] if C > 8 else chsum[0, :4]
    w1 = (rng.standard_normal((rd, C)) * np.sqrt(2 / C)).astype(np.float32)
    b1 = (rng.standard_normal(rd) * 2).astype(np.float32)   # large fc1 outputs: expf far from 1
    w2t = (rng.standard_normal((rd, C)) * np.sqrt(2 / rd)).astype(np.float32)
    b2 = (rng.standard_normal(C) * 3).astype(np.float32)
    cs, c_ws = strided(chsum, 3)
    dc = H.DeviceArray.from_host(cs)
    dt = [H.DeviceArray.from_host(a) for a in (w1, b1, w2t, b2)]
    g_ws = C + 5
    dg = H.DeviceArray.from_host(np.zeros((B, g_ws), np.float32))
    D = rng.standard_normal((B, P, C)).astype(np.float32) if inplace else None
    dD, d_ws = (None, 0)
    if inplace:
        Ds, d_ws = strided(D, 9)
        dD = H.DeviceArray.from_host(Ds)
    dwk = H.DeviceArray.from_host(np.full((B, rd), 3.0, np.float32)) if ws else None
    say("se", C, rd, P, inplace, ws)
    H.check(H.lib().bnh_se_f32(dc.ptr, c_ws, C, rd, P, dt[0].ptr, dt[1].ptr, dt[2].ptr, dt[3].ptr, dg.ptr, g_ws,
                               dwk.ptr if ws else None, dD.ptr if inplace else None, d_ws, B, None), "se")
    H.sync()
    g = dg.numpy()[:, :C]
    for i in range(B):
        want = O.se_gate_f32(chsum[i], P, w1, b1, w2t, b2)
        assert same_bits(g[i], want), i
        if inplace:
            got = dD.numpy()[i, :P * C].reshape(P, C)
            assert same_bits(got, (D[i] * want[None, :]).astype(np.float32)), i


def test_mean_and_pad(hip):
    H = hip
    rng = np.random.default_rng(9)
    B, P, C, ld = 3, 64, 1536, 1544
    x = rng.standard_normal((B, P, ld)).astype(np.float32)
    xs, x_ws = strided(x, 11)
    dx = H.DeviceArray.from_host(xs)
    do = H.DeviceArray.from_host(np.zeros((B, C + 4), np.float32))
    say("mean")
    H.check(H.lib().bnh_mean_f32(dx.ptr, x_ws, P, C, ld, do.ptr, C + 4, B, None), "mean")
    H.sync()
    for i in range(B):
        assert same_bits(do.numpy()[i, :C], O.mean_f32(x[i], C))
    # 16-byte vectors (strides that allow them) and single elements (odd window strides)
    for esz, dt, slack, pslack in ((4, np.float32, 3, 6), (2, np.float16, 3, 6), (4, np.float32, 8, 4),
                                   (2, np.float16, 16, 8)):
        Hh, W, C, ld, h = 9, 7, 24, 32, 2
        x = rng.standard_normal((B, Hh * W, ld)).astype(dt)
        xs, x_ws = strided(x, slack)
        dx = H.DeviceArray.from_host(xs)
        per = (Hh + 2 * h) * (W + 2 * h) * C
        dp = H.DeviceArray.from_host(np.full((B, per + pslack), 9, dt))
        say("pad", esz, slack)
        H.check(H.lib().bnh_pad(dx.ptr, x_ws, Hh, W, C, ld, h, esz, dp.ptr, per + pslack, B, None), "pad")
        H.sync()
        got = dp.numpy()[:, :per]
        for i in range(B):
            assert np.array_equal(got[i].reshape(-1), O.pad(x[i], Hh, W, C, h).reshape(-1)), (esz, i)
        assert (dp.numpy()[:, per:] == 9).all()


# ---------------------------------------------------------------- the fp16 path's ops around its GEMMs
@pytest.mark.parametrize("Hh,W,k,s,co,opad,ldo", [(257, 96, 3, 2, 24, 0, 24), (33, 20, 5, 1, 12, 1, 16),
                                                  (17, 19, 3, 2, 20, 2, 24)])
def test_stem_f32to16(hip, Hh, W, k, s, co, opad, ldo):
    H = hip
    rng = np.random.default_rng(Hh + k + co)
    B = 3
    img = (rng.standard_normal((B, Hh, W)) * 3).astype(np.float32)
    img[0, 0, :4] = [1e5, -1e5, 7e4, np.nan]    # fp16 overflow to +-inf and a NaN pixel
    w = (rng.standard_normal((co, k * k)) * np.sqrt(2 / (k * k))).astype(np.float32)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    panels, bb, (N, K, Kp, Np) = O.fpack(w, b)
    Ho, Wo = (Hh - k) // s + 1, (W - k) // s + 1
    xs, x_ws = strided(img, 7)
    dx = H.DeviceArray.from_host(xs)
    dw = H.DeviceArray.from_host(panels)
    db = H.DeviceArray.from_host(bb)
    rows = (Ho + 2 * opad) * (Wo + 2 * opad)
    o_ws = rows * ldo + 8
    do = H.DeviceArray.from_host(np.full((B, o_ws), 5.0, np.float16))
    say("stem f32to16", Hh, W, k, s, co, opad)
    H.check(H.lib().bnh_stem_f32to16(dx.ptr, x_ws, Hh, W, k, s, Ho, Wo, dw.ptr, db.ptr, Kp, co, Np, 1, do.ptr, o_ws,
                                     ldo, opad, B, None), "stem_f32to16")
    H.sync()
    got = do.numpy()
    assert (got[:, rows * ldo:] == 5.0).all()
    got = got[:, :rows * ldo].reshape(B, rows, ldo)
    for i in range(B):
        want = O.stem_f32to16(img[i], k, s, panels, bb, Kp, co, Np, act=1, opad=opad, ldo=ldo, fill=5.0)
        assert same_bits(got[i], want), i


@pytest.mark.parametrize("C,rd,P,ws", [(72, 6, 1536, True), (1536, 48, 24, True), (288, 9, 384, False),
                                        (16, 1, 7, True), (40, 3, 33, False)])
def test_se_f16(hip, C, rd, P, ws):
    """ws: with a gate workspace (gates, then a scaling kernel over all pixels) or without (one kernel)."""
    H = hip
    rng = np.random.default_rng(C + rd)
    B = 3
    D = rng.standard_normal((B, P, C)).astype(np.float16)
    D[0, 0, :3] = [np.inf, -np.inf, 60000]
    chsum = np.stack([D[i].astype(np.float32).sum(0) for i in range(B)]).astype(np.float32)
    chsum[0, :3] = [1.0, -2.0, 3.0]
    w1 = (rng.standard_normal((rd, C)) * np.sqrt(2 / C)).astype(np.float32)
    b1 = (rng.standard_normal(rd) * 2).astype(np.float32)
    w2t = (rng.standard_normal((rd, C)) * np.sqrt(2 / rd)).astype(np.float32)
    b2 = (rng.standard_normal(C) * 3).astype(np.float32)
    cs, c_ws = strided(chsum, 3)
    dc = H.DeviceArray.from_host(cs)
    dt = [H.DeviceArray.from_host(a) for a in (w1, b1, w2t, b2)]
    Ds, d_ws = strided(D, 9)
    dD = H.DeviceArray.from_host(Ds)
    g_ws = C + 4
    dg = H.DeviceArray.from_host(np.zeros((B, g_ws), np.float32)) if ws else None
    dwk = H.DeviceArray.from_host(np.zeros((B, rd), np.float32)) if ws else None
    say("se f16", C, rd, P, ws)
    H.check(H.lib().bnh_se_f16(dc.ptr, c_ws, C, rd, P, dt[0].ptr, dt[1].ptr, dt[2].ptr, dt[3].ptr,
                               dg.ptr if ws else None, g_ws, dwk.ptr if ws else None, dD.ptr, d_ws, B, None),
            "se_f16")
    H.sync()
    got = dD.numpy()
    for i in range(B):
        assert same_bits(got[i, :P * C].reshape(P, C), O.se_f16(D[i], chsum[i], w1, b1, w2t, b2)), i
        assert (got[i, P * C:] == 0).all()
        if ws:   # the gates as the fp32 SE computes them, with the dividing sigmoid
            assert same_bits(O.se_f16(np.ones((P, C), np.float16), chsum[i], w1, b1, w2t, b2)[0],
                             dg.numpy()[i, :C].astype(np.float16)), i
    if ws and C % 8 == 0:   # the gates alone: fp32 and their fp16 roundings
        dg2 = H.DeviceArray.from_host(np.zeros((B, g_ws), np.float32))
        gh_ws = C + 8
        dh = H.DeviceArray.from_host(np.zeros((B, gh_ws), np.float16))
        H.check(H.lib().bnh_se_gate_f16(dc.ptr, c_ws, C, rd, P, dt[0].ptr, dt[1].ptr, dt[2].ptr, dt[3].ptr, dg2.ptr,
                                        g_ws, dwk.ptr, dh.ptr, gh_ws, B, None), "se_gate_f16")
        H.sync()
        assert np.array_equal(dg2.numpy()[:, :C].view(np.uint32), dg.numpy()[:, :C].view(np.uint32))
        assert same_bits(dh.numpy()[:, :C], dg.numpy()[:, :C].astype(np.float16))
        assert (dh.numpy()[:, C:] == 0).all()


def test_mean_f16_and_gemv(hip):
    H = hip
    rng = np.random.default_rng(12)
    B, P, C, ld = 3, 24, 1024, 1032
    x = rng.standard_normal((B, P, ld)).astype(np.float16)
    x[1, 3, 5] = np.inf
    xs, x_ws = strided(x, 5)
    dx = H.DeviceArray.from_host(xs)
    do = H.DeviceArray.from_host(np.zeros((B, C + 4), np.float32))
    say("mean f16")
    H.check(H.lib().bnh_mean_f16(dx.ptr, x_ws, P, C, ld, do.ptr, C + 4, B, None), "mean_f16")
    H.sync()
    m = do.numpy()[:, :C]
    for i in range(B):
        assert same_bits(m[i], O.mean_f16(x[i], C))
    # GEMV, fp16 and fp32 weights, K with 8-lane, 4-lane and scalar remainders, ReLU; 8, 4 and 2 windows a block (K up
    # to 2048, 4096 and 8192: their inputs fill at most 64 KB of LDS)
    for K, N, w16, act in ((1024, 6522, 1, 0), (1027, 300, 1, 2), (1536, 1000, 0, 0), (13, 33, 0, 2), (6, 17, 1, 0),
                           (3001, 70, 1, 0), (5003, 40, 0, 2)):
        w = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float16 if w16 else np.float32)
        b = (rng.standard_normal(N) * 0.1).astype(np.float32)
        xv = rng.standard_normal((B, K)).astype(np.float32)
        xvs, xv_ws = strided(xv, 3)
        dxv = H.DeviceArray.from_host(xvs)
        dwt = H.DeviceArray.from_host(w)
        dbt = H.DeviceArray.from_host(b)
        dy = H.DeviceArray.from_host(np.full((B, N + 2), 9.0, np.float32))
        say("gemv", K, N, w16, act)
        H.check(H.lib().bnh_gemv(dwt.ptr, w16, dbt.ptr, N, K, dxv.ptr, xv_ws, act, dy.ptr, N + 2, B, None), "gemv")
        H.sync()
        y = dy.numpy()
        assert (y[:, N:] == 9.0).all()
        for i in range(B):
            assert same_bits(y[i, :N], O.gemv(w, b, xv[i], act)), (K, N, w16, i)
    # 20 windows: two full groups of 8 and a partial one
    K, N, B2 = 1024, 500, 20
    w = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    xv = rng.standard_normal((B2, K)).astype(np.float32)
    dxv, dwt, dbt = H.DeviceArray.from_host(xv), H.DeviceArray.from_host(w), H.DeviceArray.from_host(b)
    dy = H.DeviceArray.from_host(np.zeros((B2, N), np.float32))
    say("gemv 20 windows")
    H.check(H.lib().bnh_gemv(dwt.ptr, 1, dbt.ptr, N, K, dxv.ptr, K, 0, dy.ptr, N, B2, None), "gemv")
    H.sync()
    y = dy.numpy()
    for i in (0, 15, 16, 19):
        assert same_bits(y[i], O.gemv(w, b, xv[i], 0)), i
