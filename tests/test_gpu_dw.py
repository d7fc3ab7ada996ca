"""GPU parity of the depthwise convolutions against the CPU oracle (oracle/dw.c).

fp32 and fp16 DWK / DW3 outputs and per-channel sums are bit-identical to the
oracle (any NaN equal to any NaN); the int8 depthwise is bit-exact. Cases: the
EfficientNet block shape (C = 672, 24 x 64, k 3 / 5, strides 1 / 2, 'same'
pads), every row-tail form (Wo % 4 = 0..3), k = 7, channel counts that are not a
multiple of the wavefront, padded per-window strides, and inputs holding
infinities and NaNs.
"""
import numpy as np
import pytest

import pyoracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same_bits(a, b):
    """Bit equality of float arrays, any NaN equal to any NaN."""
    a, b = np.asarray(a), np.asarray(b)
    assert a.dtype == b.dtype and a.shape == b.shape
    an, bn = np.isnan(a), np.isnan(b)
    u = np.uint16 if a.dtype == np.float16 else np.uint32
    return bool(np.array_equal(an, bn) and np.array_equal(a.view(u)[~an], b.view(u)[~bn]))


def same_pads(n, k, s):
    """TF 'same': output size and leading pad."""
    o = (n - 1) // s + 1
    return o, max((o - 1) * s + k - n, 0) // 2


def haloed(rng, B, H, W, C, h, dtype, specials=False):
    xp = np.zeros((B, H + 2 * h, W + 2 * h, C), dtype)
    x = rng.standard_normal((B, H, W, C)).astype(np.float32)
    if specials:
        flat = x.reshape(-1)
        idx = rng.choice(flat.size, 8, replace=False)
        flat[idx] = [np.inf, -np.inf, np.nan, 7e4, -7e4, 1e-6, -0.0, 300.0]
    xp[:, h:h + H, h:h + W] = x.astype(dtype)
    return xp


def weights(rng, k, C, dtype):
    w = (rng.standard_normal((k * k, C)) * np.sqrt(2.0 / (k * k))).astype(dtype)
    b = (rng.standard_normal(C) * 0.1).astype(dtype)
    return w, b


def with_slack(a, slack):
    """[B][...] -> [B][n + slack] (padded per-window stride) and the stride."""
    B = a.shape[0]
    n = a[0].size
    out = np.zeros((B, n + slack), a.dtype)
    out[:, :n] = a.reshape(B, n)
    return out, n + slack


def run_dw(hip, form, xp, H, W, C, k, s, pt, pl, w, b, act, Ho, Wo, chsum=True, slack=40):
    """Runs one of the four float depthwise entry points over the B windows of xp."""
    Hh = hip
    B = xp.shape[0]
    xs, x_ws = with_slack(xp, slack)
    o_ws = Ho * Wo * C + slack
    cs_ws = C + 8
    dt = xp.dtype
    dx = Hh.DeviceArray.from_host(xs)
    dw_, db = Hh.DeviceArray.from_host(w), Hh.DeviceArray.from_host(b)
    do = Hh.DeviceArray.zeros((B, o_ws), dt)
    dcs = Hh.DeviceArray.zeros((B, cs_ws), np.float32) if chsum else None
    L = Hh.lib()
    csp = dcs.ptr if chsum else None
    if form == "dwk":
        f = L.bnh_dwk_f32 if dt == np.float32 else L.bnh_dwk_f16
        rc = f(dx.ptr, x_ws, H, W, C, k, s, pt, pl, dw_.ptr, db.ptr, act, do.ptr, o_ws, Ho, Wo, csp, cs_ws, B, None)
    elif dt == np.float32:
        rc = L.bnh_dw3_f32(dx.ptr, x_ws, H, W, C, s, dw_.ptr, db.ptr, do.ptr, o_ws, Ho, Wo, csp, cs_ws, B, None)
    else:
        rc = L.bnh_dw3_f16(dx.ptr, x_ws, H, W, C, s, pt, pl, dw_.ptr, db.ptr, do.ptr, o_ws, Ho, Wo, csp, cs_ws, B,
                           None)
    Hh.check(rc, form)
    Hh.sync()
    out = do.numpy()[:, :Ho * Wo * C].reshape(B, Ho, Wo, C)
    cs = dcs.numpy()[:, :C] if chsum else None
    return out, cs


def oracle_dw(form, xp1, H, W, C, k, s, pt, pl, w, b, act, Ho, Wo):
    if form == "dwk":
        f = O.dwk_f32 if xp1.dtype == np.float32 else O.dwk_f16
        return f(xp1, H, W, C, k, s, pt, pl, w, b, act, Ho, Wo)
    if xp1.dtype == np.float32:
        return O.dw3_f32(xp1, H, W, C, s, w, b, Ho, Wo)
    return O.dw3_f16(xp1, H, W, C, s, pt, pl, w, b, Ho, Wo)


def check_case(hip, form, dtype, B, H, W, C, k, s, pt, pl, act, seed, specials=False, windows=None):
    rng = np.random.default_rng(seed)
    h = (k - 1) // 2
    Ho, _ = same_pads(H, k, s)
    Wo, _ = same_pads(W, k, s)
    if form == "dw3" and dtype == np.float32:
        pt = pl = 1   # the fp32 DW3 kernels read rows oy*s, columns ox*s of the halo-1 input
    xp = haloed(rng, B, H, W, C, h, dtype, specials)
    w, b = weights(rng, k, C, dtype)
    say(form, np.dtype(dtype).name, "B", B, "HWC", H, W, C, "k", k, "s", s, "pads", pt, pl, "act", act)
    out, cs = run_dw(hip, form, xp, H, W, C, k, s, pt, pl, w, b, act, Ho, Wo)
    for i in (windows if windows is not None else range(B)):
        ro, rc = oracle_dw(form, xp[i], H, W, C, k, s, pt, pl, w, b, act, Ho, Wo)
        assert same_bits(out[i], ro), ("window", i)
        assert same_bits(cs[i], rc), ("chsum window", i)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("k,s", [(3, 1), (3, 2), (5, 1), (5, 2)])
def test_dwk_block_shape(hip, dtype, k, s):
    """C = 672, 24 x 64, SiLU: the shape of the batched depthwise benchmark."""
    H, W, C = 24, 64, 672
    _, pt = same_pads(H, k, s)
    _, pl = same_pads(W, k, s)
    check_case(hip, "dwk", dtype, 3, H, W, C, k, s, pt, pl, 1, seed=k * 10 + s, windows=[0, 2])


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("Wd", [16, 17, 18, 19, 5, 2, 1])
def test_dwk_row_tails(hip, dtype, Wd):
    """Every Wo % 4, fp16 pair / single tails, rows shorter than a group."""
    for k, s in ((3, 1), (5, 2), (7, 1)):
        _, pt = same_pads(6, k, s)
        _, pl = same_pads(Wd, k, s)
        for act in (0, 1):
            check_case(hip, "dwk", dtype, 2, 6, Wd, 40, k, s, pt, pl, act, seed=Wd * 7 + k + act)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_dwk_k7_and_odd_channels(hip, dtype):
    # C = 22: the fp16 channel-pair kernel (C % 4 == 2); 72: channel quads; 3, 5: single channels
    for (H, W, C, k, s, seed) in ((9, 13, 72, 7, 2, 3), (7, 11, 3, 5, 1, 4), (10, 9, 5, 7, 1, 5),
                                  (8, 10, 22, 3, 1, 6), (6, 9, 22, 5, 2, 7)):
        _, pt = same_pads(H, k, s)
        _, pl = same_pads(W, k, s)
        check_case(hip, "dwk", dtype, 2, H, W, C, k, s, pt, pl, 1, seed=seed)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("s", [1, 2])
def test_dw3(hip, dtype, s):
    # 249 x 63 x 40: the Perch-shaped net's first block; C = 5: odd channel counts (single channels); heights 24, 5,
    # 6, 7: every band tail of the 4-row fp32 stride-1 kernel
    for H, W, C in ((24, 64, 144), (5, 7, 24), (6, 2, 8), (7, 9, 18), (249, 63, 40), (4, 6, 5)):
        _, pt = same_pads(H, 3, s)
        _, pl = same_pads(W, 3, s)
        check_case(hip, "dw3", dtype, 2, H, W, C, 3, s, pt, pl, 1, seed=H + W + s)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("form", ["dwk", "dw3"])
def test_dw_specials(hip, dtype, form):
    """Infinities, NaNs and overflowing fp16 values flow through as on the CPU."""
    check_case(hip, form, dtype, 2, 8, 12, 64, 3, 1, 1, 1, 1, seed=11, specials=True)


def test_dwk_without_chsum_and_bad_params(hip):
    rng = np.random.default_rng(5)
    H, W, C, k = 6, 8, 16, 3
    xp = haloed(rng, 1, H, W, C, 1, np.float32)
    w, b = weights(rng, k, C, np.float32)
    out, _ = run_dw(hip, "dwk", xp, H, W, C, k, 1, 1, 1, w, b, 1, H, W, chsum=False)
    ro, _ = O.dwk_f32(xp[0], H, W, C, k, 1, 1, 1, w, b, 1, H, W)
    assert same_bits(out[0], ro)
    L = hip.lib()
    d = hip.DeviceArray.zeros(4096, np.float32)
    # k = 4, a pad beyond the halo, an output reading past the halo: refused before any launch
    assert L.bnh_dwk_f32(d.ptr, 0, H, W, C, 4, 1, 1, 1, d.ptr, d.ptr, 1, d.ptr, 0, H, W, None, 0, 1, None) != 0
    assert L.bnh_dwk_f32(d.ptr, 0, H, W, C, 3, 1, 2, 1, d.ptr, d.ptr, 1, d.ptr, 0, H, W, None, 0, 1, None) != 0
    assert L.bnh_dwk_f32(d.ptr, 0, H, W, C, 3, 1, 1, 1, d.ptr, d.ptr, 1, d.ptr, 0, H + 1, W, None, 0, 1, None) != 0
    assert b"parameter check" in L.bnh_last_error()


@pytest.mark.parametrize("k,s", [(3, 1), (3, 2), (5, 1), (5, 2), (7, 2)])
def test_dw_s8(hip, k, s):
    rng = np.random.default_rng(k * 3 + s)
    B, H, W, C = 3, 24, 64, 672
    Ho, pt = same_pads(H, k, s)
    Wo, pl = same_pads(W, k, s)
    x = rng.integers(-128, 128, (B, H, W, C)).astype(np.int8)
    w = rng.integers(-127, 128, (k * k, C)).astype(np.int8)
    bias = rng.integers(-20000, 20000, C).astype(np.int32)
    mult = rng.integers(2 ** 30, 2 ** 31 - 1, C).astype(np.int32)
    shift = rng.integers(5, 11, C).astype(np.int32)
    lut = rng.integers(-128, 128, 256).astype(np.int8)
    zx, zy = -5, 3
    say("dw_s8 k", k, "s", s)
    H_ = hip
    xs, x_ws = with_slack(x, 64)
    o_ws = Ho * Wo * C + 128
    dx = H_.DeviceArray.from_host(xs)
    dwt, dbias = H_.DeviceArray.from_host(w), H_.DeviceArray.from_host(bias)
    dm, dsh, dl = H_.DeviceArray.from_host(mult), H_.DeviceArray.from_host(shift), H_.DeviceArray.from_host(lut)
    for use_lut in (False, True):
        do = H_.DeviceArray.zeros((B, o_ws), np.int8)
        H_.check(H_.lib().bnh_dw_s8(dx.ptr, x_ws, H, W, C, k, s, pt, pl, dwt.ptr, dbias.ptr, dm.ptr, dsh.ptr, zx, zy,
                                    -100, 120, dl.ptr if use_lut else None, do.ptr, o_ws, Ho, Wo, B, None), "dw_s8")
        H_.sync()
        out = do.numpy()[:, :Ho * Wo * C].reshape(B, Ho, Wo, C)
        for i in (0, B - 1):
            ref = O.dw_s8(x[i], k, s, pt, pl, w, bias, mult, shift, zx, zy, -100, 120, lut if use_lut else None,
                          Ho, Wo)
            assert np.array_equal(out[i], ref), ("window", i, "lut", use_lut)

@pytest.mark.gpu
@pytest.mark.parametrize("k,s", [(3, 1), (5, 1), (5, 2)])
def test_dw_s8_short_requant(hip, k, s):
    """Output zero points at or below the clamp's low end (zy <= lo, config 1: zy = lo = -128) with every shift in
    1..31 take the kernel's short requantisation (no sign test, the zero point outside the clamp): shifts 1 and 31,
    negative and extreme multipliers, zy = lo, zy < lo, with and without the SiLU table; then biases past the no-wrap
    bound on some channels, which must take the general form."""
    rng = np.random.default_rng(50 + k * 3 + s)
    B, H, W, C = 2, 24, 64, 672
    Ho, pt = same_pads(H, k, s)
    Wo, pl = same_pads(W, k, s)
    x = rng.integers(-128, 128, (B, H, W, C)).astype(np.int8)
    w = rng.integers(-128, 128, (k * k, C)).astype(np.int8)
    mult = rng.integers(-2 ** 31, 2 ** 31, C, dtype=np.int64)
    mult[:6] = [2 ** 31 - 1, -2 ** 31, 0, 1, -1, 2 ** 30]
    mult = mult.astype(np.int32)
    shift = rng.integers(1, 32, C).astype(np.int32)
    shift[:4] = [1, 31, 1, 31]
    lut = rng.integers(-128, 128, 256).astype(np.int8)
    H_ = hip
    dx = H_.DeviceArray.from_host(x)
    dwt = H_.DeviceArray.from_host(w)
    dm, dsh, dl = H_.DeviceArray.from_host(mult), H_.DeviceArray.from_host(shift), H_.DeviceArray.from_host(lut)
    x_ws, o_ws = H * W * C, Ho * Wo * C
    for (zx, zy, lo, hi) in ((-128, -128, -128, 127), (7, -20, -10, 100)):
        wsum = w.astype(np.int64).sum(0)
        room = 2 ** 31 - 1 - k * k * 16384
        for over in (False, True):
            a0 = rng.integers(-room + 1, room, C).astype(np.int64)
            if over:
                a0[5::97] = room + 1 + rng.integers(0, 1000, a0[5::97].size)
            bias = a0 + zx * wsum
            bias = ((bias + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int32)
            dbias = H_.DeviceArray.from_host(bias)
            for use_lut in (False, True):
                say("dw_s8 short requant k", k, "s", s, "zy", zy, "lo", lo, "over", over, "lut", use_lut)
                do = H_.DeviceArray.zeros((B, o_ws), np.int8)
                H_.check(H_.lib().bnh_dw_s8(dx.ptr, x_ws, H, W, C, k, s, pt, pl, dwt.ptr, dbias.ptr, dm.ptr, dsh.ptr,
                                            zx, zy, lo, hi, dl.ptr if use_lut else None, do.ptr, o_ws, Ho, Wo, B,
                                            None), "dw_s8")
                H_.sync()
                out = do.numpy().reshape(B, Ho, Wo, C)
                for i in range(B):
                    ref = O.dw_s8(x[i], k, s, pt, pl, w, bias, mult, shift, zx, zy, lo, hi,
                                  lut if use_lut else None, Ho, Wo)
                    assert np.array_equal(out[i], ref), ("window", i, "zy", zy, "over", over, "lut", use_lut,
                                                         np.argwhere(out[i] != ref)[:4])


@pytest.mark.parametrize("k", [3, 5])
def test_dw_s8_tiled_ragged(hip, k):
    """The stride-1 tiled int8 kernel on shapes that leave partial tiles: channel counts that are not a multiple of
    32 (the last channel group partly empty), widths past one 64-column tile and not a multiple of it, heights that
    are not a multiple of the 8-row tile, every top / left padding, outputs smaller than the input (valid-style) and
    larger (reading past the bottom and right edges, which hold the zero point); the strip kernel's results are the
    same bytes (BNH_DW_S8=strip is read once per process, so the oracle is the check here)"""
    rng = np.random.default_rng(70 + k)
    for H, W, C, pt, pl, Ho, Wo in ((5, 7, 36, 0, k - 1, 5, 7), (13, 70, 100, k // 2, 1, 13, 70),
                                    (9, 130, 44, k - 1, 0, 7, 126), (3, 64, 8, 1, k // 2, 6, 66),
                                    (17, 1, 4, k // 2, k // 2, 17, 1)):
        B = 2
        x = rng.integers(-128, 128, (B, H, W, C)).astype(np.int8)
        w = rng.integers(-128, 128, (k * k, C)).astype(np.int8)
        bias = rng.integers(-20000, 20000, C).astype(np.int32)
        mult = rng.integers(2 ** 30, 2 ** 31 - 1, C).astype(np.int32)
        shift = rng.integers(1, 12, C).astype(np.int32)
        lut = rng.integers(-128, 128, 256).astype(np.int8)
        xs, x_ws = with_slack(x, 64)
        o_ws = Ho * Wo * C + 64
        dx, dwt = hip.DeviceArray.from_host(xs), hip.DeviceArray.from_host(w)
        dbias, dm = hip.DeviceArray.from_host(bias), hip.DeviceArray.from_host(mult)
        dsh, dl = hip.DeviceArray.from_host(shift), hip.DeviceArray.from_host(lut)
        for zx, zy, lo, hi, use_lut in ((-128, -128, -128, 127, True), (9, 4, -90, 110, False)):
            say("dw_s8 tiled k", k, "shape", H, W, C, "pads", pt, pl, "out", Ho, Wo, "lut", use_lut)
            do = hip.DeviceArray.zeros((B, o_ws), np.int8)
            hip.check(hip.lib().bnh_dw_s8(dx.ptr, x_ws, H, W, C, k, 1, pt, pl, dwt.ptr, dbias.ptr, dm.ptr, dsh.ptr,
                                          zx, zy, lo, hi, dl.ptr if use_lut else None, do.ptr, o_ws, Ho, Wo, B,
                                          None), "dw_s8")
            hip.sync()
            raw = do.numpy()
            assert not raw[:, Ho * Wo * C:].any(), "wrote past the window's outputs"
            out = raw[:, :Ho * Wo * C].reshape(B, Ho, Wo, C)
            for i in range(B):
                ref = O.dw_s8(x[i], k, 1, pt, pl, w, bias, mult, shift, zx, zy, lo, hi, lut if use_lut else None,
                              Ho, Wo)
                assert np.array_equal(out[i], ref), ("window", i, np.argwhere(out[i] != ref)[:4])
