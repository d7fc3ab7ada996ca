"""The int8 1x1 expansion fused into the fp32 depthwise conv (bnh_pwdw_f32)
against the two launches it replaces: bnh_pw_s8 into a zero-haloed buffer, then
bnh_dw3_f32 / bnh_dwk_f32 over it (each pinned to the oracle by test_gpu_s8n.py
and test_gpu_dw.py). Outputs and per-channel sums are bit-identical (any NaN
equal to any NaN), and bytes past each window's outputs stay untouched.

Cases: the Perch-shaped block geometries (249 x 63 stride 2 in many bands,
125 x 32, 63 x 16 with k 5, 32 x 8, 16 x 4), every expansion activation and
both depthwise activations, K > 64 (several MFMA K steps), channel counts that
are not a multiple of 32 (16-channel groups), row tails (Wo % 4 = 1..3), 'same'
pads 0 / 1 / 2, padded window strides, and rows holding an infinity or a NaN.
"""
import numpy as np
import pytest

from bnneon import s8pack

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn]))


def same_pads(n, k, s):
    o = (n - 1) // s + 1
    return o, max((o - 1) * s + k - n, 0) // 2


def pwdw_case(H, B, Hh, Ww, K, C, k, s, form, pact, dact, seed, slack=0, specials=False):
    rng = np.random.default_rng(seed)
    M = Hh * Ww
    w = (rng.standard_normal((C, K)) * np.sqrt(2.0 / K)).astype(np.float32)
    b = (rng.standard_normal(C) * 0.1).astype(np.float32)
    pk = s8pack.pack_s8(w, b)
    N_, K_, Kp, Np = pk["shape"]
    assert Np == C
    x = rng.standard_normal((B, M, K)).astype(np.float32)
    if specials:
        x[0, 5, 3] = np.inf
        x[B - 1, M // 2, 1] = np.nan
    h = (k - 1) // 2
    Ho, pt = same_pads(Hh, k, s)
    Wo, pl = same_pads(Ww, k, s)
    if form == 2:
        assert pt == 1 and pl == 1
    M4 = (M + 3) // 4 * 4
    Wt = H.S8Weights(N_, K_, Kp, Np, pk["q"], pk["sw"], pk["cs"], pk["b"])
    dx = H.DeviceArray.from_host(x)
    dq = H.DeviceArray.zeros((B, M4 * Kp), np.int8)
    dsa = H.DeviceArray.zeros((B, M4), np.float32)
    dza = H.DeviceArray.zeros((B, M4), np.int32)
    per = (Hh + 2 * h) * (Ww + 2 * h) * C
    dmid = H.DeviceArray.from_host(np.full((B, per), 7.0, np.float32))
    e = H.epi32(dmid, C, act=pact, ow=Ww, opad=h, out_ws=per)
    wdw = (rng.standard_normal((k * k, C)) * np.sqrt(2.0 / (k * k))).astype(np.float32)
    bdw = (rng.standard_normal(C) * 0.1).astype(np.float32)
    dwd, dbd = H.DeviceArray.from_host(wdw), H.DeviceArray.from_host(bdw)
    o_ws = Ho * Wo * C + slack
    d1 = H.DeviceArray.from_host(np.full((B, o_ws), 5.0, np.float32))
    d2 = H.DeviceArray.from_host(np.full((B, o_ws), 5.0, np.float32))
    c1 = H.DeviceArray.zeros((B, C), np.float32)
    c2 = H.DeviceArray.zeros((B, C), np.float32)
    say(f"pwdw B{B} {Hh}x{Ww} K{K} C{C} k{k} s{s} form{form} pads {pt},{pl} act {pact}/{dact}")
    L = H.lib()
    H.check(L.bnh_pw_s8(dx.ptr, M * K, K, M, None, 0, dq.ptr, M4 * Kp, dsa.ptr, M4, dza.ptr, M4, B, Wt.h, e, None),
            "pw_s8")
    if form == 2:
        H.check(L.bnh_dw3_f32(dmid.ptr, per, Hh, Ww, C, s, dwd.ptr, dbd.ptr, d1.ptr, o_ws, Ho, Wo, c1.ptr, C, B,
                              None), "dw3_f32")
    else:
        H.check(L.bnh_dwk_f32(dmid.ptr, per, Hh, Ww, C, k, s, pt, pl, dwd.ptr, dbd.ptr, dact, d1.ptr, o_ws, Ho, Wo,
                              c1.ptr, C, B, None), "dwk_f32")
    H.check(L.bnh_pwdw_f32(dq.ptr, M4 * Kp, dsa.ptr, M4, dza.ptr, M4, Hh, Ww, Wt.h, pact, k, s, pt, pl, form,
                           dwd.ptr, dbd.ptr, dact, d2.ptr, o_ws, Ho, Wo, c2.ptr, C, B, None), "pwdw_f32")
    H.sync()
    o1, o2 = d1.numpy(), d2.numpy()
    assert np.all(o2[:, Ho * Wo * C:] == 5.0)
    return same_bits(o1, o2) and same_bits(c1.numpy(), c2.numpy())


def test_pwdw_perch_block_geometries(hip):
    # (H, W, K, C, k, s, form): the expansions of Perch-v2's MBConv blocks into their depthwise convs
    for i, (Hh, Ww, K, C, k, s, form) in enumerate((
            (249, 63, 24, 144, 3, 2, 2),      # stride 2 over 32 bands of 4 rows (the last band 1 row)
            (125, 32, 32, 192, 3, 1, 2),
            (125, 32, 32, 192, 5, 2, 0),      # pads 2 / 1
            (63, 16, 48, 288, 5, 1, 0),
            (63, 16, 48, 288, 3, 2, 0),       # pads 1 / 0: DWK, not DW3
            (32, 8, 136, 816, 5, 1, 0),       # K 136 (3 MFMA K steps), 16-channel groups
            (16, 4, 384, 2304, 3, 1, 2),      # K 384
            (16, 4, 232, 1392, 5, 1, 0))):
        assert pwdw_case(hip, 2, Hh, Ww, K, C, k, s, form, 1, 1, seed=i), i


@pytest.mark.parametrize("pact,dact", [(0, 0), (2, 1), (1, 0)])
def test_pwdw_activations_tails_pads(hip, pact, dact):
    for i, (Hh, Ww, K, C, k, s, form) in enumerate((
            (11, 9, 40, 48, 3, 1, 2),         # Wo % 4 = 1
            (10, 10, 24, 32, 5, 1, 0),        # Wo % 4 = 2
            (9, 11, 16, 16, 5, 2, 0),         # Wo % 4 = 2, pads 2
            (7, 15, 72, 80, 3, 2, 2),         # Wo % 4 = 0, K 72
            (6, 7, 8, 64, 3, 1, 0))):         # Wo % 4 = 3, K 8, DWK with k 3
        assert pwdw_case(hip, 3, Hh, Ww, K, C, k, s, form, pact, dact, seed=10 * i + pact, slack=40), i


def test_pwdw_nonfinite_rows_and_strides(hip):
    assert pwdw_case(hip, 3, 20, 13, 48, 96, 5, 1, 0, 1, 1, seed=77, slack=24, specials=True)
    assert pwdw_case(hip, 2, 21, 17, 32, 64, 3, 2, 2, 1, 1, seed=78, specials=True)
    assert pwdw_case(hip, 1, 1, 1, 16, 16, 3, 1, 2, 1, 1, seed=79)   # a single pixel
