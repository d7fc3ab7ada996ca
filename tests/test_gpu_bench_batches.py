"""GPU parity at the batch sizes bench.py times: 64 windows per launch for the
depthwise (C = 672, 24 x 64) and Winograd (64 -> 64, 96 x 256) kernels, 256
windows for the two nets. The first, a middle and the last window of each batch
are compared with the oracle (bit for bit; the Winograd within its stated
bound), and the nets' 256-window batches with the same windows run as separate
batches of 128 (which the runtime splits over two streams in its own way).
"""
import numpy as np
import pytest

import oracle_net  # oracle/oracle_net.py
import pyoracle as O
from bnneon import binding, perchnet, v24net
from test_gpu_dw import check_case, same_pads, with_slack
from test_gpu_wino import bound, direct, make, run as run_wino

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn])


@pytest.mark.parametrize("k", [3, 5])
def test_dw_f16_batch64(hip, k):
    H, W, C = 24, 64, 672
    _, pt = same_pads(H, k, 1)
    _, pl = same_pads(W, k, 1)
    check_case(hip, "dwk", np.float16, 64, H, W, C, k, 1, pt, pl, 1, seed=640 + k, windows=[0, 31, 63])


def test_dw_s8_batch64(hip):
    rng = np.random.default_rng(645)
    B, H, W, C, k, s = 64, 24, 64, 672, 5, 1
    Ho, pt = same_pads(H, k, s)
    Wo, pl = same_pads(W, k, s)
    x = np.clip(np.round(rng.normal(-40, 35, (B, H, W, C))), -128, 127).astype(np.int8)
    w = rng.integers(-127, 128, (k * k, C)).astype(np.int8)
    bias = rng.integers(-2 ** 14, 2 ** 14 + 1, C).astype(np.int32)
    mult = rng.integers(2 ** 30, 2 ** 31, C).astype(np.int32)
    shift = rng.integers(6, 11, C).astype(np.int32)
    lut = rng.integers(-128, 128, 256).astype(np.int8)
    xs, x_ws = with_slack(x, 0)
    o_ws = Ho * Wo * C
    dx = hip.DeviceArray.from_host(xs)
    dwt, dbias = hip.DeviceArray.from_host(w), hip.DeviceArray.from_host(bias)
    dm, dsh, dl = hip.DeviceArray.from_host(mult), hip.DeviceArray.from_host(shift), hip.DeviceArray.from_host(lut)
    do = hip.DeviceArray.zeros((B, o_ws), np.int8)
    say("dw_s8 5x5 s1 B", B)
    hip.check(hip.lib().bnh_dw_s8(dx.ptr, x_ws, H, W, C, k, s, pt, pl, dwt.ptr, dbias.ptr, dm.ptr, dsh.ptr, -128, -128,
                                  -128, 127, dl.ptr, do.ptr, o_ws, Ho, Wo, B, None), "dw_s8")
    hip.sync()
    out = do.numpy().reshape(B, Ho, Wo, C)
    for i in (0, 31, 63):
        ref = O.dw_s8(x[i], k, s, pt, pl, w, bias, mult, shift, -128, -128, -128, 127, lut, Ho, Wo)
        assert np.array_equal(out[i], ref), ("window", i)


def test_wino_f16_batch64(hip):
    rng = np.random.default_rng(646)
    B, H, W, C, K = 64, 96, 256, 64, 64
    xp, w, b = make(rng, B, H, W, C, K)
    say("wino config2 B", B)
    out = run_wino(hip, xp, w, b).astype(np.float64)
    u = 2.0 ** -11
    for i in (0, 63):
        ref = direct(xp[i].astype(np.float64), w, b).reshape(H, W, K)
        err = np.abs(out[i] - ref)
        tol = 4 * u * bound(xp[i, 88:98], w) + u * np.abs(ref[88:96]) + 2.0 ** -24  # the last band of rows
        assert (err[88:96] <= tol).all(), i
        assert err.max() <= 8 * u * np.abs(ref).max(), i


def net_batch256(path, net, emb_buf, signal, n_classes, emb_dim, seed):
    rng = np.random.default_rng(seed)
    pcm = np.stack([signal(rng) for _ in range(256)])
    on = oracle_net.OracleNet(net, 0, net.last, emb_buf)
    with binding.Model(path) as m:
        out, emb, status = m.infer_batch(pcm)
        assert not status.any()
        for w in (0, 255):
            ref, ref_emb, _ = on.run(pcm[w])
            say("window", w)
            assert same(out[w], ref[:n_classes]), w
            assert same(emb[w], ref_emb[:emb_dim]), w
        for lo in (0, 128):
            o, e, s = m.infer_batch(pcm[lo:lo + 128])
            assert not s.any() and same(o, out[lo:lo + 128]) and same(e, emb[lo:lo + 128]), lo


def test_perch_batch256(hip, tmp_path):
    pn = perchnet.PerchNet(seed=3)
    path = pn.write(str(tmp_path / "perch_s8.bnpk"))
    say("perch B 256")
    net_batch256(path, pn.net, pn.emb_buf, perchnet.signal, perchnet.N_CLASSES, perchnet.EMB, 647)


def test_v24_batch256(hip, tmp_path):
    vn = v24net.V24Net(seed=5)
    path = vn.write(str(tmp_path / "v24_f16.bnpk"))
    say("v24 B 256")
    net_batch256(path, vn.net, vn.emb_buf, v24net.signal, v24net.N_CLASSES, v24net.EMB, 648)
