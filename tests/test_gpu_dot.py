"""GPU parity of the dotprod + fp16 family's registry ops (variant 2, src/rt_ops_dot.c) run as packages through
bnn_infer_batch, against the op-by-op oracle interpreter:
  * WINO_S8 -> PAD (fp16) -> UNPAD: the int8 Winograd's fp16 output, haloed and widened back, bit for bit;
  * STEM3 -> CONV3C24 -> UNPAD: the stem bit for bit, then the fp16 Winograd 24 -> 24 with SiLU and its own input
    as residual, within the fp16 Winograd bound of the CONV3C24 kernel tests (the GPU sums in fp32 on the matrix
    cores, the reference in fp16); and the STEM3 kernel alone against the oracle;
  * the op contracts: a CONV3C24 record with a wrong channel stride is refused with the reference's message."""
import numpy as np
import pytest

import pyoracle as O
from oracle_net import OracleNet
from bnneon import binding, netbuild, pkgfmt

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn])


def wino_net(rng, H, W, C, K):
    """rows [H][W][C] -> WINO_S8 (K channels) -> PAD (fp16) -> UNPAD."""
    pkg = pkgfmt.Package()
    net = netbuild.Net(pkg)
    ib = net.buf(netbuild.F32, H, W, C)
    w8 = (rng.standard_normal((K, 3, 3, C)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b8 = (rng.standard_normal(K) * 0.1).astype(np.float32)
    out = net.unpad(net.pad(net.wino_s8(ib, w8, b8), 1))
    net.add_to("neon-fp16", netbuild.HW_FP16 | netbuild.HW_DOTPROD, in_buf=ib, out_buf=out)
    netbuild.standard_meta(pkg, H * W * C, H * W * K, model_id="synthetic_dot")
    return pkg, net, ib, out


def stem_net(rng, H, W):
    """image [H][W][3] -> STEM3 -> CONV3C24 -> UNPAD (the stage-0 plan of the dense-conv models)."""
    pkg = pkgfmt.Package()
    net = netbuild.Net(pkg)
    ib = net.buf(netbuild.F32, H, W, 3)
    ws = (rng.standard_normal((24, 3, 3, 3)) * 0.5).astype(np.float32)
    bs = (rng.standard_normal(24) * 0.1).astype(np.float32)
    s0 = net.stem3(ib, ws, bs)
    wc = (rng.standard_normal((24, 3, 3, 24)) * np.sqrt(2.0 / (9 * 24))).astype(np.float32)
    bc = (rng.standard_normal(24) * 0.1).astype(np.float32)
    out = net.unpad(net.conv3c24(s0, wc, bc))
    net.add_to("neon-fp16", netbuild.HW_FP16 | netbuild.HW_DOTPROD, in_buf=ib, out_buf=out)
    netbuild.standard_meta(pkg, H * W * 3, (H // 2) * (W // 2) * 24, model_id="synthetic_stem")
    return pkg, net, ib, out, s0, wc, bc


@pytest.mark.parametrize("H,W,n", [(12, 20, 4), (7, 9, 4), (6, 8, 70)])
def test_wino_s8_pad_unpad_package(hip, tmp_path, H, W, n):
    """(70 windows: the batch runs as two concurrent sub-batches, each on its own slots of the op's scratch)"""
    rng = np.random.default_rng(H * W)
    C, K = 16, 32
    pkg, net, ib, out = wino_net(rng, H, W, C, K)
    path = str(tmp_path / "dot.bnpk")
    pkg.write(path)
    pcm = rng.standard_normal((n, H * W * C)).astype(np.float32)
    say("dot package wino_s8", H, W)
    with binding.Model(path) as m:
        got, _, status = m.infer_batch(pcm)
        assert not status.any()
    orc = OracleNet(net, ib, out)
    for i in sorted({0, 1, n // 2 - 1, n // 2, n - 1}):
        ro, _, _ = orc.run(pcm[i])
        assert same(got[i], ro[:H * W * K]), i


@pytest.mark.parametrize("H,W", [(8, 12), (20, 34), (4, 4)])
def test_stem3_kernel(hip, H, W):
    """bnh_stem3_f16 against the oracle, bit for bit (bottom / right edges, several windows, padded strides)."""
    rng = np.random.default_rng(H + W)
    B, Ho, Wo = 3, (H + 1) // 2, (W + 1) // 2
    img = rng.standard_normal((B, H, W, 3)).astype(np.float32)
    img[0, 0, 0, 0], img[0, -1, -1, 2] = np.inf, np.nan
    w = (rng.standard_normal((24, 3, 3, 3)) * 0.5).astype(np.float32)
    b = (rng.standard_normal(24) * 0.1).astype(np.float32)
    H_ = hip
    i_ws, o_ws = H * W * 3 + 12, (Ho + 2) * (Wo + 2) * 24 + 8
    xs = np.zeros((B, i_ws), np.float32)
    xs[:, :H * W * 3] = img.reshape(B, -1)
    dx, dw_, db = H_.DeviceArray.from_host(xs), H_.DeviceArray.from_host(w), H_.DeviceArray.from_host(b)
    do = H_.DeviceArray.zeros((B, o_ws), np.float16)
    H_.check(H_.lib().bnh_stem3_f16(dx.ptr, i_ws, H, W, dw_.ptr, db.ptr, do.ptr, o_ws, B, None), "stem3")
    H_.sync()
    got = do.numpy()[:, :(Ho + 2) * (Wo + 2) * 24].reshape(B, Ho + 2, Wo + 2, 24)
    for i in range(B):
        ref = O.stem3(img[i], w, b)
        gn, rn = np.isnan(got[i]), np.isnan(ref)
        assert np.array_equal(gn, rn), i   # NaN where the oracle has NaN (any NaN equal to any NaN)
        assert np.array_equal(got[i].view(np.uint16)[~gn], ref.view(np.uint16)[~rn]), i


def test_stem3_conv3c24_package(hip, tmp_path):
    """STEM3 bit for bit (as the CONV3C24 input the oracle interpreter holds), then CONV3C24 within the fp16
    Winograd bound of the kernel tests, through bnn_infer_batch."""
    from test_gpu_wino import bound, direct, silu
    rng = np.random.default_rng(3)
    H, W, n = 32, 48, 3
    pkg, net, ib, out, s0, wc, bc = stem_net(rng, H, W)
    path = str(tmp_path / "c24.bnpk")
    pkg.write(path)
    pcm = rng.standard_normal((n, H * W * 3)).astype(np.float32)
    say("dot package stem3 + conv3c24")
    with binding.Model(path) as m:
        got, _, status = m.infer_batch(pcm)
        assert not status.any()
    orc = OracleNet(net, ib, out)
    Hs, Ws = H // 2, W // 2
    u = 2.0 ** -11
    for i in range(n):
        ro, _, bufs = orc.run(pcm[i])
        xp = bufs[s0][:(Hs + 2) * (Ws + 2) * 24].reshape(Hs + 2, Ws + 2, 24)  # the conv's input (STEM3, exact)
        y = direct(xp.astype(np.float64), wc, bc).reshape(Hs, Ws, 24)
        t = silu(y) + xp[1:-1, 1:-1].astype(np.float64)
        E = bound(xp, wc)
        tg = 1.1 * (4 * u * E + u * np.abs(y)) + 2 * u * np.abs(t) + 2.0 ** -20 * np.abs(y) + 2.0 ** -24
        to = 1.1 * 40 * u * E + 2e-3 * np.maximum(1.0, np.abs(silu(y))) + 2 * u * np.abs(t)
        g = got[i].reshape(Hs, Ws, 24).astype(np.float64)
        o = ro[:Hs * Ws * 24].reshape(Hs, Ws, 24).astype(np.float64)
        assert (np.abs(g - t) <= tg).all(), float(np.max(np.abs(g - t) / tg))
        assert (np.abs(g - o) <= tg + to).all()


def test_conv3c24_contract(hip, tmp_path):
    """A CONV3C24 record on a 32-channel buffer is refused at bnn_init with the reference's buffer message."""
    rng = np.random.default_rng(4)
    H, W, C = 8, 8, 16
    pkg = pkgfmt.Package()
    net = netbuild.Net(pkg)
    ib = net.buf(netbuild.F32, H, W, C)
    h = net.wino_s8(ib, rng.standard_normal((32, 3, 3, C)).astype(np.float32), np.zeros(32, np.float32))
    hp = net.pad(h, 1)   # 32 channels at stride 32: CONV3C24 needs 24
    ob = net.buf(netbuild.F16, H, W, 24, halo=1)
    tl = [net.tensor("w", rng.standard_normal((24, 3, 3, 24)).astype(np.float32)),
          net.tensor("b", np.zeros(24, np.float32))]
    net.emit(netbuild.OP["CONV3C24"], [hp, ob], tl, [H, W], var=2)
    out = net.unpad(ob)
    net.add_to("neon-fp16", netbuild.HW_FP16 | netbuild.HW_DOTPROD, in_buf=ib, out_buf=out)
    netbuild.standard_meta(pkg, H * W * C, H * W * 24, model_id="synthetic_dot_bad")
    path = str(tmp_path / "bad.bnpk")
    pkg.write(path)
    with pytest.raises(binding.BnnError) as ei:
        binding.Model(path)
    msg = str(ei.value)
    assert "conv3c24_wino16" in msg and "expected halo 1 and channel stride 24" in msg, msg
