"""GPU parity of the dotprod family's int8 kernels (src/gemm_s8.c, src/rt_ops_dot.c:173-585) against the oracle
(oracle/qdot.c), bit for bit unless stated: per-row quantisation of fp32 rows and of (gated) fp16 rows with every
tail form (K % 4, K % 8, K % 16), the int8 GEMM's fp32 FMA epilogue in all its output forms (fp16 + table SiLU with
and without a zero halo, fp32 + silu_f32_a / ReLU / residual), partial K steps and channel groups, the 3 x 3
implicit-im2col conv at both strides and odd sizes, the SED heads, the fp16-weight SE gate, the generalised mean
(within one unit in the last place of the C library's powf, which it does not restate) and the scalar functions.
Inputs are finite (NaN inputs are outside what these kernels are compared on)."""
import ctypes as ct

import numpy as np
import pytest

import pyoracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float16:
        a, b = a.astype(np.float32), np.asarray(b, np.float16).astype(np.float32)
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn])


def windows(a, slack):
    """[B][...] -> [B][size + slack] zero-padded window slots."""
    B = a.shape[0]
    flat = a.reshape(B, -1)
    out = np.zeros((B, flat.shape[1] + slack), a.dtype)
    out[:, :flat.shape[1]] = flat
    return out


class QdW:
    def __init__(self, H, w, b, Np=None):
        w = np.ascontiguousarray(w, np.float32)
        b = None if b is None else np.ascontiguousarray(b, np.float32)
        self.N, self.K = w.shape
        self.Np = Np or self.N
        self.Kp = (self.K + 15) // 16 * 16
        self.h = H.lib().bnh_qdw_new(w.ctypes.data, None if b is None else b.ctypes.data, self.N, self.K, self.Np)
        self.H = H
        if not self.h:
            H.check(None, "bnh_qdw_new")

    def __del__(self):
        if getattr(self, "h", None):
            self.H.lib().bnh_qdw_free(self.h)


def rand_rows(rng, B, M, K, kind):
    x = rng.standard_normal((B, M, K)).astype(np.float32)
    if kind == 1:
        x = np.abs(x)            # all positive: zp = -128 side
    elif kind == 2:
        x = -np.abs(x) * 30      # all negative, large
    x[:, 0, :] = 0.0             # an all-zero row (scale 1, zp 128)
    if M > 1:
        x[:, 1, :] = 0.75        # a constant row
    return x


@pytest.mark.parametrize("K", [8, 20, 23, 40, 136, 1152])
@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("pad", [5, 8])
def test_quant_rows_f32(hip, K, kind, pad):
    """pad 8 with K % 8 == 0: the multi-row vector kernel; pad 5 or K % 8 != 0: one wavefront per row"""
    rng = np.random.default_rng(K * 3 + kind)
    B, M, ldx = 3, 37, K + pad
    x = np.zeros((B, M, ldx), np.float32)
    x[:, :, :K] = rand_rows(rng, B, M, K, kind)
    Kp = (K + 15) // 16 * 16
    say("quant_rows_f32", K, kind)
    dx = hip.DeviceArray.from_host(windows(x, 12))
    a_ws, rq_ws = M * Kp + 48, 2 * M + 6
    da = hip.DeviceArray.from_host(np.full((B, a_ws), 99, np.int8))
    dr = hip.DeviceArray.zeros((B, rq_ws), np.float32)
    hip.check(hip.lib().bnh_qd_quant_rows(dx.ptr, 0, M * ldx + 12, ldx, M, K, None, 0, da.ptr, a_ws, dr.ptr, rq_ws, B,
                                          None), "quant")
    hip.sync()
    a, rq = da.numpy(), dr.numpy()
    for i in range(B):
        ra, rr = O.qd_quant_rows(x[i], K)
        assert np.array_equal(a[i, :M * Kp].reshape(M, Kp), ra), i
        assert same(rq[i, :2 * M].reshape(M, 2), rr), i
        assert (a[i, M * Kp:] == 99).all()


@pytest.mark.parametrize("K", [8, 24, 40, 136, 1152])
@pytest.mark.parametrize("gated", [False, True])
def test_quant_rows_f16(hip, K, gated):
    rng = np.random.default_rng(K + 7 * gated)
    B, M, ldx = 2, 29, K + 8
    x = np.zeros((B, M, ldx), np.float16)
    x[:, :, :K] = (rng.standard_normal((B, M, K)) * 3).astype(np.float16)
    x[:, 0, :] = 0
    x[:, 1, :] = np.float16(0.75)  # a constant row
    g = rng.uniform(0, 1, (B, K)).astype(np.float16) if gated else None
    Kp = (K + 15) // 16 * 16
    say("quant_rows_f16", K, gated)
    dx = hip.DeviceArray.from_host(windows(x, 16))
    dg = hip.DeviceArray.from_host(windows(g, 8)) if gated else None
    a_ws, rq_ws = M * Kp + 16, 2 * M
    da = hip.DeviceArray.zeros((B, a_ws), np.int8)
    dr = hip.DeviceArray.zeros((B, rq_ws), np.float32)
    hip.check(hip.lib().bnh_qd_quant_rows(dx.ptr, 1, M * ldx + 16, ldx, M, K, dg.ptr if gated else None,
                                          K + 8 if gated else 0, da.ptr, a_ws, dr.ptr, rq_ws, B, None), "quant16")
    hip.sync()
    a, rq = da.numpy(), dr.numpy()
    for i in range(B):
        ra, rr = O.qd_quant_rows(x[i], K, None if g is None else g[i])
        assert np.array_equal(a[i, :M * Kp].reshape(M, Kp), ra), i
        assert same(rq[i].reshape(M, 2), rr), i


def run_gemm(hip, a, rq, W, act, out16, M, opad=0, ow=0, res=None, per_tensor=False):
    """a [B][M][Kp] int8, rq [B][M][2] -> the GPU epilogue's output windows."""
    B = a.shape[0]
    ldo = W.Np + (0 if opad else 8)
    rows = M if not opad else (M // ow + 2) * (ow + 2)
    o_ws = rows * ldo + 16
    da = hip.DeviceArray.from_host(windows(a, 32))
    dr = hip.DeviceArray.from_host(windows(rq, 4))
    dt = np.float16 if out16 else np.float32
    do = hip.DeviceArray.from_host(np.full((B, o_ws), 3, dt))
    dres, r_ws = None, 0
    if res is not None:
        r_ws = M * ldo + 8
        rr = np.zeros((B, r_ws), np.float32)
        rr[:, :M * ldo] = res.reshape(B, -1)
        dres = hip.DeviceArray.from_host(rr)
    e = hip.QdEpi(act, int(out16), do.ptr, o_ws, ldo, ow, opad, dres.ptr if dres else None, r_ws)
    hip.check(hip.lib().bnh_qd_gemm(da.ptr, a[0].size + 32, a.shape[2], dr.ptr, rq[0].size + 4, int(per_tensor), M,
                                    W.h, ct.byref(e), B, None), "qd_gemm")
    hip.sync()
    return do.numpy()[:, :rows * ldo].reshape(B, rows, ldo), ldo


@pytest.mark.parametrize("M,K,N", [(1, 64, 16), (37, 40, 48), (130, 136, 80), (300, 1152, 144), (64, 24, 272)])
@pytest.mark.parametrize("form", ["f32", "f32_silu", "f32_relu_res", "f16", "f16_silu"])
def test_qd_gemm_epilogues(hip, M, K, N, form):
    rng = np.random.default_rng(M * 7 + K + N)
    B = 3
    w = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    w[3] = 0.0  # an all-zero channel: scale 1, swsum 0
    b = (rng.standard_normal(N) * 0.2).astype(np.float32)
    pk = O.qd_wpack(w, b)
    W = QdW(hip, w, b)
    x = rng.standard_normal((B, M, K)).astype(np.float32) * 2
    aq = np.zeros((B, M, W.Kp), np.int8)
    rq = np.zeros((B, M, 2), np.float32)
    for i in range(B):
        aq[i], rq[i] = O.qd_quant_rows(x[i], K)
    out16 = form.startswith("f16")
    act = 1 if "silu" in form else (2 if "relu" in form else 0)
    res = rng.standard_normal((B, M, N + 8)).astype(np.float32) if "res" in form else None
    say("qd_gemm", M, K, N, form)
    got, ldo = run_gemm(hip, aq, rq, W, act, out16, M, res=res)
    for i in range(B):
        ref = O.qd_gemm(aq[i], rq[i], pk, act=act, out16=out16, ldo=ldo, res=None if res is None else res[i])
        assert same(got[i][:, :N], ref[:, :N]), (i, form)


def test_qd_gemm_haloed_fp16_out(hip):
    rng = np.random.default_rng(3)
    B, Hh, Ww, K, N = 2, 6, 10, 48, 32
    M = Hh * Ww
    w = (rng.standard_normal((N, K)) / 7).astype(np.float32)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    pk = O.qd_wpack(w, b)
    W = QdW(hip, w, b)
    aq = np.zeros((B, M, W.Kp), np.int8)
    rq = np.zeros((B, M, 2), np.float32)
    x = rng.standard_normal((B, M, K)).astype(np.float32)
    for i in range(B):
        aq[i], rq[i] = O.qd_quant_rows(x[i], K)
    say("qd_gemm haloed fp16")
    got, ldo = run_gemm(hip, aq, rq, W, 1, True, M, opad=1, ow=Ww)
    for i in range(B):
        ref = O.qd_gemm(aq[i], rq[i], pk, act=1, out16=True, ldo=ldo, ow=Ww, opad=1)
        g = got[i].reshape(Hh + 2, Ww + 2, ldo)[1:-1, 1:-1]
        r = ref.reshape(Hh + 2, Ww + 2, ldo)[1:-1, 1:-1]
        assert same(g, r), i


@pytest.mark.parametrize("H,W,C,K,s", [(8, 12, 16, 32, 2), (7, 9, 8, 16, 2), (10, 6, 24, 48, 1), (5, 5, 40, 16, 1),
                                       (16, 32, 64, 128, 2)])
def test_qconv3(hip, H, W, C, K, s):
    rng = np.random.default_rng(H * W + C + K + s)
    B = 3
    Ho, pt = O.tf_same(H, 3, s)
    Wo, pl = O.tf_same(W, 3, s)
    w = (rng.standard_normal((K, 3, 3, C)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b = (rng.standard_normal(K) * 0.1).astype(np.float32)
    pk = O.qd_wpack(w.reshape(K, 9 * C), b)
    W8 = QdW(hip, w.reshape(K, 9 * C), b)
    x = rng.standard_normal((B, H, W, C)).astype(np.float32)
    x[1] *= 20  # a window with another scale
    ws = hip.lib().bnh_qconv3_work_bytes(H, W, C)
    work = hip.DeviceArray.zeros(ws * B, np.uint8)
    dx = hip.DeviceArray.from_host(windows(x, 4))
    o_ws = Ho * Wo * K + 8
    do = hip.DeviceArray.from_host(np.full((B, o_ws), 5, np.float16))
    say("qconv3", H, W, C, K, s)
    hip.check(hip.lib().bnh_qconv3(dx.ptr, H * W * C + 4, H, W, C, s, pt, pl, Ho, Wo, W8.h, do.ptr, o_ws, B, work.ptr,
                                   ws, None), "qconv3")
    hip.sync()
    got = do.numpy()
    for i in range(B):
        ref = O.qconv3(x[i], pk, s)
        assert same(got[i, :Ho * Wo * K].reshape(Ho * Wo, K), ref), i


@pytest.mark.parametrize("H,W,C,hid,nc", [(4, 6, 16, 16, 5), (3, 8, 32, 48, 40), (6, 2, 64, 32, 17)])
def test_heads_s8(hip, H, W, C, hid, nc):
    rng = np.random.default_rng(H * 100 + W + nc)
    B = 3
    ncp = (nc + 15) // 16 * 16
    shapes = [(nc, C)] + [(hid, C), (nc, hid), (nc, hid)] * 2
    ws_ = [(rng.standard_normal(s) / np.sqrt(s[1])).astype(np.float32) for s in shapes]
    bs_ = [(rng.standard_normal(s[0]) * 0.1).astype(np.float32) for s in shapes]
    packs = [O.qd_wpack(w, b, ncp if i == 0 or i % 3 != 1 else None) for i, (w, b) in enumerate(zip(ws_, bs_))]
    F = rng.standard_normal((B, H * W, C)).astype(np.float32)
    emb = rng.standard_normal((B, C)).astype(np.float32)
    wp = (ct.c_void_p * 7)(*[w.ctypes.data for w in ws_])
    bp = (ct.c_void_p * 7)(*[b.ctypes.data for b in bs_])
    P = hip.lib().bnh_heads8_new(C, hid, nc, wp, bp)
    if not P:
        hip.check(None, "heads8_new")
    L = max(H, W)
    ws = hip.lib().bnh_heads8_work_bytes(H, W, C, hid, nc)
    work = hip.DeviceArray.zeros(ws * B, np.uint8)
    dF = hip.DeviceArray.from_host(windows(F, 4))
    de = hip.DeviceArray.from_host(windows(emb, 4))
    l_ws, a_ws, rq_ws = ncp + 16, (L + 4) * max(C, hid) + 64, 2 * (L + 4)
    dl = hip.DeviceArray.from_host(np.full((B, l_ws), 9, np.float32))
    da = hip.DeviceArray.zeros((B, a_ws), np.int8)
    dr = hip.DeviceArray.zeros((B, rq_ws), np.float32)
    say("heads_s8", H, W, C, hid, nc)
    try:
        hip.check(hip.lib().bnh_heads_s8(dF.ptr, H * W * C + 4, de.ptr, C + 4, H, W, P, dl.ptr, l_ws, da.ptr, a_ws,
                                         dr.ptr, rq_ws, B, work.ptr, ws, None), "heads_s8")
        hip.sync()
    finally:
        hip.lib().bnh_heads8_free(P)
    got = dl.numpy()
    for i in range(B):
        ref = O.heads_s8(F[i], emb[i], H, W, packs)
        assert same(got[i, :ncp], ref), i


@pytest.mark.parametrize("C,rd", [(16, 4), (136, 12), (1280, 80)])
def test_se_gate16(hip, C, rd):
    rng = np.random.default_rng(C + rd)
    B, P_ = 3, 77
    w1 = (rng.standard_normal((rd, C)) / np.sqrt(C)).astype(np.float32)
    b1 = (rng.standard_normal(rd) * 0.1).astype(np.float32)
    w2 = (rng.standard_normal((C, rd)) / np.sqrt(rd)).astype(np.float32)
    b2 = (rng.standard_normal(C) * 0.1).astype(np.float32)
    cs = (rng.standard_normal((B, C)) * 30).astype(np.float32)
    S = hip.lib().bnh_seg16_new(C, rd, w1.ctypes.data, b1.ctypes.data, w2.ctypes.data, b2.ctypes.data)
    if not S:
        hip.check(None, "seg16_new")
    dc = hip.DeviceArray.from_host(windows(cs, 4))
    dg = hip.DeviceArray.zeros((B, C + 8), np.float16)
    say("se_gate16", C, rd)
    try:
        hip.check(hip.lib().bnh_se_gate16(dc.ptr, C + 4, P_, S, dg.ptr, C + 8, B, None), "se_gate16")
        hip.sync()
    finally:
        hip.lib().bnh_seg16_free(S)
    gc, gg = dc.numpy(), dg.numpy()
    for i in range(B):
        rm, rg = O.se_gate16(cs[i], P_, w1, b1, w2, b2)
        assert same(gc[i, :C], rm), i
        assert same(gg[i, :C], rg), i


@pytest.mark.parametrize("M,C,eps,p", [(64, 32, 1e-6, 3.0), (13, 256, 1e-4, 2.5), (300, 1280, 1e-6, 3.0)])
def test_gem_a(hip, M, C, eps, p):
    """bit for bit: the sums in row order and the final power with the C library's powf results"""
    rng = np.random.default_rng(M + C)
    B = 3
    F = np.abs(rng.standard_normal((B, M, C))).astype(np.float32) * 2
    F[:, 0, :5] = -1.0  # below eps: clamped
    dF = hip.DeviceArray.from_host(windows(F, 4))
    de = hip.DeviceArray.zeros((B, C + 4), np.float32)
    say("gem_a", M, C)
    hip.check(hip.lib().bnh_gem_a(dF.ptr, M * C + 4, M, C, eps, p, de.ptr, C + 4, B, None),
              "gem_a")
    hip.sync()
    got = de.numpy()
    for i in range(B):
        assert same(got[i, :C], O.gem_a(F[i], eps, p)), i


@pytest.mark.parametrize("f", [0, 1, 2, 3])
def test_scalar_functions(hip, f):
    rng = np.random.default_rng(f)
    if f == 0:
        x = np.concatenate([rng.uniform(-126, 126, 200000), np.arange(-126, 127)]).astype(np.float32)
    elif f == 2:
        x = np.exp(rng.uniform(-80, 80, 200000)).astype(np.float32)
        x = np.concatenate([x, 2.0 ** np.arange(-120, 120)]).astype(np.float32)
    else:
        x = np.concatenate([rng.uniform(-100, 100, 200000), rng.standard_normal(50000), [0.0, -0.0, 1e-30, -1e30,
                                                                                        1e30]]).astype(np.float32)
    fn = [O.lib().orc_exp2_p5, O.lib().orc_silu_f32_a, O.lib().orc_log2_dot,
          lambda v: _sig(v)][f]
    ref = np.array([fn(float(v)) for v in x], np.float32)
    dx = hip.DeviceArray.from_host(x)
    dy = hip.DeviceArray.zeros(x.size, np.float32)
    hip.check(hip.lib().bnh_eval_qd(f, dx.ptr, dy.ptr, x.size, None), "eval_qd")
    hip.sync()
    assert same(dy.numpy(), ref), f


def _sig(v):
    """the SE gate's sigmoid (src/rt_ops_dot.c:409-416) restated from the oracle's pieces"""
    L = O.lib()
    t = L.orc_fmin(L.orc_fmax(float(np.float32(v) * np.float32(-1.44269504)), -126.0), 126.0)
    d = float(np.float32(L.orc_exp2_p5(t)) + np.float32(1.0))
    r = L.orc_frecpe(d)
    r = float(np.float32(r) * np.float32(L.orc_frecps(d, r)))
    r = float(np.float32(r) * np.float32(L.orc_frecps(d, r)))
    return r


# ------------------------------------------------------------------ the ops in packages
def v3_net(rng, H, W, C0=16, pool="mean"):
    """rows [H][W][C0] -> QCONV3 s2 (32) -> QPW fp16 in, SiLU, zero-haloed fp16 out (64) -> DW3 fp16 (chsum) ->
    SE_GATE16 -> QPW gated fp16 in, fp32 out (32) -> QPW fp32 in, ReLU, + that as residual (32) -> MEAN, or GeM
    pooling (GEM_A, eps 1e-6, p 3) -> HEADS_S8: the dense-conv models' int8 plan (python/bnneon/compiler/lower_dot.py)."""
    from bnneon import netbuild, pkgfmt
    pkg = pkgfmt.Package()
    net = netbuild.Net(pkg)
    ib = net.buf(netbuild.F32, H, W, C0)
    nrm = lambda *s: (rng.standard_normal(s) / np.sqrt(s[-1])).astype(np.float32)
    x1 = net.qconv3(ib, nrm(32, 3, 3, C0) * 1.4, rng.standard_normal(32) * 0.1, 2)
    x2 = net.qpw(x1, nrm(64, 32), rng.standard_normal(64) * 0.1, act="silu", out16=True, opad=1)
    x3, cs = net.dw3(x2, (rng.standard_normal((9, 64)) * 0.3), rng.standard_normal(64) * 0.1, 1, 1, 1, fp16=True)
    Ho, Wo = net.bufs[x3][1], net.bufs[x3][2]
    g = net.se_gate16(cs, Ho * Wo, nrm(8, 64), rng.standard_normal(8) * 0.1, nrm(64, 8), rng.standard_normal(64) * 0.1)
    x4 = net.qpw(x3, nrm(32, 64), rng.standard_normal(32) * 0.1, gate=g)
    x5 = net.qpw(x4, nrm(32, 32), rng.standard_normal(32) * 0.1, act="relu", res=x4)
    e = net.mean(x5) if pool == "mean" else net.gem_a(x5, 1e-6, 3.0)
    nc, hid = 20, 48
    heads = [(nrm(hid, 32), rng.standard_normal(hid) * 0.1, nrm(nc, hid), rng.standard_normal(nc) * 0.1,
              nrm(nc, hid), rng.standard_normal(nc) * 0.1) for _ in range(2)]
    out = net.heads_s8(x5, e, Ho, Wo, (nrm(nc, 32), rng.standard_normal(nc) * 0.1), heads)
    net.add_to("neon-fp16", netbuild.HW_FP16 | netbuild.HW_DOTPROD, in_buf=ib, out_buf=out, emb_buf=e)
    netbuild.standard_meta(pkg, H * W * C0, 32, model_id="synthetic_v3_int8", emb_dim=32)
    return pkg, net, ib, out, e


@pytest.mark.parametrize("H,W,n,pool", [(12, 16, 5, "mean"), (9, 14, 70, "mean"), (12, 16, 6, "gem"),
                                        (9, 14, 70, "gem")])
def test_v3_int8_plan_package(hip, tmp_path, H, W, n, pool):
    """every window of the batch against the op-by-op oracle interpreter, bit for bit (70 windows: two sub-batches)"""
    from bnneon import binding
    from oracle_net import OracleNet
    rng = np.random.default_rng(H * W)
    pkg, net, ib, out, e = v3_net(rng, H, W, pool=pool)
    path = str(tmp_path / "v3.bnpk")
    pkg.write(path)
    pcm = rng.standard_normal((n, H * W * 16)).astype(np.float32)
    say("v3 int8 plan package", H, W, n)
    with binding.Model(path) as m:
        got, emb, status = m.infer_batch(pcm)
        assert not status.any()
    orc = OracleNet(net, ib, out, e)
    for i in sorted({0, 1, n // 2, n - 1}):
        ro, re, _ = orc.run(pcm[i])
        assert same(got[i], ro[:got.shape[1]]), i
        assert same(emb[i], re[:32]), i


def test_gem_a_package(hip, tmp_path):
    from bnneon import binding, netbuild, pkgfmt
    from oracle_net import OracleNet
    rng = np.random.default_rng(11)
    M, C = 96, 64
    pkg = pkgfmt.Package()
    net = netbuild.Net(pkg)
    ib = net.buf(netbuild.F32, 8, 12, C)
    out = net.gem_a(ib, 1e-6, 3.0)
    net.add_to("neon-fp16", netbuild.HW_FP16 | netbuild.HW_DOTPROD, in_buf=ib, out_buf=out)
    netbuild.standard_meta(pkg, M * C, C, model_id="synthetic_gem")
    path = str(tmp_path / "gem.bnpk")
    pkg.write(path)
    pcm = np.abs(rng.standard_normal((4, M * C))).astype(np.float32)
    with binding.Model(path) as m:
        got, _, status = m.infer_batch(pcm)
        assert not status.any()
    orc = OracleNet(net, ib, out)
    for i in range(4):
        ro, _, _ = orc.run(pcm[i])
        assert same(got[i, :C], ro[:C]), i


def test_qpw_contract_refusals(hip, tmp_path):
    """QPW records the reference refuses: ReLU into fp16, a residual with fp16 out, a gate on fp32 rows"""
    from bnneon import binding, netbuild, pkgfmt
    rng = np.random.default_rng(12)
    for bad in ("relu16", "gate32"):
        pkg = pkgfmt.Package()
        net = netbuild.Net(pkg)
        ib = net.buf(netbuild.F32, 4, 4, 16)
        if bad == "relu16":
            out = net.qpw(ib, rng.standard_normal((16, 16)), np.zeros(16), act="relu", out16=True)
        else:
            gb = net.buf(netbuild.F16, 1, 1, 16, elems=16)
            out = net.qpw(ib, rng.standard_normal((16, 16)), np.zeros(16), gate=gb)
        net.add_to("neon-fp16", netbuild.HW_FP16 | netbuild.HW_DOTPROD, in_buf=ib, out_buf=out)
        netbuild.standard_meta(pkg, 256, 16, model_id="bad_qpw")
        path = str(tmp_path / f"{bad}.bnpk")
        pkg.write(path)
        with pytest.raises(Exception) as ei:
            binding.Model(path)
        assert "parameter check failed" in str(ei.value), (bad, str(ei.value))


@pytest.mark.parametrize("P,C,n", [(64, 64, 6), (24, 40, 70)])
def test_proto_dot_package(hip, tmp_path, P, C, n):
    """QPW (fp32 rows -> fp16 cells) -> PROTO variant 2: logits and colmax against the oracle interpreter, bit for
    bit (64 cells: the batched GEMM; 24: the per-window kernel; 70 windows: two sub-batches)"""
    from bnneon import binding, netbuild, pkgfmt
    from oracle_net import OracleNet
    rng = np.random.default_rng(P * C)
    nc, ppc = 8, 3
    Np = 24
    pkg = pkgfmt.Package()
    net = netbuild.Net(pkg)
    ib = net.buf(netbuild.F32, P, 1, 32)
    ld = (C + 15) // 16 * 16  # QPW's channels are a multiple of 16: the head reads the first C of them
    cells = net.qpw(ib, (rng.standard_normal((ld, 32)) / 5).astype(np.float32), np.zeros(ld, np.float32),
                    out16=True)
    q = rng.integers(-127, 128, (Np, C)).astype(np.int8)
    q12 = np.ascontiguousarray(q.reshape(Np // 12, 12, C // 4, 4).transpose(0, 2, 1, 3))
    sw = rng.uniform(0.001, 0.01, Np).astype(np.float32)
    out = net.proto_dot(cells, q12, sw, rng.standard_normal((nc, ppc)), rng.standard_normal(nc), C=C)
    net.add_to("neon-fp16", netbuild.HW_FP16 | netbuild.HW_DOTPROD, in_buf=ib, out_buf=out)
    netbuild.standard_meta(pkg, P * 32, nc, model_id="synthetic_proto_dot")
    path = str(tmp_path / "pd.bnpk")
    pkg.write(path)
    pcm = rng.standard_normal((n, P * 32)).astype(np.float32)
    say("proto dot package", P, C, n)
    with binding.Model(path) as m:
        got, _, status = m.infer_batch(pcm)
        assert not status.any()
    orc = OracleNet(net, ib, out)
    for i in sorted({0, n // 2, n - 1}):
        ro, _, _ = orc.run(pcm[i])
        assert same(got[i, :nc], ro[:nc]), i
