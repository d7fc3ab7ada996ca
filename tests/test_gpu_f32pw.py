"""GPU parity of the fp32 1x1 convolution (the registry's PW op, variant 0) against the oracle's restatement of
gemm_f32 (oracle/fe.c: one FMA chain over k < Kp per output from +0, + b, activation, + residual), bit for bit:
K tails that are not a multiple of the kernel's 16-wide K chunk, row tails, partial channel blocks, the gate, the
zero-haloed output and residual forms, infinities / NaNs / signed zeros, several windows with padded strides; and
a package whose fp32 PW ops (one gated by SE_GATE, one adding a residual) run through bnn_infer_batch against the
op-by-op oracle interpreter."""
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


def run_gemm(H, A, panels, bb, Kp, Np, act=0, gate=None, res=None, ldr=0, rpad=0, rw=0, ow=0, opad=0, ldo=None,
             slack=24):
    """A [B][M][lda] -> the kernel's output rows per window (halo included)."""
    B, M, lda = A.shape
    ldo = ldo or Np
    rows = M if not opad else (M // ow + 2 * opad) * (ow + 2 * opad)
    a_ws = M * lda + slack
    xs = np.zeros((B, a_ws), np.float32)
    xs[:, :M * lda] = A.reshape(B, -1)
    dA = H.DeviceArray.from_host(xs)
    dW, db = H.DeviceArray.from_host(np.ascontiguousarray(panels)), H.DeviceArray.from_host(bb)
    o_ws = rows * ldo + slack
    dO = H.DeviceArray.from_host(np.full((B, o_ws), 7.0, np.float32))
    dg = dr = None
    g_ws = r_ws = 0
    if gate is not None:
        g_ws = gate.shape[1] + 8
        gs = np.zeros((B, g_ws), np.float32)
        gs[:, :gate.shape[1]] = gate
        dg = H.DeviceArray.from_host(gs)
    if res is not None:
        r_ws = res[0].size + slack
        rs = np.zeros((B, r_ws), np.float32)
        rs[:, :res[0].size] = res.reshape(B, -1)
        dr = H.DeviceArray.from_host(rs)
    e = H.Epi32(act, dO.ptr, o_ws, ldo, ow, opad, dr.ptr if dr else None, r_ws, ldr, rpad, rw)
    H.check(H.lib().bnh_gemm_f32(dA.ptr, a_ws, lda, M, dg.ptr if dg else None, g_ws, dW.ptr, db.ptr, Kp, Np,
                                 H.C.byref(e), B, None), "gemm_f32")
    H.sync()
    return dO.numpy()[:, :rows * ldo].reshape(B, rows, ldo)


@pytest.mark.parametrize("M,K,N,act", [(64, 64, 64, 0), (100, 36, 24, 1), (77, 132, 72, 2), (8, 4, 8, 1),
                                       (300, 1152, 192, 0), (1536, 192, 1152, 1)])
def test_gemm_f32_shapes(hip, M, K, N, act):
    rng = np.random.default_rng(M + K + N)
    B = 3
    w = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    panels, bb, (_, _, Kp, Np) = netbuild.Net.fpack(w, b)
    lda = Kp + 4
    A = rng.standard_normal((B, M, lda)).astype(np.float32)
    say("gemm_f32", M, K, N, act)
    out = run_gemm(hip, A, panels, bb, Kp, Np, act=act)
    for i in (0, B - 1):
        ref = O.gemm_f32(A[i], panels, bb, Kp, Np, act=act)
        assert same(out[i], ref), ("window", i)


def test_gemm_f32_gate_residual_halo(hip):
    rng = np.random.default_rng(5)
    B, Hh, W, K, N = 2, 6, 10, 48, 40
    M = Hh * W
    w = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    panels, bb, (_, _, Kp, Np) = netbuild.Net.fpack(w, b)
    A = rng.standard_normal((B, M, Kp)).astype(np.float32)
    gate = rng.uniform(0, 1, (B, K)).astype(np.float32)
    ldr, rpad = Np, 1
    res = np.zeros((B, (Hh + 2) * (W + 2), ldr), np.float32)
    res[:] = rng.standard_normal(res.shape).astype(np.float32)
    say("gemm_f32 gate + haloed residual + padded output")
    for act in (0, 1, 2):
        out = run_gemm(hip, A, panels, bb, Kp, Np, act=act, gate=gate, res=res, ldr=ldr, rpad=rpad, rw=W, ow=W,
                       opad=2, ldo=Np + 8)
        for i in range(B):
            ref = O.gemm_f32(A[i], panels, bb, Kp, Np, act=act, gate=gate[i], res=res[i], ldr=ldr, rpad=rpad,
                             rw=W, ow=W, opad=2, ldo=Np + 8)
            # the oracle leaves the halo at zero; the op zeroes it before the GEMM (the kernel stores rows only)
            o = out[i].reshape(Hh + 4, W + 4, Np + 8)[2:-2, 2:-2, :Np]
            r = ref.reshape(Hh + 4, W + 4, Np + 8)[2:-2, 2:-2, :Np]
            assert same(o, r), (act, i)


def test_gemm_f32_specials(hip):
    """inf, NaN and signed zeros flow through the chains as on the CPU (a -0 chain stays -0 until the bias)."""
    rng = np.random.default_rng(9)
    B, M, K, N = 1, 40, 20, 16
    w = rng.standard_normal((N, K)).astype(np.float32)
    w[3, :] = 0.0
    b = rng.standard_normal(N).astype(np.float32)
    b[5] = -0.0
    panels, bb, (_, _, Kp, Np) = netbuild.Net.fpack(w, b)
    A = rng.standard_normal((B, M, Kp)).astype(np.float32)
    A[0, 2, 3], A[0, 7, 1], A[0, 9, 0] = np.inf, np.nan, -np.inf
    A[0, 11, :] = -0.0
    A[0, 12, :] = 3e38
    for act in (0, 1, 2):
        out = run_gemm(hip, A, panels, bb, Kp, Np, act=act)
        assert same(out[0], O.gemm_f32(A[0], panels, bb, Kp, Np, act=act)), act


def test_gemm_f32_refusals(hip):
    H = hip
    L = H.lib()
    d = H.DeviceArray.zeros(4096, np.float32)
    e = H.Epi32(0, d.ptr, 0, 8, 0, 0, None, 0, 0, 0, 0)
    assert L.bnh_gemm_f32(d.ptr, 0, 8, 4, None, 0, d.ptr, d.ptr, 6, 8, H.C.byref(e), 1, None) != 0   # Kp % 4
    assert L.bnh_gemm_f32(d.ptr, 0, 4, 4, None, 0, d.ptr, d.ptr, 8, 8, H.C.byref(e), 1, None) != 0   # lda < Kp
    assert L.bnh_gemm_f32(d.ptr, 0, 8, 4, None, 0, d.ptr, d.ptr, 8, 12, H.C.byref(e), 1, None) != 0  # Np % 8
    assert b"parameter check" in L.bnh_last_error()


def test_pw_f32_ops_in_a_package(hip, tmp_path):
    """rows -> PW fp32 (SiLU, zero-haloed output) -> DW3 fp32 -> SE_GATE -> PW fp32 (gated, + the input as
    residual): output and channel sums against the oracle interpreter, bit for bit."""
    rng = np.random.default_rng(31)
    Hh, W, K0, N1 = 8, 12, 40, 24
    pkg = pkgfmt.Package()
    net = netbuild.Net(pkg)
    ib = net.buf(netbuild.F32, Hh, W, K0)
    w1 = (rng.standard_normal((N1, K0)) * 0.3).astype(np.float32)
    b1 = (rng.standard_normal(N1) * 0.1).astype(np.float32)
    h1 = net.pw(ib, w1, b1, act="silu", opad=1)
    wd = (rng.standard_normal((9, N1)) * 0.4).astype(np.float32)
    bd = (rng.standard_normal(N1) * 0.1).astype(np.float32)
    d, cs = net.dw3(h1, wd, bd, 1)
    rd = 6
    g = net.se_gate(cs, Hh * W, rng.standard_normal((rd, N1)).astype(np.float32) * 0.3,
                    rng.standard_normal(rd).astype(np.float32) * 0.1,
                    rng.standard_normal((N1, rd)).astype(np.float32) * 0.3,
                    rng.standard_normal(N1).astype(np.float32) * 0.1)
    w2 = (rng.standard_normal((K0, N1)) * 0.3).astype(np.float32)
    b2 = (rng.standard_normal(K0) * 0.1).astype(np.float32)
    out = net.pw(d, w2, b2, gate=g, res=ib)
    net.add_to("neon-int8", 0, in_buf=ib, out_buf=out, emb_buf=cs)
    netbuild.standard_meta(pkg, Hh * W * K0, Hh * W * K0, model_id="synthetic_pw_f32", emb_dim=N1)
    path = str(tmp_path / "pw32.bnpk")
    pkg.write(path)
    n = 5
    pcm = rng.standard_normal((n, Hh * W * K0)).astype(np.float32)
    say("runtime pw_f32")
    with binding.Model(path) as m:
        got, emb, status = m.infer_batch(pcm)
        assert not status.any()
    orc = OracleNet(net, ib, out, cs)
    for i in (0, n - 1):
        ro, re, _ = orc.run(pcm[i])
        assert same(got[i], ro[:Hh * W * K0]), i
        assert same(emb[i], re[:N1]), i
