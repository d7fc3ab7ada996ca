"""The fp32 / fp16 prototype heads on the GPU (PROTO variant 0, PROTO_F32H, PROTO variant 1): the L2 normalisation,
the column maxima and whole packages through bnn_infer_batch, every output bit for bit against the oracle
(oracle/proto.c; src/rt_ops_f32.c:548-591, src/rt_ops_f16.c:227-250)."""
import numpy as np
import pytest

import pyoracle as O
from bnneon import netbuild

pytestmark = pytest.mark.gpu
f32, f16 = np.float32, np.float16


def say(*a):
    print(*a, flush=True)


def same(a, b):
    a, b = np.asarray(a, f32), np.asarray(b, f32)
    an, bn = np.isnan(a), np.isnan(b)
    return np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn])


def pack(kind, protos):
    """The package tensor of kind's prototypes (as netbuild writes it) and Np."""
    N, K = protos.shape
    Np = (N + 7) // 8 * 8
    if kind == "f32":
        panels, _, (_, _, Kp, Np) = netbuild.Net.fpack(protos, np.zeros(N, f32), K_pad=8)
        return panels, Np
    if kind == "f16":
        w, _, _, (_, _, Kp, Np) = netbuild.Net.pack_h16(protos, np.zeros(N, f32), K)
        return w, Np
    w16p = np.zeros((Np, K), f16)
    w16p[:N] = protos.astype(f16)
    return np.ascontiguousarray(w16p.reshape(Np // 8, 8, K).transpose(0, 2, 1)), Np


KIND = {"f32": 0, "f32h": 1, "f16": 2}


def oracle_colmax(kind, a, w, Np):
    if kind == "f32":
        return O.colmax_f32(a, w, a.shape[1], Np)
    if kind == "f32h":
        return O.colmax_f32h(a, w, Np)
    return O.colmax_f16(a, w, a.shape[1], Np)


@pytest.mark.parametrize("fp16", [False, True])
@pytest.mark.parametrize("P,C,ld", [(64, 1536, 1536), (24, 40, 48), (8, 8, 8), (136, 264, 272)])
def test_l2norm_cells(hip, fp16, P, C, ld):
    H = hip
    rng = np.random.default_rng(P + C)
    B = 3
    x = rng.standard_normal((B, P, ld)).astype(f32)
    x[1, 0] = 0                      # den = eps
    x[1, 1] = 1e-30                  # squares underflow to 0
    x[1, 2, 3] = np.inf
    x[2, 5, 7] = np.nan
    x[2, 6, :C] = 3e19               # squares overflow to inf
    if fp16:
        x = np.clip(x, -60000, 60000).astype(f16)
        x[2, 5, 7] = np.nan
    dt = f16 if fp16 else f32
    dx = H.DeviceArray.from_host(x)
    da = H.DeviceArray.zeros((B, P, C), dt)
    say("l2norm", fp16, P, C, ld)
    H.check(H.lib().bnh_l2norm_cells(dx.ptr, P * ld, P, C, ld, 1e-5, int(fp16), da.ptr, P * C, B, None), "l2norm")
    H.sync()
    got = da.numpy()
    for b in range(B):
        ref = O.l2norm(x[b], C, 1e-5, f16=fp16)
        if fp16:
            assert same(got[b].astype(f32), ref.view(f16).astype(f32)), b
        else:
            assert same(got[b], ref), b


@pytest.mark.parametrize("kind", ["f32", "f32h", "f16"])
@pytest.mark.parametrize("P,K,N,B", [(64, 1536, 2056, 2), (24, 40, 300, 3), (136, 264, 24, 2), (8, 8, 8, 1),
                                     (72, 136, 520, 2)])
def test_colmax(hip, kind, P, K, N, B):
    """every window's column maxima against the oracle, bit for bit: normalised cells, prototypes of both signs,
    Np % 16 == 8 tails, cells past a 64-cell tile, K tails of 8 and K blocks of the fp16 chains"""
    H = hip
    rng = np.random.default_rng(P * K + N)
    protos = rng.standard_normal((N, K)).astype(f32) / np.sqrt(K)
    w, Np = pack(kind, protos)
    cells = rng.standard_normal((B, P, K)).astype(f32)
    if kind == "f16":
        cells = cells.astype(f16)
    a = np.stack([O.l2norm(cells[b], K, 1e-5, f16=kind == "f16") for b in range(B)])
    if kind == "f16":
        a = a.view(f16)
    Wd = H.FProto(KIND[kind], Np, K, w)
    da = H.DeviceArray.from_host(a)
    dcm = H.DeviceArray.zeros((B, Np), f32)
    say("fproto colmax", kind, P, K, N, B)
    H.check(H.lib().bnh_fproto_colmax(da.ptr, P * K, P, Wd.h, dcm.ptr, Np, B, None), "colmax")
    H.sync()
    got = dcm.numpy()
    for b in range(B):
        ref = oracle_colmax(kind, a[b], w, Np)
        assert same(got[b], ref), (b, np.argwhere(got[b] != ref)[:4])


@pytest.mark.parametrize("kind", ["f32", "f32h", "f16"])
def test_colmax_orders_and_specials(hip, kind):
    """rows whose chains the reference's order decides (absorption at 2^24 / fp16 2048, a fused product on -1),
    infinite products, all-zero prototypes (+0 chains); then a NaN in one cell, which every column's max keeps"""
    H = hip
    P, K, N = 16, 264, 40
    a = np.zeros((P, K), f32)
    W = np.zeros((N, K), f32)
    a[0, 200], a[0, 201:208], a[0, 208], a[0, 209] = 64, 1, -64, 1   # products 4096, seven 1s, -4096, -1
    W[1, 200], W[1, 201:208], W[1, 208], W[1, 209] = 64, 1, 64, -1
    a[1, :] = 1
    W[3, 0], W[3, 87], W[3, 88], W[3, 127] = 2048, 1, 1, 1          # fp16 blocks of 88: 2050
    a[2, 0], a[2, 1] = 1, 1 + 2 ** -6
    W[5, 0], W[5, 1] = -1, 1 + 2 ** -6                                # a fused product: 2^-5 + 2^-12
    a[3, 10] = 30000
    W[7, 10] = 30000                                                  # fp16: inf; fp32: 9e8
    w, Np = pack(kind, W)
    Wd = H.FProto(KIND[kind], Np, K, w)
    a1 = a.copy()
    a1[4, 11] = np.nan                                                # window 1: a NaN in one cell
    A = np.stack([a, a1]).astype(f16 if kind == "f16" else f32)
    da = H.DeviceArray.from_host(A)
    dcm = H.DeviceArray.zeros((2, Np), f32)
    say("fproto specials", kind)
    H.check(H.lib().bnh_fproto_colmax(da.ptr, P * K, P, Wd.h, dcm.ptr, Np, 2, None), "colmax")
    H.sync()
    got = dcm.numpy()
    for b in range(2):
        ref = oracle_colmax(kind, A[b], w, Np)
        assert same(got[b], ref), (b, np.argwhere(got[b].view(np.uint32) != ref.view(np.uint32))[:6])
    if kind == "f16":
        assert got[0, 3] == 2050 and got[0, 5] == f32(2 ** -5 + 2 ** -12) and np.isinf(got[0, 7])
    assert not np.isnan(got[0]).any() and np.isnan(got[1]).all()   # NaN x 0 is NaN: every column


def test_colmax_perch_head(hip):
    """the Perch v2 head's shape, 64 cells x 1536 channels x 59,180 prototypes: fp32 column maxima of every
    prototype against the oracle; fp16 and PROTO_F32H on a spread of 1,032 prototypes (the oracle's software fp16
    FMA is too slow for all of them), with the same prototypes at their own positions in the full tensor"""
    H = hip
    P, K, N = 64, 1536, 59180
    rng = np.random.default_rng(59180)
    protos = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(f32)
    cells = rng.standard_normal((P, K)).astype(f32)
    pick = np.unique(np.concatenate([np.arange(0, 512), np.arange(N - 512, N),
                                     rng.choice(N, 8, replace=False)]))
    for kind in ("f32", "f32h", "f16"):
        w, Np = pack(kind, protos)
        a = O.l2norm(cells.astype(f16) if kind == "f16" else cells, K, 1e-5, f16=kind == "f16")
        if kind == "f16":
            a = a.view(f16)
        Wd = H.FProto(KIND[kind], Np, K, w)
        da = H.DeviceArray.from_host(a)
        dcm = H.DeviceArray.zeros((1, Np), f32)
        say("perch head colmax", kind)
        H.check(H.lib().bnh_fproto_colmax(da.ptr, 0, P, Wd.h, dcm.ptr, 0, 1, None), "colmax")
        H.sync()
        got = dcm.numpy()[0]
        if kind == "f32":
            ref = oracle_colmax(kind, a, w, Np)
            assert same(got, ref), np.argwhere(got != ref)[:4]
        else:
            sub, sNp = pack(kind, protos[pick])
            ref = oracle_colmax(kind, a, sub, sNp)[:len(pick)]
            assert same(got[pick], ref), np.argwhere(got[pick] != ref)[:4]
        del Wd, da, dcm


# ------------------------------------------------------------------ the ops in packages
def head_net(kind, rng, P, C, ld, N, nc):
    """fp32 / f32h: input rows [P][ld] -> the head; fp16: a P-pixel image -> STEM (fp16 out, C channels) -> head"""
    from bnneon import pkgfmt
    pkg = pkgfmt.Package()
    net = netbuild.Net(pkg)
    protos = rng.standard_normal((N, C)).astype(f32)
    clsw = rng.uniform(0.5, 1.5, N).astype(f32)
    clsb = rng.standard_normal(nc).astype(f32)
    if kind == "f16":
        Hh, Wh = 18, 20                                              # 3x3 VALID: 16 x 18 = 288 cells
        ib = net.buf(netbuild.F32, Hh, Wh, 1)
        cells = net.stem_f16(ib, rng.standard_normal((C, 9)).astype(f32) / 3, rng.standard_normal(C) * 0.1, 3, 1,
                             ldo=C)
        nsamp, hw = Hh * Wh, netbuild.HW_FP16
        path = "neon-fp16"
    else:
        ib = net.buf(netbuild.F32, P, 1, C, ld=ld)
        cells, nsamp, hw, path = ib, P * ld, 0, "neon-fp32"
    out = net.proto_fp(cells, protos, clsw, clsb, kind=kind)
    net.add_to(path, hw, in_buf=ib, out_buf=out)
    netbuild.standard_meta(pkg, nsamp, nc, model_id=f"synthetic_proto_{kind}")
    return pkg, net, ib, out, nsamp


@pytest.mark.parametrize("kind,n", [("f32", 5), ("f32", 70), ("f32h", 6), ("f16", 5), ("f16", 70)])
def test_proto_fp_package(hip, tmp_path, kind, n):
    """logits of every checked window against the op-by-op oracle interpreter, bit for bit (70 windows: two
    sub-batches on two streams)"""
    from bnneon import binding
    from oracle_net import OracleNet
    rng = np.random.default_rng(n + len(kind))
    nc = 12
    pkg, net, ib, out, nsamp = head_net(kind, rng, 40, 48, 56, nc * 5, nc)
    path = str(tmp_path / f"{kind}.bnpk")
    pkg.write(path)
    pcm = rng.standard_normal((n, nsamp)).astype(f32)
    say("proto package", kind, n)
    with binding.Model(path) as m:
        got, _, status = m.infer_batch(pcm)
        assert not status.any()
    orc = OracleNet(net, ib, out)
    for i in sorted({0, 1, n // 2, n - 1}):
        ro, _, _ = orc.run(pcm[i])
        assert same(got[i, :nc], ro[:nc]), i


def test_proto_fp_failed_window(hip, tmp_path):
    """a window whose logit is not finite fails with the op named (pc_proto_logits' -2), the others score"""
    from bnneon import binding
    rng = np.random.default_rng(3)
    nc = 4
    pkg, net, ib, out, nsamp = head_net("f32", rng, 8, 16, 16, nc * 2, nc)
    path = str(tmp_path / "bad.bnpk")
    pkg.write(path)
    pcm = rng.standard_normal((3, nsamp)).astype(f32)
    pcm[1, 5] = np.nan
    with binding.Model(path) as m:
        got, _, status = m.infer_batch(pcm, check=False)
    assert status[0] == 0 and status[2] == 0 and status[1] != 0
