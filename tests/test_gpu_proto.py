"""GPU parity of the int8 prototype head kernels (quantize cells, column
maxima, logits) against the oracle, bit for bit, at small shapes and at
Perch v2's head shape (64 cells x 1536 channels x 59,180 prototypes)."""
import numpy as np
import pytest

import pyoracle as O
from bnneon import s8pack

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn])


def run_head(H, x, protos, clsw, clsb, nc, eps=1e-5):
    """x [B][P][ld] cells; returns (qa, sx, colmax, logits, fail) from the GPU."""
    B, P, ld = x.shape
    N, C = protos.shape
    Kp, Np = s8pack.r16(C), (N + 3) // 4 * 4
    q, sw = s8pack.quant_rows_s8(protos)
    qp = np.zeros((Np, Kp), np.int8)
    qp[:N, :C] = q
    swp = np.zeros(Np, np.float32)
    swp[:N] = sw
    qw = s8pack.pack_panels(qp)
    W = H.lib().bnh_s8p_new(Np, Kp, qw.ctypes.data, swp.ctypes.data)
    assert W
    dx = H.DeviceArray.from_host(x)
    dqa = H.DeviceArray.zeros((B, P * Kp), np.int8)
    dsx = H.DeviceArray.zeros((B, P), np.float32)
    dcm = H.DeviceArray.zeros((B, Np), np.float32)
    dlg = H.DeviceArray.zeros((B, nc), np.float32)
    dcw = H.DeviceArray.from_host(clsw.astype(np.float32))
    dcb = H.DeviceArray.from_host(clsb.astype(np.float32))
    dfl = H.DeviceArray.zeros(B, np.int32)
    L = H.lib()
    H.check(L.bnh_quant_cells(dx.ptr, P * ld, P, C, ld, eps, dqa.ptr, P * Kp, Kp, dsx.ptr, P, B, None))
    H.check(L.bnh_proto_colmax(dqa.ptr, P * Kp, dsx.ptr, P, P, W, dcm.ptr, Np, B, None))
    H.check(L.bnh_proto_logits(dcm.ptr, Np, dcw.ptr, dcb.ptr, nc, N // nc, dlg.ptr, nc, B, dfl.ptr, 7, None))
    H.sync()
    L.bnh_s8p_free(W)
    res = (dqa.numpy().reshape(B, P, Kp), dsx.numpy(), dcm.numpy(), dlg.numpy(), dfl.numpy())
    return res, (qw, swp, Np, Kp)


# (64, 256, ...) and (64, 512, ...) take the batched GEMM (64 cells per window, K in 64-byte slices); the others the
# per-window kernel
@pytest.mark.parametrize("P,C,N,nc", [(4, 8, 4, 1), (12, 48, 20, 5), (64, 136, 400, 100), (100, 96, 1000, 250),
                                      (64, 256, 1000, 250), (64, 512, 2044, 511)])
def test_head_small_shapes(hip, P, C, N, nc):
    rng = np.random.default_rng(P + C)
    B = 3
    ld = C + 8
    x = rng.standard_normal((B, P, ld)).astype(np.float32)
    x[1, 0, :] = 0                        # a zero cell
    x[1, 1, :C] = np.where(np.arange(C) % 2, -1e-38, 1e-38)  # a cell whose scale overflows
    x[2, P - 1, C // 2] = np.nan          # a NaN window
    protos = rng.standard_normal((N, C)).astype(np.float32)
    protos[N - 1] = 0                     # an all-zero prototype (sw = 0)
    clsw = rng.uniform(0.5, 1.5, N).astype(np.float32)
    clsb = rng.standard_normal(nc).astype(np.float32)
    say("proto head", P, C, N, nc)
    (qa, sx, cm, lg, fl), (qw, swp, Np, Kp) = run_head(hip, x, protos, clsw, clsb, nc)
    for b in range(B):
        rc, rlg, rcm, rqa = O.proto_s8(x[b], C, 1e-5, qw, swp, Np, Kp, clsw, clsb, nc, N // nc)
        assert np.array_equal(qa[b], rqa), b
        assert same(cm[b], rcm), b
        assert same(lg[b], rlg), b
        assert (fl[b] != 0) == (rc != 0) and (rc == 0 or fl[b] == 7)


def test_head_perch_shape(hip):
    """Perch v2's prototype head: 16 x 4 cells of 1536 channels, 14,795
    classes x 4 prototypes, batch of 2 windows."""
    rng = np.random.default_rng(11)
    B, P, C, nc, ppc = 2, 64, 1536, 14795, 4
    N = nc * ppc
    x = np.maximum(rng.standard_normal((B, P, C)), 0).astype(np.float32)
    protos = rng.standard_normal((N, C)).astype(np.float32)
    clsw = rng.uniform(0, 1, N).astype(np.float32)
    clsb = rng.standard_normal(nc).astype(np.float32) * 0.1
    say("proto head perch shape")
    (qa, sx, cm, lg, fl), (qw, swp, Np, Kp) = run_head(hip, x, protos, clsw, clsb, nc)
    for b in range(B):
        rc, rlg, rcm, rqa = O.proto_s8(x[b], C, 1e-5, qw, swp, Np, Kp, clsw, clsb, nc, ppc)
        assert np.array_equal(qa[b], rqa)
        assert same(cm[b], rcm)
        assert same(lg[b], rlg)


@pytest.mark.parametrize("B", [5, 37])
def test_batched_gemm_matches_per_window_kernel(hip, monkeypatch, B):
    """The batched column-max GEMM (tiles of 4 windows x 256 prototypes, split over the XCDs) against the
    one-window-per-block kernel on every window, and both against the oracle on some: B = 5 leaves a partial cell
    tile and splits the prototypes over XCD regions, B = 37 gives 10 cell tiles over 8 regions."""
    H = hip
    rng = np.random.default_rng(40 + B)
    P, C, nc, ppc = 64, 1536, 1500, 4
    N = nc * ppc
    x = np.maximum(rng.standard_normal((B, P, C)), 0).astype(np.float32)
    x[B - 1, 5, :] = 0                    # a zero cell in the last window
    protos = rng.standard_normal((N, C)).astype(np.float32)
    protos[7] = 0
    clsw = rng.uniform(0, 1, N).astype(np.float32)
    clsb = rng.standard_normal(nc).astype(np.float32)
    say("proto batched gemm B", B)
    (qa, sx, cm, lg, fl), (qw, swp, Np, Kp) = run_head(H, x, protos, clsw, clsb, nc)
    monkeypatch.setenv("BNH_PROTO_WINDOW", "1")
    (qa2, sx2, cm2, lg2, fl2), _ = run_head(H, x, protos, clsw, clsb, nc)
    assert same(cm, cm2) and same(lg, lg2)
    for b in (0, B // 2, B - 1):
        rc, rlg, rcm, rqa = O.proto_s8(x[b], C, 1e-5, qw, swp, Np, Kp, clsw, clsb, nc, ppc)
        assert same(cm[b], rcm) and same(lg[b], rlg), b
