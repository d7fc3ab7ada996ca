"""Pins the oracle of the int8 prototype head (oracle/proto.c): the edge cases
of the reference's own kernel test (bench/test_proto_s8n.c:139-175: a tiny
cell whose scale overflows keeps its bytes in [-127, 127], a zero cell stays
finite, padding is zero), closed forms of the normalisation, a brute-force
column maximum and the n4 loader check against s8pack's flags."""
import numpy as np

import pyoracle as O
from bnneon import s8pack


def test_quant_cells_tiny_zero_and_padding():
    C, Kp = 1528, 1536
    rng = np.random.default_rng(7)
    x = (rng.integers(-1000, 1001, (4, C)) / 512.0).astype(np.float32)
    x[1] = np.where(np.arange(C) % 2, -1e-38, 1e-38)   # 127 / max|x| is +inf
    x[2] = 0
    qa, sx = O.quant_cells(x, C, Kp, 1e-5)
    assert qa[:, :C].min() >= -127
    assert not qa[:, C:].any()
    assert np.isfinite(sx).all()
    assert (qa[1, :C] == np.where(np.arange(C) % 2, -127, 127)).all()
    assert not qa[2].any()


def test_quant_cells_scale_closed_form():
    # a cell whose max |x| is exactly representable: q = round(x * 127 / mx)
    x = np.array([[3.0, -1.5, 0.75, 0, 0, 0, 0, 0]], np.float32)
    qa, sx = O.quant_cells(x, 8, 16, 0.0)
    assert qa[0, :8].tolist() == [127, -64, 32, 0, 0, 0, 0, 0]  # 63.5 rounds away to 64, 31.75 -> 32
    norm = np.float32(np.sqrt(np.float32(9 + 2.25 + 0.5625)))
    assert sx[0] == np.float32(3.0) / (np.float32(127) * norm)


def test_colmax_brute_force_and_logits():
    rng = np.random.default_rng(8)
    P, C, N, nc = 12, 48, 20, 5
    x = rng.standard_normal((P, C)).astype(np.float32)
    protos = rng.standard_normal((N, C)).astype(np.float32)
    q, sw = s8pack.quant_rows_s8(protos)
    Kp, Np = 48, 20
    qw = s8pack.pack_panels(q)
    clsw = rng.standard_normal(N).astype(np.float32)
    clsb = rng.standard_normal(nc).astype(np.float32)
    rc, lg, cm, qa = O.proto_s8(x, C, 1e-5, qw, sw, Np, Kp, clsw, clsb, nc, N // nc)
    assert rc == 0
    qa2, sx = O.quant_cells(x, C, Kp, 1e-5)
    acc = qa2.astype(np.int64) @ q.astype(np.int64).T            # [P][N]
    ref = ((acc.astype(np.int32).astype(np.float32) * sx[:, None]).max(0) * sw).astype(np.float32)
    assert np.array_equal(cm[:N], ref)
    # the int8 similarity approximates the cosine of cell and prototype
    cos = (x / np.linalg.norm(x, axis=1, keepdims=True)) @ (protos / 1).T
    approx = (acc * sx[:, None] * sw[None, :])
    assert np.abs(approx - cos).max() < 0.05 * np.abs(cos).max() * np.abs(protos).max() + 0.05
    s = np.zeros(nc, np.float32)
    for c in range(nc):
        acc_f = np.float32(0)
        for j in range(N // nc):
            acc_f = np.float32(acc_f + np.float32(cm[c * 4 + j] * clsw[c * 4 + j]))
        s[c] = np.float32(acc_f + clsb[c])
    assert np.array_equal(lg, s)


def test_logits_nonfinite_flag():
    rng = np.random.default_rng(9)
    P, C, N, nc = 4, 8, 4, 1
    # a cell with a NaN: its norm and scale are NaN, the column maxima and the
    # logit follow; values far above fp32 range in the cells only zero the
    # scale (3e38^2 overflows the norm), which stays finite
    x = rng.standard_normal((P, C)).astype(np.float32)
    q, sw = s8pack.quant_rows_s8(rng.standard_normal((N, C)).astype(np.float32))
    qw = s8pack.pack_panels(np.pad(q, ((0, 0), (0, 8))))
    args = (sw, 4, 16, np.ones(N, np.float32), np.zeros(1, np.float32), nc, N)
    assert O.proto_s8(x, C, 1e-5, qw, *args)[0] == 0
    x[2, 5] = np.nan
    rc, lg, _, _ = O.proto_s8(x, C, 1e-5, qw, *args)
    assert rc == -2 and np.isnan(lg).all()
    rc, lg, _, _ = O.proto_s8(np.full((P, C), 3e38, np.float32), C, 1e-5, qw, *args)
    assert rc == 0 and (lg == 0).all()


def test_n4_check_matches_flags():
    rng = np.random.default_rng(10)
    q = rng.integers(-90, 91, (16, 64)).astype(np.int8)
    flags = s8pack.n4_panel_flags(q)
    assert O.n4_check(s8pack.pack_panels(q), 64, flags) == -1
    forged = np.ones_like(flags)
    bad = O.n4_check(s8pack.pack_panels(q), 64, forged)
    assert bad == int(np.argmin(flags))     # the first panel the compiler did not flag
    assert O.n4_check(s8pack.pack_panels(np.zeros((8, 48), np.int8)), 48, np.ones(2, np.int8)) == -1
