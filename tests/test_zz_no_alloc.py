"""bnh_pw_s8_static, the PW_S8 run without a workspace or any allocation: the
same bytes as bnh_pw_s8 with a caller workspace (and as the oracle), on two
calls in a row, the second with a smaller input, plus its size refusal."""
import numpy as np
import pytest

import pyoracle as O
from bnneon import s8pack

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same_f32(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn]))


class Case:
    """One PW_S8 launch: B windows of H x W pixels, K -> N channels, optional zero-haloed output and residual."""

    def __init__(self, H, seed, B, H_, W_, K, N, act, opad=0, res=False, gate=False):
        rng = np.random.default_rng(seed)
        self.H, self.B, self.M, self.K, self.act, self.opad = H, B, H_ * W_, K, act, opad
        w = (rng.standard_normal((N, K)) * rng.uniform(0.01, 1, (N, 1))).astype(np.float32)
        self.pk = s8pack.pack_s8(w, rng.standard_normal(N).astype(np.float32))
        _, _, self.Kp, self.Np = self.pk["shape"]
        self.W = H.S8Weights(N, K, self.Kp, self.Np, self.pk["q"], self.pk["sw"], self.pk["cs"], self.pk["b"])
        self.x = (rng.standard_normal((B, self.M, K)) * 2).astype(np.float32)
        self.x[0, 3] = 0.0                       # a constant row
        self.g = rng.uniform(0, 1, (B, K)).astype(np.float32) if gate else None
        self.rs = rng.standard_normal((B, self.M, self.Np)).astype(np.float32) if res else None
        self.ldo = self.Np + 4
        self.ow = W_ if opad else 0
        self.rows = self.M if not opad else (H_ + 2 * opad) * (W_ + 2 * opad)
        self.dx = H.DeviceArray.from_host(self.x)
        self.dg = H.DeviceArray.from_host(self.g) if gate else None
        self.dres = H.DeviceArray.from_host(self.rs) if res else None

    def out(self):
        d = self.H.DeviceArray.from_host(np.full((self.B, self.rows * self.ldo), 5.0, np.float32))
        e = self.H.epi32(d, self.ldo, act=self.act, ow=self.ow, opad=self.opad, res=self.dres,
                         ldr=self.Np if self.dres is not None else 0, out_ws=self.rows * self.ldo,
                         res_ws=self.M * self.Np)
        return d, e

    def run_workspace(self):
        H, M, Kp = self.H, self.M, self.Kp
        dq = H.DeviceArray.zeros((self.B, M * Kp), np.int8)
        dsa = H.DeviceArray.zeros((self.B, M), np.float32)
        dza = H.DeviceArray.zeros((self.B, M), np.int32)
        d, e = self.out()
        H.check(H.lib().bnh_pw_s8(self.dx.ptr, M * self.K, self.K, M, H.ptr(self.dg), self.K if self.g is not None
                                  else 0, dq.ptr, M * Kp, dsa.ptr, M, dza.ptr, M, self.B, self.W.h, e, None), "pw_s8")
        H.sync()
        return d.numpy().reshape(self.B, self.rows, self.ldo)

    def run_static(self):
        H, M = self.H, self.M
        d, e = self.out()
        H.check(H.lib().bnh_pw_s8_static(self.dx.ptr, M * self.K, self.K, M, H.ptr(self.dg),
                                         self.K if self.g is not None else 0, self.B, self.W.h, e, None),
                "pw_s8_static")
        H.sync()
        return d.numpy().reshape(self.B, self.rows, self.ldo)

    def oracle(self, b):
        ref, *_ = O.pw_s8(self.x[b], self.pk, act=self.act, ldo=self.ldo, ow=self.ow, opad=self.opad,
                          res=None if self.rs is None else self.rs[b], ldr=self.Np if self.rs is not None else 0,
                          gate=None if self.g is None else self.g[b])
        return ref


def test_static_matches_workspace_twice_smaller_second(hip):
    # the first call fills most of the scratch (4 windows x 1536 rows x 1152 bytes = 7 MB of quantized rows), the
    # second is smaller and finds the first call's contents there
    big = Case(hip, 21, 4, 24, 64, 1152, 256, 1)
    small = Case(hip, 22, 2, 7, 9, 40, 136, 2, opad=1, res=True, gate=True)
    for c in (big, small):
        say(f"pw_s8_static B{c.B} M{c.M} K{c.K} Kp{c.Kp} Np{c.Np}")
        got = c.run_static()
        want = c.run_workspace()
        assert same_f32(got[..., :c.Np], want[..., :c.Np])
        for b in (0, c.B - 1):
            assert same_f32(got[b, :, :c.Np], c.oracle(b)[:, :c.Np]), b


def test_static_refuses_oversized(hip):
    H = hip
    c = Case(hip, 23, 1, 4, 4, 1152, 16, 0)
    d, e = c.out()
    # 40 windows of 1536 rows of Kp 1152 = 70.8 MB > 64 MiB: refused on the host, nothing launched
    rc = H.lib().bnh_pw_s8_static(c.dx.ptr, 0, c.K, 1536, None, 0, 40, c.W.h, e, None)
    assert rc != 0
    assert b"more than its" in H.lib().bnh_last_error()
