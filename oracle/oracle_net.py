"""Runs a package's op records on the CPU oracle, one window at a time.

Test infrastructure: the interpreter walks the op list that netbuild wrote
into the package (the same records the GPU runtime executes) and calls the
oracle's restatement of each op, with every buffer as a flat numpy array of
the buffer's element count, so a net's logits can be compared bit for bit with
the GPU's. Buffers follow the package's descriptors (dtype, H, W, C, ld, halo).
"""
import numpy as np

import pyoracle as O

DT = {0: np.float32, 1: np.float16, 2: np.int8, 3: np.int32}
OP_FE_LOGMEL, OP_STEM, OP_DW3, OP_DWK, OP_PAD, OP_MEAN = 8, 9, 4, 10, 11, 12
OP_SE, OP_SE_GATE, OP_PW_S8, OP_GEMV_S8, OP_PROTO_S8 = 5, 25, 22, 23, 35


class OracleNet:
    def __init__(self, net, in_buf, out_buf, emb_buf=None):
        self.net, self.in_buf, self.out_buf, self.emb_buf = net, in_buf, out_buf, emb_buf
        self.T = [a for (_, a, _) in net.pkg.tensors]

    def t(self, i):
        return self.T[i]

    def run(self, pcm, upto=None):
        """Returns (out, emb, bufs) for one window; upto stops after that many ops."""
        net = self.net
        bufs = [np.zeros(d[6], DT[d[0]]) for d in net.bufs]
        bufs[self.in_buf][:] = np.asarray(pcm, np.float32).reshape(-1)
        for n, (code, b, t, p) in enumerate(net.ops):
            if upto is not None and n >= upto:
                break
            base, var = code & 0xff, code >> 8
            getattr(self, f"op_{base}")(var, b, [self.t(i) for i in t], p, bufs)
        emb = None if self.emb_buf is None else bufs[self.emb_buf]
        return bufs[self.out_buf], emb, bufs

    def desc(self, i):
        d = self.net.bufs[i]
        return dict(dtype=d[0], H=d[1], W=d[2], C=d[3], ld=d[4], halo=d[5], elems=d[6])

    @staticmethod
    def put(dst, a):
        a = np.asarray(a).reshape(-1)
        dst[:a.size] = a

    # FE_LOGMEL
    def op_8(self, var, b, t, p, bufs):
        nsamp, frame, hop, pad, nfft, nmel = p
        spec = O.logmel(bufs[b[0]][:nsamp], frame, hop, pad, nfft, t[0], t[1].reshape(nmel, -1), t[2][0], t[2][1])
        self.put(bufs[b[1]], spec)

    # STEM
    def op_9(self, var, b, t, p, bufs):
        N, K, Kp, Np, H, W, Ho, Wo, k, s, act, ldo, opad = p
        out = O.stem_f32(bufs[b[0]][:H * W].reshape(H, W), k, s, t[0], t[1], Kp, Np, act=act, opad=opad, ldo=ldo)
        self.put(bufs[b[1]], out)

    # DW3 (fp32)
    def op_4(self, var, b, t, p, bufs):
        assert var == 0
        H, W, C, s, Ho, Wo = p[:6]
        out, cs = O.dw3_f32(bufs[b[0]][:(H + 2) * (W + 2) * C], H, W, C, s, t[0], t[1], Ho, Wo)
        self.put(bufs[b[1]], out)
        self.put(bufs[b[2]], cs)

    # DWK (fp32)
    def op_10(self, var, b, t, p, bufs):
        assert var == 0
        H, W, C, k, s, pt, pl, Ho, Wo, act = p
        h = (k - 1) // 2
        out, cs = O.dwk_f32(bufs[b[0]][:(H + 2 * h) * (W + 2 * h) * C], H, W, C, k, s, pt, pl, t[0], t[1], act, Ho,
                            Wo)
        self.put(bufs[b[1]], out)
        self.put(bufs[b[2]], cs)

    # PAD
    def op_11(self, var, b, t, p, bufs):
        H, W, C, ld, h = p
        self.put(bufs[b[1]], O.pad(bufs[b[0]][:H * W * ld].reshape(H * W, ld), H, W, C, h))

    # MEAN
    def op_12(self, var, b, t, p, bufs):
        P_, C, ld = p
        self.put(bufs[b[1]], O.mean_f32(bufs[b[0]][:P_ * ld].reshape(P_, ld), C))

    # SE_GATE
    def op_25(self, var, b, t, p, bufs):
        C, rd, P_ = p
        self.put(bufs[b[1]], O.se_gate_f32(bufs[b[0]][:C], P_, t[0].reshape(rd, C), t[1], t[2], t[3]))

    # SE (in place)
    def op_5(self, var, b, t, p, bufs):
        C, rd, P_ = p
        g = O.se_gate_f32(bufs[b[1]][:C], P_, t[0].reshape(rd, C), t[1], t[2], t[3])
        D = bufs[b[0]][:P_ * C].reshape(P_, C)
        bufs[b[0]][:P_ * C] = (D * g[None, :]).reshape(-1)

    # PW_S8
    def op_22(self, var, b, t, p, bufs):
        N, K, Kp, Np, M, lda, act, ldo, ow, opad, ldr = p
        pk = dict(q=t[0], sw=t[1], cs=t[2], b=t[3], shape=(N, K, Kp, Np))
        o = self.desc(b[1])
        res = None
        rpad = rw = 0
        if b[2] >= 0:
            r = self.desc(b[2])
            res = bufs[b[2]]
            rpad, rw = r["halo"], r["W"]
        gate = bufs[b[6]] if len(b) > 6 and b[6] >= 0 else None
        out_rows = o["elems"] // ldo
        out, q, sa, za = O.pw_s8(bufs[b[0]][:M * lda].reshape(M, lda), pk, act=act, out_rows=out_rows, ldo=ldo,
                                 ow=ow, opad=opad, res=res, ldr=ldr, rpad=rpad, rw=rw, gate=gate)
        self.put(bufs[b[1]], out)

    # GEMV_S8
    def op_23(self, var, b, t, p, bufs):
        N, K, Kp, Np, act = p
        pk = dict(q=t[0], sw=t[1], cs=t[2], b=t[3], shape=(N, K, Kp, Np))
        out, *_ = O.pw_s8(bufs[b[0]][:K].reshape(1, K), pk, act=act, ldo=Np)
        self.put(bufs[b[1]], out)
