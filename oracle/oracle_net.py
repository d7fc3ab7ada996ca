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
OP_PW, OP_GEMV = 3, 15


def unpack_h16(panels, N, Kp, Np):
    """fp16 weights [N][Kp] from hp_pack's panels [Np/16][Kp][16] + tail [Kp][8] (src/gemm_f16.c:18-40)."""
    panels = np.asarray(panels).view(np.float16).reshape(-1)
    n16 = Np // 16
    W = np.zeros((Np, Kp), np.float16)
    W[:n16 * 16] = panels[:n16 * Kp * 16].reshape(n16, Kp, 16).transpose(0, 2, 1).reshape(n16 * 16, Kp)
    if Np % 16:
        W[n16 * 16:] = panels[n16 * Kp * 16:n16 * Kp * 16 + Kp * 8].reshape(Kp, 8).T
    return W[:N]


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

    # STEM (variant 1: fp32 math, fp16 output)
    def op_9(self, var, b, t, p, bufs):
        N, K, Kp, Np, H, W, Ho, Wo, k, s, act, ldo, opad = p
        img = bufs[b[0]][:H * W].reshape(H, W)
        if var == 1:
            out = O.stem_f32to16(img, k, s, t[0], t[1], Kp, N, Np, act=act, opad=opad, ldo=ldo)
        else:
            out = O.stem_f32(img, k, s, t[0], t[1], Kp, Np, act=act, opad=opad, ldo=ldo)
        self.put(bufs[b[1]], out)

    # DW3 (variant 1: fp16 with TF-same offsets)
    def op_4(self, var, b, t, p, bufs):
        H, W, C, s, Ho, Wo = p[:6]
        xp = bufs[b[0]][:(H + 2) * (W + 2) * C]
        if var == 1:
            out, cs = O.dw3_f16(xp, H, W, C, s, p[6], p[7], t[0], t[1], Ho, Wo)
        else:
            out, cs = O.dw3_f32(xp, H, W, C, s, t[0], t[1], Ho, Wo)
        self.put(bufs[b[1]], out)
        self.put(bufs[b[2]], cs)

    # DWK (variant 1: fp16)
    def op_10(self, var, b, t, p, bufs):
        H, W, C, k, s, pt, pl, Ho, Wo, act = p
        h = (k - 1) // 2
        xp = bufs[b[0]][:(H + 2 * h) * (W + 2 * h) * C]
        f = O.dwk_f16 if var == 1 else O.dwk_f32
        out, cs = f(xp, H, W, C, k, s, pt, pl, t[0], t[1], act, Ho, Wo)
        self.put(bufs[b[1]], out)
        self.put(bufs[b[2]], cs)

    # PW (variant 0: the fp32 GEMM, optional gate b[3]; variant 1: the fp16 GEMM)
    def op_3(self, var, b, t, p, bufs):
        N, K, Kp, Np, M, lda, act, ldo, ow, opad, ldr = p
        if var == 0:
            rd = None if b[2] < 0 else self.desc(b[2])
            res = None if b[2] < 0 else bufs[b[2]]
            gate = bufs[b[3]][:K] if len(b) == 4 and b[3] >= 0 else None
            out = O.gemm_f32(bufs[b[0]][:M * lda].reshape(M, lda), np.asarray(t[0], np.float32),
                             np.asarray(t[1], np.float32), Kp, Np, act=act, gate=gate, res=res, ldr=ldr,
                             rpad=rd["halo"] if rd else 0, rw=rd["W"] if rd else 0, ow=ow if opad else 0, opad=opad,
                             ldo=ldo)
            self.put(bufs[b[1]], out)
            return
        assert var == 1
        W = unpack_h16(t[0], N, Kp, Np)
        res = None if b[2] < 0 else bufs[b[2]][:M * ldr].reshape(M, ldr)
        out = O.gemm_f16(bufs[b[0]][:M * lda].reshape(M, lda), W, t[1][:N], act=act, ldo=ldo, ow=ow, opad=opad,
                         res=res, b16=np.asarray(t[2]).view(np.float16)[:Np])
        self.put(bufs[b[1]], out)

    # STEM3 (variant 2): the 3-channel image's stride-2 conv into 24 fp16 channels
    def op_26(self, var, b, t, p, bufs):
        H, W, Ho, Wo = p
        img = bufs[b[0]][:H * W * 3].reshape(H, W, 3)
        self.put(bufs[b[1]], O.stem3(img, np.asarray(t[0], np.float32), np.asarray(t[1], np.float32)))

    # CONV3C24 (variant 2): the fp16 Winograd of src/wino_s0.c, residual = its own input, zero-haloed output
    def op_27(self, var, b, t, p, bufs):
        H, W = p
        xp = bufs[b[0]][:(H + 2) * (W + 2) * 24].reshape(H + 2, W + 2, 24)
        w = np.asarray(t[0], np.float32).reshape(24, 3, 3, 24)
        self.put(bufs[b[1]], O.wino_s0(xp, w, np.asarray(t[1], np.float32)))

    # UNPAD (variant 2): the haloed fp16 interior widened to fp32 rows
    def op_28(self, var, b, t, p, bufs):
        H, W, C = p
        xp = bufs[b[0]][:(H + 2) * (W + 2) * C].reshape(H + 2, W + 2, C)
        self.put(bufs[b[1]], xp[1:-1, 1:-1].astype(np.float32))

    # WINO_S8 (variant 2): the int8 Winograd of src/wino.c
    def op_29(self, var, b, t, p, bufs):
        H, W, C, K = p
        w = np.asarray(t[0], np.float32).reshape(K, 3, 3, C)
        self.put(bufs[b[1]], O.wino8(bufs[b[0]][:H * W * C].reshape(H, W, C), O.wino8_pack(w), t[1]))

    # PROTO variant 2 (the dotprod head): buffers [cells f16, logits, qa, colmax], tensors [qw 12-panels, sw, clsw,
    # clsb, eps]
    # PROTO variants 0 (fp32) and 1 (fp16): buffers [cells, logits, a, colmax], tensors [panels, bias (fp16: b32, b16),
    # clsw, clsb, eps]
    def op_13(self, var, b, t, p, bufs):
        if var in (0, 1):
            N, K, Kp, Np, P_, C, ld, nc, ppc = p
            x = bufs[b[0]][:P_ * ld].reshape(P_, ld)
            ct = 2 if var == 0 else 3
            rc, lg, cm, a = O.proto_fp("f32" if var == 0 else "f16", x, C, float(np.asarray(t[ct + 2]).reshape(-1)[0]),
                                       t[0], Np, np.asarray(t[ct]).reshape(-1), t[ct + 1], nc, ppc)
            self.put(bufs[b[1]], lg)
            self.put(bufs[b[2]], a.view(np.float16) if var == 1 else a)
            self.put(bufs[b[3]], cm)
            return
        assert var == 2
        N, K, Np, P_, C, ld, nc, ppc = p
        x = bufs[b[0]][:P_ * ld].reshape(P_, ld)
        rc, lg, cm = O.proto_s8_dot(x, C, float(np.asarray(t[4]).reshape(-1)[0]), t[0], t[1][:Np], Np,
                                    np.asarray(t[2]).reshape(-1), t[3], nc, ppc)
        self.put(bufs[b[1]], lg)
        self.put(bufs[b[3]], cm)

    # PROTO_F32H: buffers [cells f32, logits, a, colmax], tensors [fp16 panels [Np/8][K][8], clsw, clsb, eps]
    def op_14(self, var, b, t, p, bufs):
        N, K, Np, P_, C, ld, nc, ppc = p
        x = bufs[b[0]][:P_ * ld].reshape(P_, ld)
        rc, lg, cm, a = O.proto_fp("f32h", x, C, float(np.asarray(t[3]).reshape(-1)[0]), t[0], Np,
                                   np.asarray(t[1]).reshape(-1), t[2], nc, ppc)
        self.put(bufs[b[1]], lg)
        self.put(bufs[b[2]], a)
        self.put(bufs[b[3]], cm)

    # QCONV3: x f32 [H][W][C] -> fp16 rows
    def op_30(self, var, b, t, p, bufs):
        H, W, C, K, s, Ho, Wo = p
        pk = O.qd_wpack(np.asarray(t[0], np.float32).reshape(K, 9 * C), t[1])
        self.put(bufs[b[1]], O.qconv3(bufs[b[0]][:H * W * C].reshape(H, W, C), pk, s))

    # QPW: buffers [in, out, a8, rq, res | -1, gate | -1]
    def op_31(self, var, b, t, p, bufs):
        N, K, M, idt, ldx, act, odt, ldo, ow, opad = p
        pk = O.qd_wpack(np.asarray(t[0], np.float32).reshape(N, K), t[1])
        x = bufs[b[0]][:M * ldx].reshape(M, ldx)
        res = None if b[4] < 0 else bufs[b[4]][:M * ldo].reshape(M, ldo)
        gate = None if b[5] < 0 else bufs[b[5]][:K]
        out, a8, rq = O.qpw(x, pk, act, out16=odt == 1, ldo=ldo, ow=ow, opad=opad, res=res, gate=gate)
        self.put(bufs[b[1]], out)
        self.put(bufs[b[2]], a8)
        self.put(bufs[b[3]], rq)

    # SE_GATE16: buffers [chsum (scaled in place), gate]
    def op_32(self, var, b, t, p, bufs):
        C, rd, P_ = p
        m, g = O.se_gate16(bufs[b[0]][:C], P_, np.asarray(t[0]).reshape(rd, C), t[1], np.asarray(t[2]).reshape(C, rd),
                           t[3])
        self.put(bufs[b[0]], m)
        self.put(bufs[b[1]], g)

    # GEM_A
    def op_33(self, var, b, t, p, bufs):
        M, C = p
        k = np.asarray(t[0], np.float32).reshape(-1)
        self.put(bufs[b[1]], O.gem_a(bufs[b[0]][:M * C].reshape(M, C), k[0], k[1]))

    # HEADS_S8: buffers [F, e, logits, a8, rq]
    def op_34(self, var, b, t, p, bufs):
        H, W, C, hid, nc = p
        ncp = (nc + 15) // 16 * 16
        T = [np.asarray(a, np.float32) for a in t]
        packs = [O.qd_wpack(T[0].reshape(nc, C), T[1], ncp)]
        for i in range(2):
            j = 2 + 6 * i
            packs += [O.qd_wpack(T[j].reshape(hid, C), T[j + 1]), O.qd_wpack(T[j + 2].reshape(nc, hid), T[j + 3], ncp),
                      O.qd_wpack(T[j + 4].reshape(nc, hid), T[j + 5], ncp)]
        self.put(bufs[b[2]], O.heads_s8(bufs[b[0]][:H * W * C].reshape(H * W, C), bufs[b[1]][:C], H, W, packs))

    # PROTO_S8: buffers [cells, logits, q, colmax], tensors [q panels, sw, n4, clsw, clsb, eps]
    def op_35(self, var, b, t, p, bufs):
        N, K, Kp, Np, P_, C, ld, nc, ppc = p
        x = bufs[b[0]][:P_ * ld].reshape(P_, ld)
        rc, lg, cm, _ = O.proto_s8(x, C, float(np.asarray(t[5]).reshape(-1)[0]), t[0], t[1][:Np], Np, Kp,
                                   np.asarray(t[3]).reshape(-1), t[4], nc, ppc)
        self.put(bufs[b[1]], lg)
        self.put(bufs[b[3]], cm)

    # GEMV (variant 0: fp32 weights, 1: fp16 weights)
    def op_15(self, var, b, t, p, bufs):
        N, K, act = p
        w = np.asarray(t[0]).view(np.float16 if var == 1 else np.float32).reshape(N, K)
        self.put(bufs[b[1]], O.gemv(w, t[1], bufs[b[0]][:K], act))

    # PAD
    def op_11(self, var, b, t, p, bufs):
        H, W, C, ld, h = p
        self.put(bufs[b[1]], O.pad(bufs[b[0]][:H * W * ld].reshape(H * W, ld), H, W, C, h))

    # MEAN (variant 1: of fp16 rows)
    def op_12(self, var, b, t, p, bufs):
        P_, C, ld = p
        f = O.mean_f16 if var == 1 else O.mean_f32
        self.put(bufs[b[1]], f(bufs[b[0]][:P_ * ld].reshape(P_, ld), C))

    # SE_GATE
    def op_25(self, var, b, t, p, bufs):
        C, rd, P_ = p
        self.put(bufs[b[1]], O.se_gate_f32(bufs[b[0]][:C], P_, t[0].reshape(rd, C), t[1], t[2], t[3]))

    # SE (in place; variant 1: the fp16 path's)
    def op_5(self, var, b, t, p, bufs):
        C, rd, P_ = p
        if var == 1:
            D = bufs[b[0]][:P_ * C].reshape(P_, C)
            bufs[b[0]][:P_ * C] = O.se_f16(D, bufs[b[1]][:C], t[0].reshape(rd, C), t[1], t[2], t[3]).reshape(-1)
            return
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
