"""Builds .bnpk packages of synthetic networks from int8 / fp32 / fp16 ops.

The op records are the ones libbnneon's compiler emits for these layers
(python/bnneon/compiler/lower.py: pw :787-823 with s8_tensors :883-914,
l_dwconv :916-951; the PROTO_S8 and GEMV_S8 records of src/rt_ops_s8n.c:92-253),
so a package built here is a valid package for the reference library too.
Every buffer gets its own memory slot (no lifetime sharing): simple and safe.
"""
import hashlib

import numpy as np

from . import pkgfmt, s8pack

F32, F16, I8, I32 = 0, 1, 2, 3
HW_FP16 = 1
OP = {"PW": 3, "DW3": 4, "SE": 5, "FE_LOGMEL": 8, "STEM": 9, "DWK": 10, "PROTO": 13,
      "PAD": 11, "MEAN": 12, "GEMV": 15, "PW_S8": 22, "GEMV_S8": 23,
      "SE_GATE": 25, "STEM3": 26, "CONV3C24": 27, "UNPAD": 28, "WINO_S8": 29, "QCONV3": 30, "QPW": 31,
      "SE_GATE16": 32, "GEM_A": 33, "HEADS_S8": 34, "PROTO_S8": 35, "PROTO_F32H": 14}
HW_DOTPROD = 2
ACT = {None: 0, "none": 0, "silu": 1, "relu": 2}


class Net:
    """One path of a package: buffers, op records and tensors."""

    def __init__(self, pkg=None, prefix=""):
        self.pkg = pkg or pkgfmt.Package()
        self.prefix = prefix
        self.bufs = []   # (dtype, H, W, C, ld, halo, elems, slot)
        self.ops = []
        self.k = 0
        self.last = None   # the output buffer of the last op emitted

    def buf(self, dtype, H, W, C, ld=None, halo=0, elems=None):
        ld = C if ld is None else ld
        if elems is None:
            elems = (H + 2 * halo) * (W + 2 * halo) * ld
        self.bufs.append((dtype, H, W, C, ld, halo, int(elems), len(self.bufs)))
        return len(self.bufs) - 1

    def tensor(self, name, a):
        self.k += 1
        return self.pkg.tensor(f"{self.prefix}{name}.{self.k}", a)

    def emit(self, code, b, t, p, var=0):
        self.ops.append((code | (var << 8), list(b), list(t), [int(x) for x in p]))

    # ---------------------------------------------------------------- int8 ops
    def pw_s8(self, ib, w, b, act=None, H=None, W=None, opad=0, res=-1, gate=-1):
        """A 1x1 conv on rows of buffer ib (NHWC, no halo): PW_S8."""
        d = self.bufs[ib]
        H = d[1] if H is None else H
        W = d[2] if W is None else W
        M, lda = H * W, d[4]
        pk = s8pack.pack_s8(np.asarray(w, np.float32), np.asarray(b, np.float32))
        N, K, Kp, Np = pk["shape"]
        tl = [self.tensor("s8n/pw.q", pk["q"]), self.tensor("s8n/pw.sw", pk["sw"]),
              self.tensor("s8n/pw.cs", pk["cs"]), self.tensor("s8n/pw.b", pk["b"])]
        ob = self.buf(F32, H, W, N, ld=Np, halo=opad)
        m4 = (M + 3) // 4 * 4
        qb = self.buf(I8, m4, 1, Kp)
        sb = self.buf(F32, m4, 1, 1)
        zb = self.buf(I32, m4, 1, 1)
        ldr = self.bufs[res][4] if res >= 0 else 0
        bl = [ib, ob, res, qb, sb, zb] + ([gate] if gate >= 0 else [])
        self.emit(OP["PW_S8"], bl, tl, [N, K, Kp, Np, M, lda, ACT[act], Np,
                                        W if opad else W, opad, ldr])
        self.last = ob
        return ob

    def gemv_s8(self, ib, w, b, act=None):
        pk = s8pack.pack_s8(np.asarray(w, np.float32), np.asarray(b, np.float32))
        N, K, Kp, Np = pk["shape"]
        tl = [self.tensor("s8n/lin.q", pk["q"]), self.tensor("s8n/lin.sw", pk["sw"]),
              self.tensor("s8n/lin.cs", pk["cs"]), self.tensor("s8n/lin.b", pk["b"])]
        ob = self.buf(F32, 1, 1, N, ld=Np, elems=Np)
        qb = self.buf(I8, 4, 1, Kp)
        sb = self.buf(F32, 4, 1, 1)
        zb = self.buf(I32, 4, 1, 1)
        self.emit(OP["GEMV_S8"], [ib, ob, qb, sb, zb], tl, [N, K, Kp, Np, ACT[act]])
        self.last = ob
        return ob

    def proto_s8(self, ib, protos, clsw, clsb, eps=1e-5, n4=None):
        """ProtoPNet head on cells [P][C] of buffer ib: int8 prototypes."""
        d = self.bufs[ib]
        P, C, ld = d[1] * d[2], d[3], d[4]
        protos = np.asarray(protos, np.float32)
        N, K = protos.shape
        Kp, Np = s8pack.r16(K), (N + 3) // 4 * 4
        q, sw = s8pack.quant_rows_s8(protos)
        qp = np.zeros((Np, Kp), np.int8)
        qp[:N, :K] = q
        swp = np.zeros(Np, np.float32)
        swp[:N] = sw
        flags = s8pack.n4_panel_flags(qp) if n4 is None else np.asarray(n4, np.int8)
        nc = len(clsb)
        ppc = N // nc
        tl = [self.tensor("s8n/proto.q", s8pack.pack_panels(qp)), self.tensor("s8n/proto.sw", swp),
              self.tensor("s8n/proto.n4", flags), self.tensor("proto.clsw", np.asarray(clsw, np.float32).reshape(nc, ppc)),
              self.tensor("proto.clsb", np.asarray(clsb, np.float32)), self.tensor("proto.eps", np.array([eps], np.float32))]
        ob = self.buf(F32, 1, 1, nc)
        qb = self.buf(I8, P, 1, Kp)
        cb = self.buf(F32, 1, 1, Np)
        self.emit(OP["PROTO_S8"], [ib, ob, qb, cb], tl, [N, K, Kp, Np, P, C, ld, nc, ppc])
        self.last = ob
        return ob

    def proto_fp(self, ib, protos, clsw, clsb, eps=1e-5, kind="f32"):
        """The fp32 / fp16 prototype heads on cells [P][C] of buffer ib (l_proto / emit_proto / proto_f32h,
        python/bnneon/compiler/lower.py:429-504): kind "f32" PROTO variant 0 (fp32 panels, zero bias, Kp = C),
        "f16" PROTO variant 1 (hpack panels; fp16 cells), "f32h" PROTO_F32H (fp16 panels [Np/8][K][8], fp32 cells).
        The record's buffers: cells, logits [nc], the normalised cells [P][C], column maxima [Np]."""
        d = self.bufs[ib]
        P, C, ld = d[1] * d[2], d[3], d[4]
        protos = np.asarray(protos, np.float32)
        N, K = protos.shape
        assert K == C and C % 8 == 0 and P % 8 == 0
        nc = len(clsb)
        ppc = N // nc
        Np = (N + 7) // 8 * 8
        cls = [self.tensor("cls.w", np.asarray(clsw, np.float32).reshape(nc, ppc)),
               self.tensor("cls.b", np.asarray(clsb, np.float32)), self.tensor("cls.eps", np.array([eps], np.float32))]
        if kind == "f32":
            panels, bb, shp = self.fpack(protos, np.zeros(N, np.float32), K_pad=8)
            tl = [self.tensor("proto.w", panels), self.tensor("proto.b", bb)] + cls
            code, var, ints, adt = OP["PROTO"], 0, list(shp) + [P, C, ld, nc, ppc], F32
        elif kind == "f16":
            w16, b32, b16, shp = self.pack_h16(protos, np.zeros(N, np.float32), K)
            tl = [self.tensor("proto.w", w16), self.tensor("proto.b32", b32), self.tensor("proto.b16", b16)] + cls
            code, var, ints, adt = OP["PROTO"], 1, list(shp) + [P, C, ld, nc, ppc], F16
        else:
            w16p = np.zeros((Np, C), np.float16)
            w16p[:N] = protos.astype(np.float16)
            wp = np.ascontiguousarray(w16p.reshape(Np // 8, 8, C).transpose(0, 2, 1))
            tl = [self.tensor("f32h/proto.w", wp)] + cls
            code, var, ints, adt = OP["PROTO_F32H"], 0, [N, C, Np, P, C, ld, nc, ppc], F32
        ob = self.buf(F32, 1, 1, nc)
        ab = self.buf(adt, P, 1, C)
        cb = self.buf(F32, 1, 1, Np)
        self.emit(code, [ib, ob, ab, cb], tl, ints, var=var)
        self.last = ob
        return ob

    # ---------------------------------------------------------------- fp16 path (variant 1)
    @staticmethod
    def pack_h16(w, b, k_pad):
        """pack_h16 (python/bnneon/compiler/lower.py:99-128; hp_pack, src/gemm_f16.c:18-40): fp16 panels
        [Np/16][Kp][16] + a tail [Kp][8] when Np % 16 == 8, the bias as fp32 and fp16 [Np + 16]."""
        w = np.asarray(w, np.float32)
        N, K = w.shape
        Np = (N + 7) // 8 * 8
        wp = np.zeros((Np, k_pad), np.float16)
        wp[:N, :K] = w
        n16 = Np // 16
        main = wp[:n16 * 16].reshape(n16, 16, k_pad).transpose(0, 2, 1).reshape(-1)
        tail = wp[n16 * 16:].T.reshape(-1) if Np % 16 else np.zeros(0, np.float16)
        b32 = np.zeros(Np + 16, np.float32)
        b32[:N] = b
        return np.concatenate([main, tail]), b32, b32.astype(np.float16), (N, K, k_pad, Np)

    def pw_f16(self, ib, w, b, act=None, opad=0, res=-1, ldo=None):
        """A 1x1 conv on fp16 rows of buffer ib (the fp16 path's PW, lower.py:787-823)."""
        d = self.bufs[ib]
        H, W, M, lda = d[1], d[2], d[1] * d[2], d[4]
        w = np.asarray(w, np.float32)
        K = w.shape[1]
        panels, b32, b16, (N, K, Kp, Np) = self.pack_h16(w, b, (K + 7) // 8 * 8)
        tl = [self.tensor("f16/pw.w", panels), self.tensor("f16/pw.b32", b32), self.tensor("f16/pw.b16", b16)]
        ldo = (N if opad else Np) if ldo is None else ldo
        ob = self.buf(F16, H, W, N, ld=ldo, halo=opad)
        ldr = self.bufs[res][4] if res >= 0 else 0
        self.emit(OP["PW"], [ib, ob, res], tl, [N, K, Kp, Np, M, lda, ACT[act], ldo, W, opad, ldr], var=1)
        self.last = ob
        return ob

    def stem_f16(self, ib, w, b, k, s, act="silu", opad=0, ldo=None):
        """The fp16 path's STEM (fp32 math, fp16 output, src/rt_ops_f16.c:167-180)."""
        d = self.bufs[ib]
        H, W = d[1], d[2]
        w = np.asarray(w, np.float32).reshape(len(b), k * k)
        co = w.shape[0]
        Ho, Wo = (H - k) // s + 1, (W - k) // s + 1
        Kp, Np = (k * k + 3) // 4 * 4, (co + 7) // 8 * 8
        wp = np.zeros((Np, Kp), np.float32)
        wp[:co, :k * k] = w
        panels = np.ascontiguousarray(wp.reshape(Np // 8, 8, Kp).transpose(0, 2, 1))
        bb = np.zeros(Np + 8, np.float32)
        bb[:co] = b
        tl = [self.tensor("f32/stem.w", panels), self.tensor("f32/stem.b", bb)]
        ldo = Np if ldo is None else ldo
        ob = self.buf(F16, Ho, Wo, co, ld=ldo, halo=opad)
        col = self.buf(F32, (Ho * Wo + 7) // 8 * 8, 1, Kp)
        tmp = self.buf(F32, Ho * Wo, 1, Np)
        self.emit(OP["STEM"], [ib, ob, col, tmp], tl, [co, k * k, Kp, Np, H, W, Ho, Wo, k, s, ACT[act], ldo, opad],
                  var=1)
        self.last = ob
        return ob

    def se_f16(self, ib, cs, w1, b1, w2, b2):
        """SE in place on the fp16 activation ib [P][C] (the fp16 path's SE)."""
        w1 = np.asarray(w1, np.float32)
        rd, C = w1.shape
        d = self.bufs[ib]
        tl = [self.tensor("se.w1", w1), self.tensor("se.b1", np.asarray(b1, np.float32)),
              self.tensor("se.w2t", np.ascontiguousarray(np.asarray(w2, np.float32).T)),
              self.tensor("se.b2", np.asarray(b2, np.float32))]
        self.emit(OP["SE"], [ib, cs], tl, [C, rd, d[1] * d[2]], var=1)
        return ib

    def mean_f16(self, ib):
        d = self.bufs[ib]
        assert not d[5]
        ob = self.buf(F32, 1, 1, d[3])
        self.emit(OP["MEAN"], [ib, ob], [], [d[1] * d[2], d[3], d[4]], var=1)
        self.last = ob
        return ob

    def gemv(self, ib, w, b, act=None, fp16=False):
        """Dense layer on a vector: GEMV (fp32 weights) or its fp16-weight form."""
        w = np.asarray(w, np.float32)
        N, K = w.shape
        tl = [self.tensor("lin.w", w.astype(np.float16 if fp16 else np.float32)),
              self.tensor("lin.b", np.asarray(b, np.float32))]
        ob = self.buf(F32, 1, 1, N)
        self.emit(OP["GEMV"], [ib, ob], tl, [N, K, ACT[act]], var=1 if fp16 else 0)
        self.last = ob
        return ob

    # ---------------------------------------------------------------- depthwise
    def dwk(self, ib, w, b, k, s=1, pt=None, pl=None, act="silu", fp16=False):
        """k x k depthwise conv (DWK) on the zero-haloed buffer ib (halo (k-1)/2,
        ld = C), TF-'same' pads by default; returns (out, chsum) buffers.
        w [k*k][C], b [C] (fp16 when fp16, else fp32): l_dwconv's record
        (python/bnneon/compiler/lower.py:916-951)."""
        d = self.bufs[ib]
        H, W, C = d[1], d[2], d[4]
        assert d[5] == (k - 1) // 2, "DWK input needs halo (k-1)/2"
        Ho, Wo = (H - 1) // s + 1, (W - 1) // s + 1
        if pt is None:
            pt = max((Ho - 1) * s + k - H, 0) // 2
        if pl is None:
            pl = max((Wo - 1) * s + k - W, 0) // 2
        dt, npdt = (F16, np.float16) if fp16 else (F32, np.float32)
        tl = [self.tensor("dw.w", np.asarray(w, npdt).reshape(k * k, C)),
              self.tensor("dw.b", np.asarray(b, npdt).reshape(C))]
        ob = self.buf(dt, Ho, Wo, C)
        cb = self.buf(F32, 1, 1, C)
        self.emit(OP["DWK"], [ib, ob, cb], tl, [H, W, C, k, s, pt, pl, Ho, Wo, ACT[act]], var=1 if fp16 else 0)
        self.last = ob
        return ob, cb

    def dw3(self, ib, w, b, s=1, pt=1, pl=1, fp16=False):
        """3 x 3 depthwise + SiLU (DW3) on the halo-1 buffer ib; the fp32 form
        has pads 1, the fp16 form takes pt, pl in {0, 1}."""
        d = self.bufs[ib]
        H, W, C = d[1], d[2], d[4]
        assert d[5] == 1
        if fp16:
            Ho, Wo = (H - 1) // s + 1, (W - 1) // s + 1
        else:
            Ho, Wo = (H + 2 - 3) // s + 1, (W + 2 - 3) // s + 1
        dt, npdt = (F16, np.float16) if fp16 else (F32, np.float32)
        tl = [self.tensor("dw3.w", np.asarray(w, npdt).reshape(9, C)),
              self.tensor("dw3.b", np.asarray(b, npdt).reshape(C))]
        ob = self.buf(dt, Ho, Wo, C)
        cb = self.buf(F32, 1, 1, C)
        p = [H, W, C, s, Ho, Wo] + ([pt, pl] if fp16 else [])
        self.emit(OP["DW3"], [ib, ob, cb], tl, p, var=1 if fp16 else 0)
        self.last = ob
        return ob, cb

    # ---------------------------------------------------------------- fp32 ops
    def logmel(self, ib, nsamp, frame, hop, pad, nfft, window, mel, floor_, scale):
        """FE_LOGMEL on the pcm buffer ib (l_fe_logmel, python/bnneon/compiler/lower.py:390-413): spec
        [nfr][nmel] as an (nfr, nmel, 1) buffer."""
        mel = np.asarray(mel, np.float32)
        nmel = mel.shape[0]
        assert mel.shape[1] == nfft // 2 + 1
        nfr = (nsamp + 2 * pad - frame) // hop + 1
        tl = [self.tensor("fe/window", np.asarray(window, np.float32)), self.tensor("fe/mel", mel),
              self.tensor("fe/consts", np.array([floor_, scale], np.float32))]
        ob = self.buf(F32, nfr, nmel, 1)
        self.emit(OP["FE_LOGMEL"], [ib, ob], tl, [nsamp, frame, hop, pad, nfft, nmel])
        self.last = ob
        return ob

    @staticmethod
    def fpack(w, b, K_pad=4):
        """fp_pack (src/gemm_f32.c:22-35): w [N][K] -> panels [Np/8][Kp][8] (Kp = K rounded up to 4), bias [Np + 8]."""
        w = np.asarray(w, np.float32)
        N, K = w.shape
        Kp, Np = (K + K_pad - 1) // K_pad * K_pad, (N + 7) // 8 * 8
        wp = np.zeros((Np, Kp), np.float32)
        wp[:N, :K] = w
        panels = np.ascontiguousarray(wp.reshape(Np // 8, 8, Kp).transpose(0, 2, 1))
        bb = np.zeros(Np + 8, np.float32)
        bb[:N] = b
        return panels, bb, (N, K, Kp, Np)

    def pw(self, ib, w, b, act=None, H=None, W=None, opad=0, res=-1, gate=-1):
        """A 1x1 conv in fp32 (PW, variant 0; the projections the reference's default int8 policy keeps in fp32,
        lower.py:874-881): fp32 panels; the input buffer grows to whole 8-row tiles (rt_pw_check)."""
        d = self.bufs[ib]
        H = d[1] if H is None else H
        W = d[2] if W is None else W
        M, lda = H * W, d[4]
        panels, bb, (N, K, Kp, Np) = self.fpack(w, b)
        assert lda >= Kp, "the input rows must hold Kp channels"
        mr = (M + 7) // 8 * 8
        if d[6] < mr * lda:
            self.bufs[ib] = d[:6] + (mr * lda,) + d[7:]
        tl = [self.tensor("f32/pw.w", panels), self.tensor("f32/pw.b", bb)]
        ob = self.buf(F32, H, W, N, ld=Np, halo=opad)
        ldr = self.bufs[res][4] if res >= 0 else 0
        bl = [ib, ob, res] + ([gate] if gate >= 0 else [])
        self.emit(OP["PW"], bl, tl, [N, K, Kp, Np, M, lda, ACT[act], Np, W, opad, ldr])
        self.last = ob
        return ob

    def stem(self, ib, w, b, k, s, act="silu", opad=0, ldo=None):
        """k x k VALID conv of stride s on the 1-channel image ib (stem, lower.py:760-785): fp32 panels
        [Np/8][Kp][8], Kp = k*k rounded up to 4; output [Ho][Wo][ldo] with halo opad."""
        d = self.bufs[ib]
        H, W = d[1], d[2]
        w = np.asarray(w, np.float32).reshape(len(b), k * k)
        co = w.shape[0]
        Ho, Wo = (H - k) // s + 1, (W - k) // s + 1
        Kp, Np = (k * k + 3) // 4 * 4, (co + 7) // 8 * 8
        wp = np.zeros((Np, Kp), np.float32)
        wp[:co, :k * k] = w
        panels = np.ascontiguousarray(wp.reshape(Np // 8, 8, Kp).transpose(0, 2, 1))
        bb = np.zeros(Np + 8, np.float32)
        bb[:co] = b
        tl = [self.tensor("f32/stem.w", panels), self.tensor("f32/stem.b", bb)]
        ldo = Np if ldo is None else ldo
        ob = self.buf(F32, Ho, Wo, co, ld=ldo, halo=opad)
        col = self.buf(F32, (Ho * Wo + 7) // 8 * 8, 1, Kp)
        self.emit(OP["STEM"], [ib, ob, col], tl, [co, k * k, Kp, Np, H, W, Ho, Wo, k, s, ACT[act], ldo, opad])
        self.last = ob
        return ob

    def se_gate(self, cs, P, w1, b1, w2, b2):
        """SE_GATE from the channel sums cs of P pixels (l_se, lower.py:981-1015): w1 [rd][C], w2 [C][rd];
        returns the gate buffer (f32 [C]) a 1x1 conv applies to its input."""
        w1 = np.asarray(w1, np.float32)
        rd, C = w1.shape
        tl = [self.tensor("se.w1", w1), self.tensor("se.b1", np.asarray(b1, np.float32)),
              self.tensor("se.w2t", np.ascontiguousarray(np.asarray(w2, np.float32).T)),
              self.tensor("se.b2", np.asarray(b2, np.float32))]
        gb = self.buf(F32, 1, 1, C, elems=C)
        self.emit(OP["SE_GATE"], [cs, gb], tl, [C, rd, P])
        return gb

    def se(self, ib, cs, w1, b1, w2, b2):
        """SE in place on the activation ib [P][C] (its channel sums cs)."""
        w1 = np.asarray(w1, np.float32)
        rd, C = w1.shape
        d = self.bufs[ib]
        tl = [self.tensor("se.w1", w1), self.tensor("se.b1", np.asarray(b1, np.float32)),
              self.tensor("se.w2t", np.ascontiguousarray(np.asarray(w2, np.float32).T)),
              self.tensor("se.b2", np.asarray(b2, np.float32))]
        self.emit(OP["SE"], [ib, cs], tl, [C, rd, d[1] * d[2]])
        return ib

    def mean(self, ib):
        """MEAN of rows ib [P][ld] -> f32 [C] (l_mean, lower.py:415-427)."""
        d = self.bufs[ib]
        assert not d[5]
        ob = self.buf(F32, 1, 1, d[3])
        self.emit(OP["MEAN"], [ib, ob], [], [d[1] * d[2], d[3], d[4]])
        self.last = ob
        return ob

    def pad(self, ib, h):
        """PAD of rows ib into a zero-haloed buffer with ld = C (dw_input, lower.py:967-974)."""
        d = self.bufs[ib]
        pb = self.buf(d[0], d[1], d[2], d[3], ld=d[3], halo=h)
        self.emit(OP["PAD"], [ib, pb], [], [d[1], d[2], d[3], d[4], h], var=1 if d[0] == F16 else 0)
        self.last = pb
        return pb

    # ---------------------------------------------------------------- the dotprod + fp16 family (variant 2)
    def stem3(self, ib, w, b):
        """STEM3 (src/rt_ops_dot.c:46-61): the 3-channel fp32 image ib [H][W][3] (H, W even) -> zero-haloed fp16
        [H/2][W/2][24] = SiLU(3 x 3 stride-2 conv + b); w OHWI fp32 [24][3][3][3]."""
        d = self.bufs[ib]
        H, W = d[1], d[2]
        assert d[0] == F32 and d[3] == 3 and d[4] == 3 and d[5] == 0
        tl = [self.tensor("dot/stem3.w", np.asarray(w, np.float32).reshape(24, 3, 3, 3)),
              self.tensor("dot/stem3.b", np.asarray(b, np.float32).reshape(24))]
        ob = self.buf(F16, H // 2, W // 2, 24, halo=1)
        self.emit(OP["STEM3"], [ib, ob], tl, [H, W, H // 2, W // 2], var=2)
        self.last = ob
        return ob

    def wino_s8(self, ib, w, b):
        """WINO_S8 (src/rt_ops_dot.c:130-170): x f32 rows [H][W][C] -> fp16 rows [H][W][K] = SiLU(3 x 3 conv + b)
        through the int8 Winograd; w OHWI fp32 [K][3][3][C]."""
        d = self.bufs[ib]
        H, W, C = d[1], d[2], d[3]
        assert d[0] == F32 and d[4] == C and d[5] == 0
        w = np.asarray(w, np.float32)
        K = w.shape[0]
        tl = [self.tensor("dot/wino.w", w), self.tensor("dot/wino.b", np.asarray(b, np.float32).reshape(K))]
        ob = self.buf(F16, H, W, K)
        self.emit(OP["WINO_S8"], [ib, ob], tl, [H, W, C, K], var=2)
        self.last = ob
        return ob

    def conv3c24(self, ib, w, b):
        """CONV3C24 (src/rt_ops_dot.c:63-107): SiLU(3 x 3 conv + b) + x on the zero-haloed fp16 buffer ib of 24
        channels, into a zero-haloed buffer; w OHWI fp32 [24][3][3][24]."""
        d = self.bufs[ib]
        H, W = d[1], d[2]
        assert d[0] == F16 and d[3] == 24 and d[4] == 24 and d[5] == 1
        tl = [self.tensor("dot/c24.w", np.asarray(w, np.float32).reshape(24, 3, 3, 24)),
              self.tensor("dot/c24.b", np.asarray(b, np.float32).reshape(24))]
        ob = self.buf(F16, H, W, 24, halo=1)
        self.emit(OP["CONV3C24"], [ib, ob], tl, [H, W], var=2)
        self.last = ob
        return ob

    def unpad(self, ib):
        """UNPAD (src/rt_ops_dot.c:109-128): the interior of a zero-haloed fp16 buffer as fp32 rows."""
        d = self.bufs[ib]
        H, W, C = d[1], d[2], d[3]
        assert d[0] == F16 and d[4] == C and d[5] == 1
        ob = self.buf(F32, H, W, C)
        self.emit(OP["UNPAD"], [ib, ob], [], [H, W, C], var=2)
        self.last = ob
        return ob

    def qconv3(self, ib, w, b, s):
        """QCONV3 (src/rt_ops_dot.c:173-216; conv3_s8, python/bnneon/compiler/lower_dot.py:192-223): fp32 rows
        [H][W][C] -> fp16 rows [Ho][Wo][K] = SiLU(3 x 3 stride-s TF-same conv + b) on per-tensor int8 inputs;
        w OHWI fp32 [K][3][3][C]."""
        d = self.bufs[ib]
        H, W, C = d[1], d[2], d[3]
        assert d[0] == F32 and d[4] == C and d[5] == 0
        w = np.asarray(w, np.float32)
        K = w.shape[0]
        Ho, Wo = (H + s - 1) // s, (W + s - 1) // s
        tl = [self.tensor("dot/qconv.w", w.reshape(K, 3, 3, C)),
              self.tensor("dot/qconv.b", np.asarray(b, np.float32).reshape(K))]
        ob = self.buf(F16, Ho, Wo, K)
        self.emit(OP["QCONV3"], [ib, ob], tl, [H, W, C, K, s, Ho, Wo], var=2)
        self.last = ob
        return ob

    def qpw(self, ib, w, b, act=None, gate=-1, res=-1, out16=False, opad=0):
        """QPW (src/rt_ops_dot.c:226-339; qpw, lower_dot.py:248-271): 1 x 1 conv of fp32 rows, or of fp16 rows
        (multiplied by an SE_GATE16 gate when one is given), with per-row int8 inputs; fp16 out (zero-haloed for a
        depthwise consumer when opad) or fp32 rows (+ the fp32 rows res); w [N][K]."""
        d = self.bufs[ib]
        idt, H, W, K, ldx = d[0], d[1], d[2], d[3], d[4]
        assert d[5] == 0 and idt in (F32, F16)
        w = np.asarray(w, np.float32)
        N = w.shape[0]
        M, Kp = H * W, (K + 15) // 16 * 16
        odt = F16 if out16 else F32
        ob = self.buf(odt, H, W, N, halo=opad)
        a8 = self.buf(I8, M + 4, 1, Kp)
        rq = self.buf(F32, M + 4, 1, 2)
        tl = [self.tensor("dot/qpw.w", w.reshape(N, K)), self.tensor("dot/qpw.b", np.asarray(b, np.float32))]
        self.emit(OP["QPW"], [ib, ob, a8, rq, res, gate], tl,
                  [N, K, M, idt, ldx, ACT[act], odt, N, W if opad else 0, opad], var=2)
        self.last = ob
        return ob

    def se_gate16(self, cs, P, w1, b1, w2, b2):
        """SE_GATE16 (src/rt_ops_dot.c:347-420): the fp16 gate [C] from the channel sums cs of P pixels (scaled to
        means in place); w1 [rd][C], w2 [C][rd] fp32."""
        w1 = np.asarray(w1, np.float32)
        rd, C = w1.shape
        tl = [self.tensor("dot/seg.w1", w1), self.tensor("dot/seg.b1", np.asarray(b1, np.float32)),
              self.tensor("dot/seg.w2", np.asarray(w2, np.float32).reshape(C, rd)),
              self.tensor("dot/seg.b2", np.asarray(b2, np.float32))]
        gb = self.buf(F16, 1, 1, C, elems=C)
        self.emit(OP["SE_GATE16"], [cs, gb], tl, [C, rd, P], var=2)
        return gb

    def gem_a(self, ib, eps, p):
        """GEM_A (src/rt_ops_dot.c:428-465): fp32 rows [M][C] -> the generalised mean [C]."""
        d = self.bufs[ib]
        assert d[0] == F32 and d[4] == d[3] and d[5] == 0
        M, C = d[1] * d[2], d[3]
        ob = self.buf(F32, 1, 1, C)
        self.emit(OP["GEM_A"], [ib, ob], [self.tensor("dot/gem.k", np.array([eps, p], np.float32))], [M, C],
                  var=2)
        self.last = ob
        return ob

    def heads_s8(self, fb, eb, H, W, lin, heads):
        """HEADS_S8 (src/rt_ops_dot.c:467-585): logits [ncp] = lin(e) + the SED heads over F fp32 rows [H*W][C];
        lin = (w [nc][C], b), heads = two (fc w [hid][C], fc b, att w [nc][hid], att b, cla w [nc][hid], cla b)."""
        d = self.bufs[fb]
        C = d[3]
        assert d[0] == F32 and d[4] == C and d[5] == 0 and d[1] * d[2] == H * W
        nc = np.asarray(lin[0]).shape[0]
        hid = np.asarray(heads[0][0]).shape[0]
        ncp, L = (nc + 15) // 16 * 16, max(H, W)
        tl = [self.tensor("dot/heads.lin.w", np.asarray(lin[0], np.float32)),
              self.tensor("dot/heads.lin.b", np.asarray(lin[1], np.float32))]
        for hd in heads:
            for j, a in enumerate(hd):
                tl.append(self.tensor(f"dot/heads.{j}", np.asarray(a, np.float32)))
        ob = self.buf(F32, 1, 1, ncp, elems=ncp)
        a8 = self.buf(I8, 1, 1, 1, elems=(L + 4) * max(C, hid))
        rq = self.buf(F32, 1, 1, 1, elems=2 * (L + 4))
        self.emit(OP["HEADS_S8"], [fb, eb, ob, a8, rq], tl, [H, W, C, hid, nc], var=2)
        self.last = ob
        return ob

    def proto_dot(self, ib, qw12, sw, clsw, clsb, eps=1e-5, C=None):
        """PROTO variant 2 (src/rt_ops_f16.c:252-281): the dotprod prototype head on the first C channels (all by
        default) of the fp16 cells ib [P][ld]; qw12 int8 [Np/12][C/4][12][4] prototype panels, sw [Np], clsw [nc][ppc],
        clsb [nc]."""
        d = self.bufs[ib]
        P, C, ld = d[1] * d[2], d[3] if C is None else C, d[4]
        assert d[0] == F16 and d[5] == 0
        clsw = np.asarray(clsw, np.float32)
        nc, ppc = clsw.shape
        N = nc * ppc
        sw = np.asarray(sw, np.float32)
        Np = sw.shape[0]
        tl = [self.tensor("dot/proto.qw", np.asarray(qw12, np.int8)), self.tensor("dot/proto.sw", sw),
              self.tensor("dot/proto.clsw", clsw), self.tensor("dot/proto.clsb", np.asarray(clsb, np.float32)),
              self.tensor("dot/proto.eps", np.array([eps], np.float32))]
        ob = self.buf(F32, 1, 1, nc)
        qb = self.buf(I8, P, 1, C)
        cb = self.buf(F32, 1, 1, Np)
        self.emit(OP["PROTO"], [ib, ob, qb, cb], tl, [N, C, Np, P, C, ld, nc, ppc], var=2)
        self.last = ob
        return ob

    def add_to(self, name="neon-int8", hwcap=0, in_buf=0, out_buf=None, emb_buf=None):
        self.pkg.add_path(name, hwcap, self.bufs, self.ops, in_buf,
                          self.last if out_buf is None else out_buf, emb_buf)


def standard_meta(pkg, n_samples, n_classes, sample_rate=32000, family=120,
                  model_id="synthetic", emb_dim=0, labels=None, post=1):
    pkg.set("format_version", 1)
    pkg.set("family", family)
    pkg.set("model_id", model_id)
    pkg.set("sample_rate", sample_rate)
    pkg.set("n_samples", n_samples)
    pkg.set("hop_samples", 0)
    pkg.set("n_classes", n_classes)
    pkg.set("post", post)
    pkg.set("emb_dim", emb_dim)
    pkg.set("license", "synthetic weights, no license")
    pkg.set("compiler", "bnneon.netbuild")
    if labels is not None:
        pkg.set("labels", labels)
        pkg.set("labels_sha256", hashlib.sha256(labels).digest())
