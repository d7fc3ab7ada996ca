"""ctypes loader of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: loaded by tests/ (as the checker), by
__graft_entry__.smoke() (as the checker) and by bench.py's cpu_baseline leg
(as the timed CPU restatement). The product path never imports it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(ORACLE_DIR, "liboracle.so")

vp = C.c_void_p
i32 = C.c_int
f32 = C.c_float


class OrcEpi32(C.Structure):
    _fields_ = [("act", i32), ("out", vp), ("ldo", i32), ("ow", i32),
                ("opad", i32), ("res", vp), ("ldr", i32), ("rpad", i32),
                ("rw", i32)]


_SIGS = {
    "orc_frecpe": (f32, [f32]),
    "orc_frecps": (f32, [f32, f32]),
    "orc_fmax": (f32, [f32, f32]),
    "orc_fmin": (f32, [f32, f32]),
    "orc_cvtn_s32": (i32, [f32]),
    "orc_cvta_s32": (i32, [f32]),
    "orc_lrintf_s32": (i32, [f32]),
    "orc_silu_f32": (f32, [f32]),
    "orc_eval_f32": (None, [i32, vp, vp, C.c_longlong]),
    "orc_s8n_quant_rows": (None, [vp, i32, i32, i32, i32, i32, vp, vp, vp]),
    "orc_s8n_quant_rows_gate": (None, [vp, i32, i32, i32, i32, i32, vp, vp,
                                       vp, vp]),
    "orc_s8n_gemm": (None, [vp, i32, vp, vp, i32, i32, vp, vp, vp, vp,
                            C.POINTER(OrcEpi32)]),
    "orc_pw_s8": (None, [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp,
                         vp, vp, vp, vp, C.POINTER(OrcEpi32)]),
    "orc_srdhm": (i32, [i32, i32]),
    "orc_rdbypot": (i32, [i32, i32]),
    "orc_requant": (C.c_int8, [i32, i32, i32, i32, i32, i32]),
    "orc_gemm_s8_requant": (None, [vp, vp, vp, vp, vp, i32, i32, i32, i32,
                                   i32, i32, i32, vp]),
}

_lib = None


def build():
    """Builds liboracle.so with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            build()
        L = C.CDLL(ORACLE_LIB)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name, None)
            if f is None:
                continue
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def P(a):
    """Host pointer of a numpy array (or None)."""
    return None if a is None else a.ctypes.data


def eval_f32(f, x):
    """orc_eval_f32 over an array: 0 FRECPE, 1 SiLU, 2 ReLU."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_eval_f32(f, P(x), P(y), x.size)
    return y


def vec_frecpe(x):
    f = lib().orc_frecpe
    return np.array([f(float(v)) for v in np.asarray(x, np.float32)],
                    np.float32)


def vec_silu(x):
    f = lib().orc_silu_f32
    return np.array([f(float(v)) for v in np.asarray(x, np.float32)],
                    np.float32)


def quant_rows(x, K, Kp, gate=None):
    """orc_s8n_quant_rows over all rows of x [M][ld] -> (q [M][Kp], sa, za)."""
    x = np.ascontiguousarray(x, np.float32)
    M, ld = x.shape
    q = np.zeros((M, Kp), np.int8)
    sa = np.zeros(M, np.float32)
    za = np.zeros(M, np.int32)
    if gate is None:
        lib().orc_s8n_quant_rows(P(x), ld, 0, M, K, Kp, P(q), P(sa), P(za))
    else:
        gate = np.ascontiguousarray(gate, np.float32)
        lib().orc_s8n_quant_rows_gate(P(x), ld, 0, M, K, Kp, P(gate), P(q),
                                      P(sa), P(za))
    return q, sa, za


def pw_s8(x, pk, act=0, out_rows=None, ldo=None, ow=0, opad=0, res=None,
          ldr=0, rpad=0, rw=0, gate=None):
    """The PW_S8 op of one window on the oracle.

    Args:
        x: f32 [M][lda] input rows.
        pk: s8pack.pack_s8 dict.
        out_rows: rows of the output buffer (M, or the padded pixel count).
    Returns:
        (out, q, sa, za) host arrays.
    """
    x = np.ascontiguousarray(x, np.float32)
    M, lda = x.shape
    N, K, Kp, Np = pk["shape"]
    ldo = ldo or Np
    M4 = (M + 3) // 4 * 4
    if out_rows is None:
        out_rows = M if not opad else (M // ow + 2 * opad) * (ow + 2 * opad)
    out = np.zeros((out_rows, ldo), np.float32)
    q = np.zeros((M4, Kp), np.int8)
    sa = np.zeros(M4, np.float32)
    za = np.zeros(M4, np.int32)
    res_a = None if res is None else np.ascontiguousarray(res, np.float32)
    e = OrcEpi32(act, out.ctypes.data, ldo, ow, opad, P(res_a), ldr, rpad, rw)
    g = None if gate is None else np.ascontiguousarray(gate, np.float32)
    lib().orc_pw_s8(P(x), lda, M, K, Kp, N, Np, P(g), P(q), P(sa), P(za),
                    P(pk["q"]), P(pk["sw"]), P(pk["cs"]), P(pk["b"]), C.byref(e))
    return out, q, sa, za


def gemm_s8_requant(w, x, bias, mult, shift, zx, zy, lo=-128, hi=127):
    w = np.ascontiguousarray(w, np.int8)
    x = np.ascontiguousarray(x, np.int8)
    N, K = w.shape
    M = x.shape[1]
    out = np.zeros((N, M), np.int8)
    b = np.ascontiguousarray(bias, np.int32)
    m = np.ascontiguousarray(mult, np.int32)
    s = np.ascontiguousarray(shift, np.int32)
    lib().orc_gemm_s8_requant(P(w), P(x), P(b), P(m), P(s), N, K, M, zx, zy,
                              lo, hi, P(out))
    return out


_SIGS.update({
    "orc_quant_cells_f32": (None, [vp, i32, i32, i32, f32, vp, i32, vp]),
    "orc_proto_n4_check": (i32, [vp, i32, vp, i32]),
    "orc_proto_colmax_s8n": (None, [vp, i32, vp, i32, vp, vp, i32, vp]),
    "orc_proto_logits": (i32, [vp, vp, vp, i32, i32, vp]),
    "orc_proto_s8": (i32, [vp, i32, i32, i32, f32, vp, i32, vp, vp, vp, i32, vp,
                           vp, vp, i32, i32, vp]),
})


def quant_cells(x, C, Kp, eps):
    """orc_quant_cells_f32 on x [P][ld] -> (qa [P][Kp], sx [P])."""
    x = np.ascontiguousarray(x, np.float32)
    P, ld = x.shape
    qa = np.zeros((P, Kp), np.int8)
    sx = np.zeros(P, np.float32)
    lib().orc_quant_cells_f32(x.ctypes.data, P, C, ld, eps, qa.ctypes.data, Kp, sx.ctypes.data)
    return qa, sx


def proto_s8(x, C, eps, qw, sw, Np, Kp, clsw, clsb, nc, ppc):
    """The PROTO_S8 op of one window -> (rc, logits, colmax, qa)."""
    x = np.ascontiguousarray(x, np.float32)
    Pn, ld = x.shape
    qa = np.zeros((Pn, Kp), np.int8)
    sx = np.zeros(Pn, np.float32)
    cm = np.zeros(Np, np.float32)
    lg = np.zeros(nc, np.float32)
    qw = np.ascontiguousarray(qw, np.int8)
    sw = np.ascontiguousarray(sw, np.float32)
    clsw = np.ascontiguousarray(clsw, np.float32)
    clsb = np.ascontiguousarray(clsb, np.float32)
    rc = lib().orc_proto_s8(x.ctypes.data, Pn, C, ld, eps, qa.ctypes.data, Kp, sx.ctypes.data,
                            qw.ctypes.data, sw.ctypes.data, Np, cm.ctypes.data, clsw.ctypes.data,
                            clsb.ctypes.data, nc, ppc, lg.ctypes.data)
    return rc, lg, cm, qa


def n4_check(qw, Kp, n4):
    qw = np.ascontiguousarray(qw, np.int8)
    n4 = np.ascontiguousarray(n4, np.uint8)
    return lib().orc_proto_n4_check(qw.ctypes.data, Kp, n4.ctypes.data, n4.size)


u16 = C.c_uint16
_SIGS.update({
    "orc_h2f": (f32, [u16]),
    "orc_h_fma": (u16, [u16, u16, u16]),
    "orc_h_add": (u16, [u16, u16]),
    "orc_h_mul": (u16, [u16, u16]),
    "orc_silu_lut_h": (u16, [u16]),
    "orc_dwk_f32": (None, [vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, i32, vp, i32, i32, vp]),
    "orc_dw3_f32": (None, [vp, i32, i32, i32, i32, vp, vp, vp, i32, i32, vp]),
    "orc_dwk_f16": (None, [vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, i32, vp, i32, i32, vp]),
    "orc_dw3_f16": (None, [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, i32, i32, vp]),
    "orc_dw_s8": (None, [vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, i32, i32, i32, i32, vp,
                         vp, i32, i32]),
})


def _c(a, dt):
    return np.ascontiguousarray(a, dt)


def dwk_f32(xp, H, W, C, k, s, pt, pl, w, b, act, Ho, Wo):
    """orc_dwk_f32 on a haloed input xp [(H+2h)][(W+2h)][C] -> (out, chsum)."""
    xp, w, b = _c(xp, np.float32), _c(w, np.float32), _c(b, np.float32)
    out = np.zeros((Ho, Wo, C), np.float32)
    cs = np.zeros(C, np.float32)
    lib().orc_dwk_f32(xp.ctypes.data, H, W, C, k, s, pt, pl, w.ctypes.data, b.ctypes.data, act,
                      out.ctypes.data, Ho, Wo, cs.ctypes.data)
    return out, cs


def dw3_f32(xp, H, W, C, s, w, b, Ho, Wo):
    xp, w, b = _c(xp, np.float32), _c(w, np.float32), _c(b, np.float32)
    out = np.zeros((Ho, Wo, C), np.float32)
    cs = np.zeros(C, np.float32)
    lib().orc_dw3_f32(xp.ctypes.data, H, W, C, s, w.ctypes.data, b.ctypes.data, out.ctypes.data, Ho, Wo,
                      cs.ctypes.data)
    return out, cs


def dwk_f16(xp, H, W, C, k, s, pt, pl, w, b, act, Ho, Wo):
    """fp16 arrays (numpy float16) in and out."""
    xp, w, b = _c(xp, np.float16), _c(w, np.float16), _c(b, np.float16)
    out = np.zeros((Ho, Wo, C), np.float16)
    cs = np.zeros(C, np.float32)
    lib().orc_dwk_f16(xp.ctypes.data, H, W, C, k, s, pt, pl, w.ctypes.data, b.ctypes.data, act,
                      out.ctypes.data, Ho, Wo, cs.ctypes.data)
    return out, cs


def dw3_f16(xp, H, W, C, s, pt, pl, w, b, Ho, Wo):
    xp, w, b = _c(xp, np.float16), _c(w, np.float16), _c(b, np.float16)
    out = np.zeros((Ho, Wo, C), np.float16)
    cs = np.zeros(C, np.float32)
    lib().orc_dw3_f16(xp.ctypes.data, H, W, C, s, pt, pl, w.ctypes.data, b.ctypes.data, out.ctypes.data,
                      Ho, Wo, cs.ctypes.data)
    return out, cs


def dw_s8(x, k, s, pt, pl, w, bias, mult, shift, zx, zy, lo, hi, lut, Ho, Wo):
    x = _c(x, np.int8)
    H, W, C = x.shape
    w, bias = _c(w, np.int8), _c(bias, np.int32)
    mult, shift = _c(mult, np.int32), _c(shift, np.int32)
    lut_a = None if lut is None else _c(lut, np.int8)
    out = np.zeros((Ho, Wo, C), np.int8)
    lib().orc_dw_s8(x.ctypes.data, H, W, C, k, s, pt, pl, w.ctypes.data, bias.ctypes.data, mult.ctypes.data,
                    shift.ctypes.data, zx, zy, lo, hi, None if lut_a is None else lut_a.ctypes.data,
                    out.ctypes.data, Ho, Wo)
    return out


class OrcEpi16(C.Structure):
    _fields_ = [("act", i32), ("out", vp), ("ldo", i32), ("ow", i32), ("opad", i32), ("res", vp), ("ldr", i32)]


_SIGS.update({
    "orc_f2h": (u16, [f32]),
    "orc_h_max": (u16, [u16, u16]),
    "orc_gemm_f16": (None, [vp, i32, i32, vp, i32, i32, vp, vp, C.POINTER(OrcEpi16)]),
})


def gemm_f16(A, W, b32, act=0, ldo=None, ow=0, opad=0, res=None, M=None, b16=None):
    """orc_gemm_f16: A fp16 [M][lda] (lda >= Kp), W fp16 [N][Kp] -> out fp16 rows [(padded) M][ldo]; b16 the
    fp16 bias (default: b32 rounded to nearest even)."""
    A = _c(A, np.float16)
    W = _c(W, np.float16)
    b32 = _c(b32, np.float32)
    b16 = b32.astype(np.float16) if b16 is None else _c(b16, np.float16)
    M = A.shape[0] if M is None else M
    lda = A.shape[1]
    N, Kp = W.shape
    Np = (N + 7) // 8 * 8
    ldo = ldo or Np
    rows = M if not opad else (M // ow + 2 * opad) * (ow + 2 * opad)
    out = np.zeros((rows, ldo), np.float16)
    r = None if res is None else _c(res, np.float16)
    e = OrcEpi16(act, out.ctypes.data, ldo, ow, opad, None if r is None else r.ctypes.data,
                 0 if r is None else r.shape[1])
    lib().orc_gemm_f16(A.ctypes.data, lda, M, W.ctypes.data, N, Kp, b32.ctypes.data, b16.ctypes.data, C.byref(e))
    return out


_SIGS.update({
    "orc_cvtz_s32": (i32, [f32]),
    "orc_wino8_pack": (None, [vp, i32, i32, vp, vp, vp]),
    "orc_wino8": (None, [vp, i32, i32, i32, i32, vp, vp, vp, vp, vp]),
})


def wino8_pack(w):
    """w OHWI fp32 [K][3][3][C] -> (U8 [16][K][C], sw [K], zw [4][K])."""
    w = _c(w, np.float32)
    K, C = w.shape[0], w.shape[3]
    U8 = np.zeros((16, K, C), np.int8)
    sw = np.zeros(K, np.float32)
    zw = np.zeros((4, K), np.float32)
    lib().orc_wino8_pack(w.ctypes.data, K, C, U8.ctypes.data, sw.ctypes.data, zw.ctypes.data)
    return U8, sw, zw


def wino8(x, pk, bias):
    """x f32 [H][W][C] -> fp16 [H][W][K] (the WINO_S8 op of one window)."""
    x = _c(x, np.float32)
    H, W, C = x.shape
    U8, sw, zw = pk
    K = U8.shape[1]
    b = _c(bias, np.float32)
    out = np.zeros((H, W, K), np.float16)
    lib().orc_wino8(x.ctypes.data, H, W, C, K, U8.ctypes.data, sw.ctypes.data, zw.ctypes.data, b.ctypes.data,
                    out.ctypes.data)
    return out


_SIGS.update({
    "orc_frecpe_h": (u16, [u16]),
    "orc_frecps_h": (u16, [u16, u16]),
    "orc_silu_poly_h": (u16, [u16]),
    "orc_wino_s0_pack": (None, [vp, vp, vp, vp]),
    "orc_wino_s0": (None, [vp, i32, i32, vp, vp, vp]),
})


def wino_s0(xp, w, b):
    """CONV3C24 of one window: xp fp16 [H+2][W+2][24] (zero halo) -> out fp16 [H+2][W+2][24] (zero halo)."""
    xp = _c(xp, np.float16)
    U = np.zeros(16 * 24 * 24, np.uint16)
    b16 = np.zeros(24, np.uint16)
    w = _c(w, np.float32)
    b = _c(b, np.float32)
    lib().orc_wino_s0_pack(w.ctypes.data, b.ctypes.data, U.ctypes.data, b16.ctypes.data)
    out = np.zeros_like(xp)
    lib().orc_wino_s0(xp.ctypes.data, xp.shape[0] - 2, xp.shape[1] - 2, U.ctypes.data, b16.ctypes.data,
                      out.ctypes.data)
    return out


_SIGS.update({
    "orc_log2_acc": (f32, [f32]),
    "orc_exp2_f32": (f32, [f32]),
    "orc_sigmoid_f32": (f32, [f32]),
    "orc_logmel_frames": (i32, [i32, i32, i32, i32]),
    "orc_logmel": (i32, [vp, i32, i32, i32, i32, i32, i32, vp, vp, f32, f32, vp]),
    "orc_gemm_f32": (None, [vp, i32, i32, vp, vp, i32, i32, vp, C.POINTER(OrcEpi32)]),
    "orc_stem_f32": (None, [vp, i32, i32, i32, i32, i32, i32, vp, vp, i32, i32, C.POINTER(OrcEpi32)]),
    "orc_se_gate_f32": (None, [vp, i32, i32, i32, vp, vp, vp, vp, vp]),
    "orc_se_f32": (None, [vp, i32, i32, vp, i32, vp, vp, vp, vp]),
    "orc_mean_f32": (None, [vp, i32, i32, i32, vp]),
    "orc_pad": (None, [vp, i32, i32, i32, i32, i32, C.c_size_t, vp]),
    "orc_expf_n": (None, [vp, vp, C.c_longlong]),
})


def expf(x):
    """The C library's expf (the function the reference's scalar SiLU calls)."""
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().orc_expf_n(P(x), P(y), x.size)
    return y


def logmel(pcm, frame, hop, pad, nfft, window, mel, floor_, scale):
    """FE_LOGMEL of one window: pcm [nsamp] -> spec [nfr][nmel]."""
    pcm = _c(pcm, np.float32)
    mel = _c(mel, np.float32)
    nmel = mel.shape[0]
    nfr = lib().orc_logmel_frames(pcm.size, frame, hop, pad)
    spec = np.zeros((nfr, nmel), np.float32)
    r = lib().orc_logmel(P(pcm), pcm.size, frame, hop, pad, nfft, nmel, P(_c(window, np.float32)), P(mel),
                         floor_, scale, P(spec))
    if r < 0:
        raise ValueError("logmel limits")
    return spec


def fpack(w, b):
    """fp_pack (src/gemm_f32.c:22-35): w [N][K] -> panels [Np/8][Kp][8] (Kp = K rounded to 4), bias [Np + 8]."""
    w = np.asarray(w, np.float32)
    N, K = w.shape
    Np, Kp = (N + 7) // 8 * 8, (K + 3) // 4 * 4
    wp = np.zeros((Np, Kp), np.float32)
    wp[:N, :K] = w
    panels = np.ascontiguousarray(wp.reshape(Np // 8, 8, Kp).transpose(0, 2, 1))
    bb = np.zeros(Np + 8, np.float32)
    bb[:N] = b
    return panels, bb, (N, K, Kp, Np)


def gemm_f32(A, panels, bb, Kp, Np, act=0, gate=None, res=None, ldr=0, rpad=0, rw=0, ow=0, opad=0, ldo=None):
    A = _c(A, np.float32)
    M, lda = A.shape
    ldo = ldo or Np
    rows = M if not opad else (M // ow + 2 * opad) * (ow + 2 * opad)
    out = np.zeros((rows, ldo), np.float32)
    r = None if res is None else _c(res, np.float32)
    e = OrcEpi32(act, out.ctypes.data, ldo, ow, opad, P(r), ldr, rpad, rw)
    g = None if gate is None else _c(gate, np.float32)
    lib().orc_gemm_f32(P(A), lda, M, P(_c(panels, np.float32)), P(_c(bb, np.float32)), Kp, Np, P(g), C.byref(e))
    return out


def stem_f32(img, k, s, panels, bb, Kp, Np, act=1, opad=0, ldo=None):
    img = _c(img, np.float32)
    H, W = img.shape
    Ho, Wo = (H - k) // s + 1, (W - k) // s + 1
    ldo = ldo or Np
    out = np.zeros(((Ho + 2 * opad) * (Wo + 2 * opad), ldo), np.float32)
    e = OrcEpi32(act, out.ctypes.data, ldo, Wo, opad, None, 0, 0, 0)
    lib().orc_stem_f32(P(img), H, W, k, s, Ho, Wo, P(_c(panels, np.float32)), P(_c(bb, np.float32)), Kp, Np,
                       C.byref(e))
    return out


def se_gate_f32(chsum, P_, w1, b1, w2t, b2):
    chsum = _c(chsum, np.float32)
    w1 = _c(w1, np.float32)
    rd, Cc = w1.shape
    g = np.zeros(Cc, np.float32)
    lib().orc_se_gate_f32(P(chsum), Cc, rd, P_, P(w1), P(_c(b1, np.float32)), P(_c(w2t, np.float32)),
                          P(_c(b2, np.float32)), P(g))
    return g


def mean_f32(x, C_):
    x = _c(x, np.float32)
    Pp, ld = x.shape
    out = np.zeros(C_, np.float32)
    lib().orc_mean_f32(P(x), Pp, C_, ld, P(out))
    return out


def pad(x, H, W, C_, h):
    """PAD of rows x [H*W][ld] -> [(H+2h)][(W+2h)][C] (dtype kept)."""
    x = np.ascontiguousarray(x)
    ld = x.shape[-1]
    out = np.full(((H + 2 * h) * (W + 2 * h), C_), 7, x.dtype)
    lib().orc_pad(P(x), H, W, C_, ld, h, x.dtype.itemsize, P(out))
    return out


_SIGS.update({
    "orc_stem_f32to16": (None, [vp, i32, i32, i32, i32, i32, i32, vp, vp, i32, i32, i32, i32, vp, i32, i32]),
    "orc_se_f16": (None, [vp, i32, i32, vp, i32, vp, vp, vp, vp]),
    "orc_mean_f16": (None, [vp, i32, i32, i32, vp]),
    "orc_gemv": (None, [vp, vp, vp, i32, i32, vp, i32, vp]),
})


def stem_f32to16(img, k, s, panels, bb, Kp, N, Np, act=1, opad=0, ldo=None, fill=0):
    """The fp16 path's STEM: fp32 stem, then fp16 channels [0, N) of a zero-haloed output [rows][ldo]; the other
    channels keep `fill`."""
    img = _c(img, np.float32)
    H, W = img.shape
    Ho, Wo = (H - k) // s + 1, (W - k) // s + 1
    ldo = ldo or Np
    out = np.full(((Ho + 2 * opad) * (Wo + 2 * opad), ldo), fill, np.float16)
    lib().orc_stem_f32to16(P(img), H, W, k, s, Ho, Wo, P(_c(panels, np.float32)), P(_c(bb, np.float32)), Kp, N, Np,
                           act, P(out), ldo, opad)
    return out


def se_f16(D, chsum, w1, b1, w2t, b2):
    """SE of the fp16 path on D fp16 [P][C] (a gated copy is returned)."""
    D = np.array(D, np.float16, copy=True, order="C")
    Pp, Cc = D.shape
    w1 = _c(w1, np.float32)
    rd = w1.shape[0]
    lib().orc_se_f16(P(D), Pp, Cc, P(_c(chsum, np.float32)), rd, P(w1), P(_c(b1, np.float32)),
                     P(_c(w2t, np.float32)), P(_c(b2, np.float32)))
    return D


def mean_f16(x, C_):
    x = _c(x, np.float16)
    Pp, ld = x.shape
    out = np.zeros(C_, np.float32)
    lib().orc_mean_f16(P(x), Pp, C_, ld, P(out))
    return out


def gemv(w, b, x, act=0):
    """bnn_gemv_f32 (w float32 [N][K]) or bnn_gemv_h16 (w float16 [N][K]) on x f32 [K]."""
    w = np.ascontiguousarray(w)
    N, K = w.shape
    out = np.zeros(N, np.float32)
    w32 = P(w) if w.dtype == np.float32 else None
    w16 = P(_c(w, np.float16)) if w.dtype == np.float16 else None
    assert w32 is not None or w16 is not None
    lib().orc_gemv(w32, w16, P(_c(b, np.float32)), N, K, P(_c(x, np.float32)), act, P(out))
    return out


_SIGS.update({"orc_stem3_f32h": (None, [vp, i32, i32, vp, vp, vp])})


def stem3(img, w, b):
    """STEM3 of one window: img f32 [H][W][3] -> fp16 zero-haloed [(H+1)/2 + 2][(W+1)/2 + 2][24]."""
    img = _c(img, np.float32)
    H, W = img.shape[:2]
    Ho, Wo = (H + 1) // 2, (W + 1) // 2
    out = np.zeros((Ho + 2, Wo + 2, 24), np.uint16)
    lib().orc_stem3_f32h(img.ctypes.data, H, W, _c(w, np.float32).ctypes.data, _c(b, np.float32).ctypes.data,
                         out.ctypes.data)
    return out.view(np.float16)


# ---------------------------------------------------------------- dotprod int8 family (qdot.c)
class OrcQdEpi(C.Structure):
    _fields_ = [("act", i32), ("out16", vp), ("out32", vp), ("ldo", i32), ("ow", i32), ("opad", i32),
                ("res32", vp)]


_SIGS.update({
    "orc_qd_wpack": (None, [vp, vp, i32, i32, vp, vp, vp, vp]),
    "orc_qd_quant_rows_f32": (None, [vp, i32, i32, i32, vp, i32, i32, vp]),
    "orc_qd_quant_rows_f16": (None, [vp, i32, i32, i32, vp, vp, i32, i32, vp]),
    "orc_exp2_p5": (f32, [f32]),
    "orc_silu_f32_a": (f32, [f32]),
    "orc_log2_dot": (f32, [f32]),
    "orc_qd_params": (None, [f32, f32, vp, vp, vp]),
    "orc_qd_gemm": (None, [vp, i32, vp, i32, i32, i32, i32, vp, vp, vp, vp, C.POINTER(OrcQdEpi)]),
    "orc_qd_quant_tensor_pad": (None, [vp, i32, i32, i32, vp, vp]),
    "orc_qconv3": (None, [vp, i32, i32, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp]),
    "orc_se_gate16": (None, [vp, i32, i32, i32, vp, vp, vp, vp, vp]),
    "orc_gem_a": (None, [vp, i32, i32, f32, f32, vp]),
    "orc_heads_s8": (None, [vp, vp, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp]),
})


def qd_wpack(w, b, Np=None):
    """qw_pack of w f32 [N][K] -> dict(q int8 [Np][Kp], scale, swsum, b [Np]); rows past N are zero (pack_padded)."""
    w = _c(w, np.float32)
    N, K = w.shape
    Np = Np or N
    Kp = (K + 15) // 16 * 16
    wp = np.zeros((Np, K), np.float32)
    wp[:N] = w
    bp = np.zeros(Np, np.float32)
    if b is not None:
        bp[:N] = b
    q = np.zeros((Np, Kp), np.int8)
    sc, ss, bb = (np.zeros(Np, np.float32) for _ in range(3))
    lib().orc_qd_wpack(P(wp), P(bp), Np, K, P(q), P(sc), P(ss), P(bb))
    return dict(q=q, scale=sc, swsum=ss, b=bb, shape=(N, K, Kp, Np))


def qd_params(mn, mx):
    s, zp, inv = (np.zeros(1, np.float32) for _ in range(3))
    lib().orc_qd_params(float(mn), float(mx), P(s), P(zp), P(inv))
    return float(s[0]), float(zp[0]), float(inv[0])


def qd_quant_rows(x, K, gate=None):
    """quant_rows_f32 (x float32) or quant_rows_f16 (x float16, optional fp16 gate) of x [M][ldx] -> (a [M][Kp], rq)."""
    x = np.ascontiguousarray(x)
    M, ldx = x.shape
    Kp = (K + 15) // 16 * 16
    a = np.zeros((M, Kp), np.int8)
    rq = np.zeros((M, 2), np.float32)
    if x.dtype == np.float16:
        g = None if gate is None else _c(gate, np.float16)
        lib().orc_qd_quant_rows_f16(P(x), ldx, M, K, P(g), P(a), Kp, Kp, P(rq))
    else:
        assert gate is None
        lib().orc_qd_quant_rows_f32(P(_c(x, np.float32)), ldx, M, K, P(a), Kp, Kp, P(rq))
    return a, rq


def qd_gemm(a, rq, pk, act=0, out16=False, ldo=None, ow=0, opad=0, res=None, per_tensor=False, M=None):
    """gemm_s8 of a int8 [M][Kp] -> out [rows][ldo] (fp16 when out16)."""
    a = _c(a, np.int8)
    M = M or a.shape[0]
    N, K, Kp, Np = pk["shape"]
    ldo = ldo or Np
    rows = M if not opad else (M // ow + 2) * (ow + 2)
    out = np.zeros((rows, ldo), np.float16 if out16 else np.float32)
    r = None if res is None else _c(res, np.float32)
    e = OrcQdEpi(act, P(out) if out16 else None, None if out16 else P(out), ldo, ow, opad, P(r))
    lib().orc_qd_gemm(P(a), a.shape[1], P(_c(rq, np.float32)), int(per_tensor), M, Np, Kp, P(pk["q"]),
                      P(pk["scale"]), P(pk["swsum"]), P(pk["b"]), C.byref(e))
    return out


def qpw(x, pk, act=0, out16=False, ldo=None, ow=0, opad=0, res=None, gate=None):
    """QPW of one window: x rows [M][ldx] (float32, or float16 with an optional gate) -> (out, a8, rq)."""
    N, K, Kp, Np = pk["shape"]
    a, rq = qd_quant_rows(x, K, gate)
    return qd_gemm(a, rq, pk, act, out16, ldo, ow, opad, res), a, rq


def qd_quant_tensor_pad(x):
    x = _c(x, np.float32)
    H, W, Cc = x.shape
    out = np.zeros((H + 2, W + 2, Cc), np.int8)
    rq = np.zeros(2, np.float32)
    lib().orc_qd_quant_tensor_pad(P(x), H, W, Cc, P(out), P(rq))
    return out, rq


def tf_same(n, k, s):
    o = (n + s - 1) // s
    tot = (o - 1) * s + k - n
    return o, max(tot, 0) // 2


def qconv3(x, pk, s):
    """QCONV3 of one window: x f32 [H][W][C], pk = qd_wpack of OHWI weights viewed [K][9C] -> fp16 [Ho*Wo][K]."""
    x = _c(x, np.float32)
    H, W, Cc = x.shape
    N, K9, Kp, Np = pk["shape"]
    Ho, pt = tf_same(H, 3, s)
    Wo, pl = tf_same(W, 3, s)
    xp = np.zeros((H + 2) * (W + 2) * Cc, np.int8)
    col = np.zeros(Ho * Wo * Kp, np.int8)
    out = np.zeros((Ho * Wo, Np), np.float16)
    lib().orc_qconv3(P(x), H, W, Cc, Np, s, pt, pl, Ho, Wo, P(pk["q"]), P(pk["scale"]), P(pk["swsum"]),
                     P(pk["b"]), P(xp), P(col), P(out))
    return out


def se_gate16(chsum, P_, w1, b1, w2, b2):
    """SE_GATE16 of one window -> (means [C], gate fp16 [C])."""
    cs = _c(chsum, np.float32).copy()
    rd, Cc = w1.shape
    g = np.zeros(Cc, np.float16)
    lib().orc_se_gate16(P(cs), Cc, rd, P_, P(_c(w1, np.float32)), P(_c(b1, np.float32)), P(_c(w2, np.float32)),
                        P(_c(b2, np.float32)), P(g))
    return cs, g


def gem_a(F, eps, p):
    F = _c(F, np.float32)
    M, Cc = F.shape
    e = np.zeros(Cc, np.float32)
    lib().orc_gem_a(P(F), M, Cc, float(eps), float(p), P(e))
    return e


def heads_s8(F, emb, H, W, packs):
    """HEADS_S8 of one window: F f32 [H*W][C], emb f32 [C]; packs: 7 qd_wpack dicts (lin, fc0, att0, cla0, fc1,
    att1, cla1; lin / att / cla padded to ncp) -> logits [ncp]."""
    F = _c(F, np.float32)
    Cc = F.shape[1]
    hid = packs[1]["shape"][3]
    nc = packs[0]["shape"][0]
    ncp = packs[0]["shape"][3]
    L = max(H, W)
    wmax = max(Cc, hid, ncp)
    work = np.zeros(5 * (L + 4) * wmax + (L + 4) * max(Cc, hid) // 4 + 16, np.float32)
    logits = np.zeros(ncp, np.float32)
    arr = lambda key: (vp * 7)(*[pk[key].ctypes.data for pk in packs])
    lib().orc_heads_s8(P(F), P(_c(emb, np.float32)), H, W, Cc, hid, nc, arr("q"), arr("scale"), arr("swsum"),
                       arr("b"), P(logits), P(work))
    return logits


_SIGS.update({
    "orc_quant_cells_f16": (None, [vp, i32, i32, i32, f32, vp, i32, vp]),
    "orc_proto_colmax_c12": (None, [vp, i32, vp, i32, i32, vp, vp, i32, vp]),
})


def proto_s8_dot(x, C, eps, qw, sw, Np, clsw, clsb, nc, ppc):
    """PROTO variant 2 of one window (src/rt_ops_f16.c:268-281): fp16 cells x [P][ld], panels qw [Np/12][K/4][12][4]
    -> (rc, logits, colmax)."""
    x = np.ascontiguousarray(x, np.float16)
    Pn, ld = x.shape
    Kp = (C + 15) // 16 * 16
    qa = np.zeros((Pn, Kp), np.int8)
    sx = np.zeros(Pn, np.float32)
    cm = np.zeros(Np, np.float32)
    lg = np.zeros(nc, np.float32)
    lib().orc_quant_cells_f16(P(x), Pn, C, ld, float(eps), P(qa), Kp, P(sx))
    lib().orc_proto_colmax_c12(P(qa), Kp, P(sx), Pn, C, P(_c(qw, np.int8)), P(_c(sw, np.float32)), Np, P(cm))
    rc = lib().orc_proto_logits(P(cm), P(_c(clsw, np.float32)), P(_c(clsb, np.float32)), nc, ppc, P(lg))
    return rc, lg, cm


def _h(a):
    """fp16 data as contiguous uint16 bit patterns (float16 arrays are reinterpreted, not converted)."""
    a = np.asarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return np.ascontiguousarray(a)


_SIGS.update({
    "orc_l2norm_f32": (None, [vp, i32, i32, i32, f32, vp]),
    "orc_l2norm_f16": (None, [vp, i32, i32, i32, f32, vp]),
    "orc_colmax_f32": (None, [vp, i32, i32, vp, i32, i32, vp]),
    "orc_colmax_f32h": (None, [vp, i32, i32, vp, i32, vp]),
    "orc_colmax_f16": (None, [vp, i32, i32, vp, i32, i32, vp]),
    "orc_proto_f32": (i32, [vp, i32, i32, i32, f32, vp, vp, i32, vp, vp, vp, i32, i32, vp]),
    "orc_proto_f32h": (i32, [vp, i32, i32, i32, f32, vp, vp, i32, vp, vp, vp, i32, i32, vp]),
    "orc_proto_f16": (i32, [vp, i32, i32, i32, f32, vp, vp, i32, vp, vp, vp, i32, i32, vp]),
})


def l2norm(x, C, eps, f16=False):
    """orc_l2norm_f32 / _f16 of cells x [P][ld] -> a [P][C] (fp32, or fp16 bit patterns)."""
    x = _h(x) if f16 else _c(x, np.float32)
    Pn, ld = x.shape
    a = np.zeros((Pn, C), np.uint16 if f16 else np.float32)
    (lib().orc_l2norm_f16 if f16 else lib().orc_l2norm_f32)(P(x), Pn, C, ld, float(eps), P(a))
    return a


def colmax_f32(a, wp, Kp, Np):
    """orc_colmax_f32: rows a [M][lda], fp32 panels [Np/8][Kp][8] -> colmax [Np]."""
    a = _c(a, np.float32)
    cm = np.zeros(Np, np.float32)
    lib().orc_colmax_f32(P(a), a.shape[1], a.shape[0], P(_c(wp, np.float32)), Kp, Np, P(cm))
    return cm


def colmax_f32h(a, w16, Np):
    """orc_colmax_f32h: cells a [P][K] fp32, fp16 panels [Np/8][K][8] (bit patterns) -> colmax [Np]."""
    a = _c(a, np.float32)
    cm = np.zeros(Np, np.float32)
    lib().orc_colmax_f32h(P(a), a.shape[0], a.shape[1], P(_h(w16)), Np, P(cm))
    return cm


def colmax_f16(a, W, Kp, Np):
    """orc_colmax_f16: fp16 rows a [M][lda] (bit patterns), hpack panels (bit patterns) -> colmax [Np]."""
    a = _h(a)
    cm = np.zeros(Np, np.float32)
    lib().orc_colmax_f16(P(a), a.shape[1], a.shape[0], P(_h(W)), Kp, Np, P(cm))
    return cm


def proto_fp(kind, x, C, eps, w, Np, clsw, clsb, nc, ppc):
    """PROTO variant 0 (kind "f32": fp32 panels), PROTO_F32H ("f32h": fp16 panels [Np/8][K][8]) or PROTO variant 1
    ("f16": fp16 cells, hpack panels) of one window -> (rc, logits, colmax, a)."""
    f16 = kind == "f16"
    x = _h(x) if f16 else _c(x, np.float32)
    Pn, ld = x.shape
    a = np.zeros((Pn, C), np.uint16 if f16 else np.float32)
    cm = np.zeros(Np, np.float32)
    lg = np.zeros(nc, np.float32)
    fn = {"f32": lib().orc_proto_f32, "f32h": lib().orc_proto_f32h, "f16": lib().orc_proto_f16}[kind]
    rc = fn(P(x), Pn, C, ld, float(eps), P(a), P(_c(w, np.float32) if kind == "f32" else _h(w)), Np, P(cm), P(_c(clsw, np.float32)),
            P(_c(clsb, np.float32)), nc, ppc, P(lg))
    return rc, lg, cm, a


_SIGS.update({"orc_powf_vec": (None, [vp, vp, vp, C.c_longlong])})


def powf(x, y):
    """The C library's powf, elementwise on float32 arrays."""
    x, y = np.broadcast_arrays(np.asarray(x, np.float32), np.asarray(y, np.float32))
    x, y = _c(x, np.float32), _c(y, np.float32)
    z = np.empty_like(x)
    lib().orc_powf_vec(P(x), P(y), P(z), x.size)
    return z


_SIGS.update({
    "orc_fft_dit": (None, [vp, vp, i32, vp, vp]),
    "orc_se_fc1": (None, [vp, i32, i32, vp, i32, vp, vp]),
    "orc_heads_pool": (None, [vp, i32, i32, i32, i32, vp, vp]),
    "orc_heads_softmax": (None, [vp, vp, i32, i32, i32, vp]),
})


def fft_twiddles(M):
    """fft_twiddles (src/fft_tab.h:9-14): e^{-2 pi i k / M}, k < M / 2, in double, rounded once to float."""
    a = -2 * np.pi * np.arange(M // 2) / M
    return np.cos(a).astype(np.float32), np.sin(a).astype(np.float32)


def fft_dit(re, im):
    """orc_fft_dit: M points (bit-reversed order) of one lane -> (re, im)."""
    re, im = _c(re, np.float32).copy(), _c(im, np.float32).copy()
    twr, twi = fft_twiddles(re.size)
    lib().orc_fft_dit(P(re), P(im), re.size, P(twr), P(twi))
    return re, im


def se_fc1(mean, w1, b1, h16=False):
    """orc_se_fc1: mean [C], w1 [rd][C], b1 [rd] -> s1 [rd]."""
    w1 = _c(w1, np.float32)
    rd, C = w1.shape
    s1 = np.zeros(rd, np.float32)
    lib().orc_se_fc1(P(_c(mean, np.float32)), C, rd, P(w1), int(h16), P(_c(b1, np.float32)), P(s1))
    return s1


def heads_pool(F, H, W, i):
    """orc_heads_pool: F [H*W][C], head i -> (means [L][C], pooled [L][C])."""
    F = _c(F, np.float32)
    C = F.shape[-1]
    L = H if i == 0 else W
    s = np.zeros((L, C), np.float32)
    pooled = np.zeros((L, C), np.float32)
    lib().orc_heads_pool(P(F), H, W, C, i, P(s), P(pooled))
    return s, pooled


def heads_softmax(att, cla, nc, logits):
    """orc_heads_softmax: att, cla [L][ncp] -> logits [ncp] (+= the attention-pooled class scores; att is clipped)."""
    att = _c(att, np.float32).copy()
    cla = _c(cla, np.float32)
    lg = _c(logits, np.float32).copy()
    L, ncp = att.shape
    lib().orc_heads_softmax(P(att), P(cla), L, nc, ncp, P(lg))
    return lg
