"""ctypes binding of libbnneon_hip's kernel-level C ABI (include/bnneon_hip.h).

The library is the only compute path: if libbnneon_hip.so is missing or
cannot be loaded, importing this module's `lib()` raises. Device memory is
owned through `DeviceArray` (hipMalloc'd by the library itself), so hosts need
no HIP runtime of their own.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libbnneon_hip.so")

_lib = None

vp = C.c_void_p
i32 = C.c_int
i64 = C.c_longlong


class Epi32(C.Structure):
    """bnh_epi32: the fp32 epilogue of the int8 GEMM (per-window strides)."""
    _fields_ = [("act", i32), ("out", vp), ("out_ws", i64), ("ldo", i32),
                ("ow", i32), ("opad", i32), ("res", vp), ("res_ws", i64),
                ("ldr", i32), ("rpad", i32), ("rw", i32)]


class Epi16(C.Structure):
    """bnh_epi16: the fp16 GEMM epilogue (per-window strides)."""
    _fields_ = [("act", i32), ("out", vp), ("out_ws", i64), ("ldo", i32),
                ("ow", i32), ("opad", i32), ("res", vp), ("res_ws", i64),
                ("ldr", i32)]


class QdEpi(C.Structure):
    """bnh_qd_epi: the dotprod int8 GEMM's epilogue (per-window strides)."""
    _fields_ = [("act", i32), ("out_f16", i32), ("out", vp), ("out_ws", i64),
                ("ldo", i32), ("ow", i32), ("opad", i32), ("res", vp),
                ("res_ws", i64)]


_SIGS = {
    "bnh_last_error": (C.c_char_p, []),
    "bnh_device_count": (i32, []),
    "bnh_malloc": (vp, [C.c_size_t]),
    "bnh_free": (i32, [vp]),
    "bnh_memcpy_h2d": (i32, [vp, vp, C.c_size_t]),
    "bnh_memcpy_d2h": (i32, [vp, vp, C.c_size_t]),
    "bnh_memset": (i32, [vp, i32, C.c_size_t]),
    "bnh_stream_new": (vp, []),
    "bnh_stream_free": (i32, [vp]),
    "bnh_stream_sync": (i32, [vp]),
    "bnh_event_new": (vp, []),
    "bnh_event_free": (i32, [vp]),
    "bnh_event_record": (i32, [vp, vp]),
    "bnh_event_ms": (C.c_float, [vp, vp]),
    "bnh_eval_f32": (i32, [i32, vp, vp, i64, vp]),
    "bnh_eval_requant": (i32, [vp, vp, vp, i32, i32, i32, vp, i64, vp]),
    "bnh_copy": (i32, [vp, vp, C.c_size_t, vp]),
    "bnh_s8w_new": (vp, [i32, i32, i32, i32, vp, vp, vp, vp]),
    "bnh_s8w_free": (None, [vp]),
    "bnh_s8n_quant_rows": (i32, [vp, i64, i32, i32, i32, i32, vp, i64, vp,
                                 i64, vp, i64, vp, i64, i32, vp]),
    "bnh_s8n_gemm": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, vp,
                           C.POINTER(Epi32), vp]),
    "bnh_pw_s8": (i32, [vp, i64, i32, i32, vp, i64, vp, i64, vp, i64, vp,
                        i64, i32, vp, C.POINTER(Epi32), vp]),
    "bnh_pw_s8_static": (i32, [vp, i64, i32, i32, vp, i64, i32, vp, C.POINTER(Epi32), vp]),
    "bnh_s8p_new": (vp, [i32, i32, vp, vp]),
    "bnh_s8p_free": (None, [vp]),
    "bnh_quant_cells": (i32, [vp, i64, i32, i32, i32, C.c_float, vp, i64, i32,
                              vp, i64, i32, vp]),
    "bnh_proto_colmax": (i32, [vp, i64, vp, i64, i32, vp, vp, i64, i32, vp]),
    "bnh_proto_logits": (i32, [vp, i64, vp, vp, i32, i32, vp, i64, i32, vp,
                               i32, vp]),
    "bnh_q8w_new": (vp, [i32, i32, vp, vp, vp, vp, i32, i32, i32, i32]),
    "bnh_q8w_free": (None, [vp]),
    "bnh_gemm_s8_requant": (i32, [vp, vp, i64, i32, i32, vp, i64, vp]),
    "bnh_h16w_new": (vp, [i32, i32, i32, i32, vp, vp, vp]),
    "bnh_h16w_free": (None, [vp]),
    "bnh_gemm_f16": (i32, [vp, i64, i32, i32, i32, vp, C.POINTER(Epi16), vp]),
    "bnh_gemm_f16_mfma": (i32, [vp, i64, i32, i32, i32, vp, C.POINTER(Epi16), vp]),
    "bnh_gemm_f16_body": (i32, [vp, i64, i32, i32, i32, vp, C.POINTER(Epi16), vp]),
    "bnh_gemm_f16_ws_bytes": (C.c_size_t, [i32, i32, vp]),
    "bnh_gemm_f16_ws": (i32, [vp, i64, i32, i32, i32, vp, C.POINTER(Epi16), vp, C.c_size_t, vp]),
    "bnh_gemm_f16_gated_ws": (i32, [vp, i64, i32, i32, i32, vp, C.POINTER(Epi16), vp, i64, vp, C.c_size_t,
                                    vp]),
    "bnh_wino16_new": (vp, [i32, i32, vp, vp]),
    "bnh_wino16_free": (None, [vp]),
    "bnh_wino_f16": (i32, [vp, i64, i32, i32, i32, vp, i32, vp, i64, i32, i32, vp, i64, i32, i32, i32, vp]),
    "bnh_wino8_new": (vp, [i32, i32, vp, vp]),
    "bnh_wino8_free": (None, [vp]),
    "bnh_wino8_work_bytes": (C.c_size_t, [i32, i32, i32, i32]),
    "bnh_wino_s8": (i32, [vp, i64, i32, i32, vp, vp, i64, i32, vp, C.c_size_t, vp]),
    "bnh_dwk_f32": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, i32, vp, vp,
                          i32, vp, i64, i32, i32, vp, i64, i32, vp]),
    "bnh_dw3_f32": (i32, [vp, i64, i32, i32, i32, i32, vp, vp, vp, i64, i32,
                          i32, vp, i64, i32, vp]),
    "bnh_pwdw_f32": (i32, [vp, i64, vp, i64, vp, i64, i32, i32, vp, i32, i32,
                           i32, i32, i32, i32, vp, vp, i32, vp, i64, i32, i32,
                           vp, i64, i32, vp]),
    "bnh_dwk_f16": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, i32, vp, vp,
                          i32, vp, i64, i32, i32, vp, i64, i32, vp]),
    "bnh_dw3_f16": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, vp, vp, vp,
                          i64, i32, i32, vp, i64, i32, vp]),
    "bnh_dw_s8": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp,
                        vp, i32, i32, i32, i32, vp, vp, i64, i32, i32, i32,
                        vp]),
    "bnh_logmel_new": (vp, [i32, i32, i32, i32, i32, i32, vp, vp, C.c_float, C.c_float]),
    "bnh_logmel_free": (None, [vp]),
    "bnh_logmel_frames": (i32, [vp]),
    "bnh_logmel_run": (i32, [vp, vp, i64, vp, i64, i32, vp]),
    "bnh_stem3_f16": (i32, [vp, i64, i32, i32, vp, vp, vp, i64, i32, vp]),
    "bnh_unpad_f16": (i32, [vp, i64, i32, i32, i32, vp, i64, i32, vp]),
    "bnh_gemm_f32": (i32, [vp, i64, i32, i32, vp, i64, vp, vp, i32, i32, C.POINTER(Epi32), i32, vp]),
    "bnh_stem_f32": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, vp, vp, i32, i32, i32, vp, i64, i32, i32, i32, vp]),
    "bnh_se_f32": (i32, [vp, i64, i32, i32, i32, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, vp]),
    "bnh_mean_f32": (i32, [vp, i64, i32, i32, i32, vp, i64, i32, vp]),
    "bnh_pad": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, vp, i64, i32, vp]),
    "bnh_zero_halo": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, vp]),
    "bnh_eval_expf": (i32, [vp, vp, i64, vp]),
    "bnh_eval_powf": (i32, [vp, vp, vp, i64, vp]),
    "bnh_stem_f32to16": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, vp, vp, i32, i32, i32, i32, vp, i64, i32, i32,
                               i32, vp]),
    "bnh_se_f16": (i32, [vp, i64, i32, i32, i32, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, vp]),
    "bnh_se_gate_f16": (i32, [vp, i64, i32, i32, i32, vp, vp, vp, vp, vp, i64, vp, vp, i64, i32, vp]),
    "bnh_mean_f16": (i32, [vp, i64, i32, i32, i32, vp, i64, i32, vp]),
    "bnh_gemv": (i32, [vp, i32, vp, i32, i32, vp, i64, i32, vp, i64, i32, vp]),
    "bnh_qdw_new": (vp, [vp, vp, i32, i32, i32]),
    "bnh_qdw_free": (None, [vp]),
    "bnh_qdw_shape": (i32, [vp, vp, vp, vp, vp]),
    "bnh_qd_quant_rows": (i32, [vp, i32, i64, i32, i32, i32, vp, i64, vp, i64, vp, i64, i32, vp]),
    "bnh_qd_gemm": (i32, [vp, i64, i32, vp, i64, i32, i32, vp, C.POINTER(QdEpi), i32, vp]),
    "bnh_qconv3_work_bytes": (C.c_size_t, [i32, i32, i32]),
    "bnh_qconv3": (i32, [vp, i64, i32, i32, i32, i32, i32, i32, i32, i32, vp, vp, i64, i32, vp, C.c_size_t, vp]),
    "bnh_heads8_new": (vp, [i32, i32, i32, vp, vp]),
    "bnh_heads8_free": (None, [vp]),
    "bnh_heads8_work_bytes": (C.c_size_t, [i32, i32, i32, i32, i32]),
    "bnh_heads_s8": (i32, [vp, i64, vp, i64, i32, i32, vp, vp, i64, vp, i64, vp, i64, i32, vp, C.c_size_t, vp]),
    "bnh_seg16_new": (vp, [i32, i32, vp, vp, vp, vp]),
    "bnh_seg16_free": (None, [vp]),
    "bnh_se_gate16": (i32, [vp, i64, i32, vp, vp, i64, i32, vp]),
    "bnh_gem_a": (i32, [vp, i64, i32, i32, C.c_float, C.c_float, vp, i64, i32, vp]),
    "bnh_eval_qd": (i32, [i32, vp, vp, i64, vp]),
    "bnh_quant_cells_f16": (i32, [vp, i64, i32, i32, i32, C.c_float, vp, i64, i32, vp, i64, i32, vp]),
    "bnh_s8p_new_c12": (vp, [i32, i32, vp, vp]),
    "bnh_gemm_f16_mfma_gated": (i32, [vp, i64, i32, i32, i32, vp, C.POINTER(Epi16), vp, i64, vp]),
    "bnh_fproto_new": (vp, [i32, i32, i32, vp]),
    "bnh_fproto_free": (None, [vp]),
    "bnh_l2norm_cells": (i32, [vp, i64, i32, i32, i32, C.c_float, i32, vp, i64, i32, vp]),
    "bnh_fproto_colmax": (i32, [vp, i64, i32, vp, vp, i64, i32, vp]),
}


def lib():
    """The loaded libbnneon_hip.so (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run birdnet-neon-engine_amd/build.py"
                " (the HIP library is the only compute path)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name, None)
            if f is None:
                continue
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    """Names of _SIGS the loaded library exports."""
    L = lib()
    return [n for n in _SIGS if hasattr(L, n)]


class HipError(RuntimeError):
    """A libbnneon_hip call returned an error (message: bnh_last_error)."""


def check(rc, what="libbnneon_hip"):
    """Raises HipError with the library's message when rc is nonzero/None."""
    if rc is None or (isinstance(rc, int) and rc != 0):
        msg = lib().bnh_last_error()
        raise HipError(f"{what}: {msg.decode() if msg else 'failed'}")
    return rc


def ptr(x):
    """Device pointer of a DeviceArray (or None)."""
    return None if x is None else x.ptr


class DeviceArray:
    """A hipMalloc'd array with a numpy dtype and shape."""

    def __init__(self, shape, dtype, slack=256):
        self.shape = tuple(int(s) for s in np.atleast_1d(shape))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = lib().bnh_malloc(self.nbytes + slack)
        if not self.ptr:
            check(None, "bnh_malloc")

    @classmethod
    def from_host(cls, a, slack=256):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype, slack)
        d.upload(a)
        return d

    @classmethod
    def zeros(cls, shape, dtype, slack=256):
        d = cls(shape, dtype, slack)
        check(lib().bnh_memset(d.ptr, 0, d.nbytes + slack), "bnh_memset")
        return d

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        check(lib().bnh_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes),
              "bnh_memcpy_h2d")

    def fill(self, byte):
        check(lib().bnh_memset(self.ptr, int(byte), self.nbytes), "bnh_memset")

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        check(lib().bnh_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes),
              "bnh_memcpy_d2h")
        return out

    def free(self):
        if self.ptr:
            lib().bnh_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync(stream=None):
    check(lib().bnh_stream_sync(stream), "bnh_stream_sync")


class S8Weights:
    """bnh_s8w: one int8 GEMM's weights in HBM (from package tensors)."""

    def __init__(self, n, k, kp, np_, w, sw, colsum, b):
        w = np.ascontiguousarray(w, np.int8)
        sw = np.ascontiguousarray(sw, np.float32)
        colsum = np.ascontiguousarray(colsum, np.int32)
        b = np.ascontiguousarray(b, np.float32)
        self.N, self.K, self.Kp, self.Np = n, k, kp, np_
        self.h = lib().bnh_s8w_new(n, k, kp, np_, w.ctypes.data, sw.ctypes.data,
                                   colsum.ctypes.data, b.ctypes.data)
        if not self.h:
            check(None, "bnh_s8w_new")

    def __del__(self):
        try:
            if self.h:
                lib().bnh_s8w_free(self.h)
        except Exception:
            pass


class Q8Weights:
    """bnh_q8w: int8 weights + Q31 requant parameters in HBM."""

    def __init__(self, w, bias, mult, shift, zx, zy, lo=-128, hi=127):
        w = np.ascontiguousarray(w, np.int8)
        n, k = w.shape
        bias = np.ascontiguousarray(bias, np.int32)
        mult = np.ascontiguousarray(mult, np.int32)
        shift = np.ascontiguousarray(shift, np.int32)
        self.N, self.K = n, k
        self.h = lib().bnh_q8w_new(n, k, w.ctypes.data, bias.ctypes.data,
                                   mult.ctypes.data, shift.ctypes.data, zx, zy,
                                   lo, hi)
        if not self.h:
            check(None, "bnh_q8w_new")

    def __del__(self):
        try:
            if self.h:
                lib().bnh_q8w_free(self.h)
        except Exception:
            pass


class FProto:
    """bnh_fproto: the prototypes of an fp32 / fp16 prototype head in HBM. kind 0: fp32 panels [Np/8][K][8]
    (PROTO variant 0), 1: fp16 panels [Np/8][K][8] (PROTO_F32H), 2: fp16 hpack panels (PROTO variant 1)."""

    def __init__(self, kind, Np, K, w):
        w = np.asarray(w)
        w = np.ascontiguousarray(w.view(np.uint16) if w.dtype == np.float16 else w)
        self.kind, self.Np, self.K = kind, Np, K
        self.h = lib().bnh_fproto_new(kind, Np, K, w.ctypes.data)
        if not self.h:
            check(None, "bnh_fproto_new")

    def __del__(self):
        try:
            if self.h:
                lib().bnh_fproto_free(self.h)
        except Exception:
            pass


def epi32(out, ldo, act=0, ow=0, opad=0, res=None, ldr=0, rpad=0, rw=0,
          out_ws=0, res_ws=0):
    """A bnh_epi32 for device arrays out / res."""
    return Epi32(act, ptr(out), out_ws, ldo, ow, opad, ptr(res), res_ws, ldr,
                 rpad, rw)
