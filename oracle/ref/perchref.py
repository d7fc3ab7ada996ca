"""The reference's own scalar Perch v2 oracle (src/perch_ref.c), through oracle/_ref/libperchref.so.

Test infrastructure: a checker for the op-by-op oracle's nets and the reference code's CPU timing. The library is
built from the reference checkout by `make -C oracle ref`; `available()` is False where it was not built.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(os.path.dirname(HERE), "_ref", "libperchref.so")
EMB = 1536
_lib = None


def available():
    return os.path.exists(LIB)


def lib():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(LIB)
        L.prs_load.restype = ctypes.c_void_p
        L.prs_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]
        L.prs_n_classes.argtypes = [ctypes.c_void_p]
        L.prs_infer.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.prs_free.argtypes = [ctypes.c_void_p]
        _lib = L
    return _lib


class Model:
    """A loaded .bnp2 file; infer() runs pc_ref_infer on one window (thread-safe: a context per call)."""

    def __init__(self, path):
        err = ctypes.create_string_buffer(256)
        self.h = lib().prs_load(path.encode(), err, 256)
        if not self.h:
            raise RuntimeError(f"pc_model_load: {err.value.decode()}")
        self.n_classes = lib().prs_n_classes(self.h)

    def infer(self, pcm):
        pcm = np.ascontiguousarray(pcm, np.float32)
        lg = np.zeros(self.n_classes, np.float32)
        emb = np.zeros(EMB, np.float32)
        rc = lib().prs_infer(self.h, pcm.ctypes.data, lg.ctypes.data, emb.ctypes.data)
        if rc:
            raise RuntimeError(f"pc_ref_infer returned {rc}")
        return lg, emb

    def close(self):
        if self.h:
            lib().prs_free(self.h)
            self.h = None


def write_bnp2(path, perchnet):
    """The .bnp2 file of a bnneon.perchnet.PerchNet (its kept float weights). A net with the linear head gets a
    one-class, one-prototype head in the file (the reference's oracle always runs its ProtoPNet head)."""
    import bnp2
    from bnneon import perchnet as P
    pn = perchnet
    proto = pn.head == "proto"
    ppc, nc = (pn.ppc, pn.n_classes) if proto else (1, 1)
    consts = bnp2.fe_consts(P.FRAME, P.HOP, P.PAD, P.NFFT, pn.log_floor, pn.log_scale, pn.eps, ppc)
    fw = dict(pn.fw)
    tensors = [("fe.consts", consts)] + [(n, fw[n]) for n in ("fe.window", "fe.mel", "stem.w", "stem.b")]
    tensors += [(n, a) for n, a in pn.fw if n.startswith("m")]
    tensors += [(n, fw[n]) for n in ("top.w", "top.b")]
    if proto:
        tensors += [(n, fw[n]) for n in ("proto", "cls.w", "cls.b")]
    else:
        tensors += [("proto", np.full((1, EMB), 1.0 / EMB, np.float32)), ("cls.w", np.ones((1, 1), np.float32)),
                    ("cls.b", np.zeros(1, np.float32))]
    return bnp2.write(path, tensors, pn.blocks_table, nc)
