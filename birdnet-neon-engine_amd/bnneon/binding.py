"""ctypes binding of the libbnneon host API (include/bnneon.h) on
libbnneon_hip.so: the reference binding's interface (python/bnneon/binding.py:
Info, probe, Model.infer, Model.meta, errors with kinds) plus batched
inference.
"""
import ctypes

import numpy as np

from . import hip

API_VERSION = 2
MODE_DEFAULT, MODE_REFERENCE, MODE_FP32, MODE_FP16, MODE_INT8 = 0, 1, 2, 3, 4
ERR_KINDS = {0: "none", 1: "package", 2: "oom", 3: "cpu", 4: "window", 5: "labels", 6: "usage"}


class BnnError(RuntimeError):
    """A failed libbnneon call: message (bnn_last_error) and kind."""

    def __init__(self, message, kind):
        super().__init__(message)
        self.kind = kind


class Info(ctypes.Structure):
    """bnn_info (fields are only ever appended)."""
    _fields_ = [("struct_size", ctypes.c_uint32), ("model", ctypes.c_int),
                ("format_version", ctypes.c_int), ("sample_rate", ctypes.c_int),
                ("n_samples", ctypes.c_int), ("hop_samples", ctypes.c_int),
                ("n_classes", ctypes.c_int), ("output_kind", ctypes.c_int),
                ("post", ctypes.c_int), ("logit_scale", ctypes.c_float),
                ("emb_dim", ctypes.c_int), ("has_labels_sha", ctypes.c_int),
                ("labels_sha256", ctypes.c_ubyte * 32),
                ("model_id", ctypes.c_char * 64), ("path", ctypes.c_char * 32),
                ("precision", ctypes.c_char_p)]


_FP = ctypes.POINTER(ctypes.c_float)
_IP = ctypes.POINTER(ctypes.c_int)
_SIGNATURES = {
    "bnn_api_version": (ctypes.c_int, []),
    "bnn_cpu_supported": (ctypes.c_int, [ctypes.c_int]),
    "bnn_probe": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(Info)]),
    "bnn_probe_meta": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]),
    "bnn_meta": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]),
    "bnn_init": (ctypes.c_void_p, [ctypes.c_char_p, ctypes.c_int]),
    "bnn_get_info": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Info)]),
    "bnn_infer": (ctypes.c_int, [ctypes.c_void_p, _FP, _FP, _FP]),
    "bnn_verify_labels": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p]),
    "bnn_last_error": (ctypes.c_char_p, []),
    "bnn_last_error_kind": (ctypes.c_int, []),
    "bnn_set_threads": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "bnn_free": (None, [ctypes.c_void_p]),
    "bnn_infer_batch": (ctypes.c_int, [ctypes.c_void_p, _FP, ctypes.c_int, _FP, _FP, _IP]),
    "bnn_infer_batch_device": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                              ctypes.c_void_p, _IP, ctypes.c_void_p]),
}

_lib = None


def load_library():
    global _lib
    if _lib is None:
        L = hip.lib()
        for name, (res, args) in _SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        if L.bnn_api_version() != API_VERSION:
            raise RuntimeError("libbnneon_hip speaks API %d, expected %d" % (L.bnn_api_version(), API_VERSION))
        _lib = L
    return _lib


def _raise(L, what):
    msg = (L.bnn_last_error() or b"").decode(errors="replace")
    raise BnnError(f"{what}: {msg}", ERR_KINDS.get(L.bnn_last_error_kind(), "?"))


def _fp(a):
    return None if a is None else a.ctypes.data_as(_FP)


def probe(path):
    L = load_library()
    info = Info()
    info.struct_size = ctypes.sizeof(Info)
    if L.bnn_probe(path.encode(), ctypes.byref(info)):
        _raise(L, "bnn_probe")
    return info


def probe_meta(path, key, raw=False):
    L = load_library()
    n = L.bnn_probe_meta(path.encode(), key.encode(), None, 0)
    if n < 0:
        return None
    buf = ctypes.create_string_buffer(n + 1)
    L.bnn_probe_meta(path.encode(), key.encode(), buf, n + 1)
    return buf.raw[:n] if raw else buf.raw[:n].decode(errors="replace")


class Model:
    """One context: a package's path running on the GPU."""

    def __init__(self, path, mode=MODE_DEFAULT):
        self.L = load_library()
        self.ctx = self.L.bnn_init(path.encode(), mode)
        if not self.ctx:
            _raise(self.L, f"bnn_init({path!r}, mode {mode})")
        self.info = Info()
        self.info.struct_size = ctypes.sizeof(Info)
        self.L.bnn_get_info(self.ctx, ctypes.byref(self.info))

    def set_threads(self, threads):
        if self.L.bnn_set_threads(self.ctx, threads):
            _raise(self.L, "bnn_set_threads")

    def meta(self, key, raw=False):
        n = self.L.bnn_meta(self.ctx, key.encode(), None, 0)
        if n < 0:
            return None
        buf = ctypes.create_string_buffer(n + 1)
        self.L.bnn_meta(self.ctx, key.encode(), buf, n + 1)
        return buf.raw[:n] if raw else buf.raw[:n].decode(errors="replace")

    def infer(self, pcm):
        """(logits [n_classes], embedding or None) of one window."""
        pcm = np.ascontiguousarray(pcm, np.float32)
        assert pcm.size == self.info.n_samples
        out = np.empty(self.info.n_classes, np.float32)
        emb = np.empty(self.info.emb_dim, np.float32) if self.info.emb_dim else None
        if self.L.bnn_infer(self.ctx, _fp(pcm), _fp(out), _fp(emb)):
            _raise(self.L, "bnn_infer")
        return out, emb

    def infer_batch(self, pcm, check=True):
        """pcm [n][n_samples] -> (logits [n][n_classes], emb or None, status [n])."""
        pcm = np.ascontiguousarray(pcm, np.float32)
        n = pcm.shape[0]
        assert pcm.shape[1] == self.info.n_samples
        out = np.empty((n, self.info.n_classes), np.float32)
        emb = np.empty((n, self.info.emb_dim), np.float32) if self.info.emb_dim else None
        status = np.zeros(n, np.int32)
        r = self.L.bnn_infer_batch(self.ctx, _fp(pcm), n, _fp(out), _fp(emb), status.ctypes.data_as(_IP))
        if r < 0 or (r > 0 and check):
            _raise(self.L, "bnn_infer_batch")
        return out, emb, status

    def close(self):
        if self.ctx:
            self.L.bnn_free(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
