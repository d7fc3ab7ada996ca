"""The .bnpk package format: writer and reader.

The layout is libbnneon's (python/bnneon/compiler/pkgfmt.py:1-22 documents
it, src/rt_pkg.c reads it), kept byte-compatible so packages move between the
CPU library and this one:

  header (64 B): "BNNPKG01", u32 bom 0x01020304, u16 format_version,
      u16 min_reader_version, u32 n_meta, n_tensors, n_paths, reserved,
      u64 meta_off, tensor_off, path_off, file_size
  metadata records: u16 key_len, u16 type (0 str, 1 i64, 2 f64, 3 bytes),
      u32 val_len, key, value, zero-padded to 8
  tensor table (96 B each): char name[48], u32 dtype (0 f32, 1 f16, 2 i8,
      3 i32), u32 ndim, u32 dims[4], u64 offset, nbytes, reserved
  path table (72 B each): char name[24], u32 hwcap, n_buf, n_ops, ops_bytes,
      in_buf, out_buf, emb_buf (0xffffffff = none), reserved, u64 buf_off,
      ops_off
  per path: buffers (40 B each: u32 dtype, H, W, C, ld, halo, slot, 0;
      u64 elems) and op records (u16 opcode, u16 rec_bytes, u16 n_buf,
      n_ten, n_int, 0; i32 bufs[], tensors[], ints[]; padded to 8)
  tensor blobs: 64-byte aligned, each followed by >= 64 zero bytes.
"""
import struct

import numpy as np

MAGIC = b"BNNPKG01"
FORMAT_VERSION = 1
MIN_READER = 1
DTYPE = {np.dtype(np.float32): 0, np.dtype(np.float16): 1,
         np.dtype(np.int8): 2, np.dtype(np.int32): 3}
NP_DTYPE = {v: k for k, v in DTYPE.items()}
HDR = struct.Struct("<8sIHH4I4Q")
TENSOR = struct.Struct("<48s6I3Q")
PATH = struct.Struct("<24s8I2Q")
BUF = struct.Struct("<8IQ")


def _pad(b, align=8):
    return b + b"\0" * (-len(b) % align)


def meta_record(key, value):
    k = key.encode()
    if isinstance(value, (bytes, bytearray)):
        ty, v = 3, bytes(value)
    elif isinstance(value, (bool, int, np.integer)):
        ty, v = 1, struct.pack("<q", int(value))
    elif isinstance(value, (float, np.floating)):
        ty, v = 2, struct.pack("<d", float(value))
    else:
        ty, v = 0, str(value).encode()
    return _pad(struct.pack("<HHI", len(k), ty, len(v)) + k + v)


def op_record(code, bufs, tensors, ints):
    body = struct.pack(f"<{len(bufs) + len(tensors) + len(ints)}i",
                       *(list(bufs) + list(tensors) + list(ints)))
    rec = _pad(struct.pack("<6H", code, 0, len(bufs), len(tensors),
                           len(ints), 0) + body)
    return rec[:2] + struct.pack("<H", len(rec)) + rec[4:]


class Package:
    """A package under construction: metadata, tensors, paths."""

    def __init__(self):
        self.meta = []
        self.tensors = []   # (name, array, nbytes)
        self.index = {}
        self.paths = []

    def set(self, key, value):
        self.meta.append((key, value))

    def tensor(self, name, a, min_bytes=0):
        """Adds a tensor (deduplicated by name); returns its index."""
        if name in self.index:
            return self.index[name]
        a = np.ascontiguousarray(a)
        assert a.dtype in DTYPE and a.ndim <= 4 and len(name) < 48, (name, a.dtype)
        self.index[name] = len(self.tensors)
        self.tensors.append((name, a, max(min_bytes, a.nbytes)))
        return self.index[name]

    def add_path(self, name, hwcap, bufs, ops, in_buf, out_buf, emb_buf=None):
        """bufs: (dtype, H, W, C, ld, halo, elems, slot); ops: (code, b, t, i)."""
        self.paths.append((name, hwcap, bufs, ops, in_buf, out_buf, emb_buf))

    def to_bytes(self):
        meta = b"".join(meta_record(k, v) for k, v in self.meta)
        meta_off = HDR.size
        tensor_off = meta_off + len(meta)
        path_off = tensor_off + TENSOR.size * len(self.tensors)
        off = path_off + PATH.size * len(self.paths)
        pdesc, blobs = [], []
        for name, hw, bufs, ops, ib, ob, eb in self.paths:
            bb = b"".join(BUF.pack(b[0], b[1], b[2], b[3], b[4], b[5], b[7], 0, b[6])
                          for b in bufs)
            ob_ = b"".join(op_record(*o) for o in ops)
            pdesc.append(PATH.pack(name.encode(), hw, len(bufs), len(ops), len(ob_),
                                   ib, ob, 0xffffffff if eb is None else eb, 0,
                                   off, off + len(bb)))
            blobs += [bb, ob_]
            off += len(bb) + len(ob_)
        off = (off + 63) & ~63
        tdesc, tblobs = [], []
        for name, a, nbytes in self.tensors:
            dims = list(a.shape) + [0] * (4 - a.ndim)
            tdesc.append(TENSOR.pack(name.encode(), DTYPE[a.dtype], a.ndim, *dims,
                                     off, nbytes, 0))
            tblobs.append((off, a, nbytes))
            off = (off + nbytes + 64 + 63) & ~63
        size = off + 64
        out = bytearray(size)
        out[:HDR.size] = HDR.pack(MAGIC, 0x01020304, FORMAT_VERSION, MIN_READER,
                                  len(self.meta), len(self.tensors),
                                  len(self.paths), 0, meta_off, tensor_off,
                                  path_off, size)
        out[meta_off:tensor_off] = meta
        p = tensor_off
        for t in tdesc:
            out[p:p + TENSOR.size] = t
            p += TENSOR.size
        for d in pdesc:
            out[p:p + PATH.size] = d
            p += PATH.size
        for b in blobs:
            out[p:p + len(b)] = b
            p += len(b)
        for o, a, _ in tblobs:
            out[o:o + a.nbytes] = a.tobytes()
        return bytes(out)

    def write(self, dst):
        data = self.to_bytes()
        with open(dst, "wb") as f:
            f.write(data)
        return len(data)


def read(src):
    """Parses a package file: dict with meta, tensors, paths (for tests)."""
    data = open(src, "rb").read() if isinstance(src, str) else bytes(src)
    magic, bom, ver, minr, n_meta, n_t, n_p, _, moff, toff, poff, size = HDR.unpack_from(data)
    assert magic == MAGIC and bom == 0x01020304 and size == len(data)
    meta, q = {}, moff
    for _ in range(n_meta):
        kl, ty, vl = struct.unpack_from("<HHI", data, q)
        key = data[q + 8:q + 8 + kl].decode()
        v = data[q + 8 + kl:q + 8 + kl + vl]
        meta[key] = (v.decode() if ty == 0 else struct.unpack("<q", v)[0] if ty == 1
                     else struct.unpack("<d", v)[0] if ty == 2 else v)
        q += (8 + kl + vl + 7) & ~7
    tensors = []
    for i in range(n_t):
        name, dt, nd, d0, d1, d2, d3, off, nb, _ = TENSOR.unpack_from(data, toff + TENSOR.size * i)
        shape = [d0, d1, d2, d3][:nd]
        arr = np.frombuffer(data, NP_DTYPE[dt], count=int(np.prod(shape)) if shape else 1,
                            offset=off).reshape(shape)
        tensors.append((name.rstrip(b"\0").decode(), arr, nb))
    paths = []
    for i in range(n_p):
        name, hw, nbuf, nops, obytes, ib, ob, eb, _, boff, ooff = PATH.unpack_from(data, poff + PATH.size * i)
        bufs = [BUF.unpack_from(data, boff + BUF.size * j) for j in range(nbuf)]
        ops, q = [], ooff
        for _ in range(nops):
            code, rb, nb_, nt, ni, _ = struct.unpack_from("<6H", data, q)
            vals = struct.unpack_from(f"<{nb_ + nt + ni}i", data, q + 12)
            ops.append((code, list(vals[:nb_]), list(vals[nb_:nb_ + nt]), list(vals[nb_ + nt:])))
            q += rb
        paths.append({"name": name.rstrip(b"\0").decode(), "hwcap": hw, "bufs": bufs,
                      "ops": ops, "in": ib, "out": ob, "emb": None if eb == 0xffffffff else eb})
    return {"version": ver, "min_reader": minr, "meta": meta, "tensors": tensors, "paths": paths}
