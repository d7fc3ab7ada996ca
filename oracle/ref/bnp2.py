"""Writes a Perch v2 engine weight file (.bnp2), the input of the reference's own scalar oracle.

Test infrastructure: the layout is the one src/perch_model.c:43-141 reads and scripts/export_perch.py:12-31
documents (little endian): magic "BNP2ENG1"; u32 version 1, n_tensors, n_classes, n_blocks, license_len; the
license (padded to 8); the label file's sha256 (32 bytes); the block table, 8 i32 per block {k, stride, cin,
cexp (0 = no expansion conv), cout, se_rd, skip, pads = top | left << 8 | bottom << 16 | right << 24}; the tensor
directory, per tensor {char name[48]; u32 dtype (0 = f32); u32 ndim; u32 dims[4]; u64 offset; u64 nbytes}; each
tensor's fp32 data 64-byte aligned at its offset from the file start.
"""
import struct

import numpy as np

MAGIC = b"BNP2ENG1"
DIR_ENTRY = struct.Struct("<48sII4IQQ")


def fe_consts(frame, hop, pad, nfft, log_floor, log_scale, norm_eps, ppc):
    """The fe.consts tensor: the front end's and the prototype head's constants."""
    return np.array([frame, hop, pad, nfft, log_floor, log_scale, norm_eps, ppc], np.float32)


def write(path, tensors, blocks, n_classes, license_text=b"synthetic weights", labels_sha=b"\0" * 32):
    """tensors: (name, array) pairs, fp32; blocks: the block table rows. Returns the file size."""
    lic = license_text + b"\0" * ((8 - len(license_text) % 8) % 8)
    head = MAGIC + struct.pack("<5I", 1, len(tensors), n_classes, len(blocks), len(lic)) + lic + labels_sha
    head += b"".join(struct.pack("<8i", *row) for row in blocks)
    off = (len(head) + len(tensors) * DIR_ENTRY.size + 63) & ~63
    entries, data = [], []
    for name, a in tensors:
        a = np.ascontiguousarray(a, np.float32)
        dims = list(a.shape) + [0] * (4 - a.ndim)
        entries.append(DIR_ENTRY.pack(name.encode(), 0, a.ndim, *dims, off, a.nbytes))
        data.append((off, a))
        off = (off + a.nbytes + 63) & ~63
    with open(path, "wb") as f:
        f.write(head + b"".join(entries))
        for o, a in data:
            f.write(b"\0" * (o - f.tell()))
            f.write(a.tobytes())
    return off
