"""Content of the golden package fixture pkg_two_paths.bnpk.

build(pkg) fills any object with the package writer's interface (set, tensor,
add_path) with the same records from fixed seeds: make_golden.py hands it the
reference compiler's writer (python/bnneon/compiler/pkgfmt.py) to write the
fixture once; the tests hand it this library's writer (bnneon/pkgfmt.py) and
require the same bytes, then load the fixture through the C API.

Two paths over one input window of M x K0 fp32 rows:
  "neon-int8": PW_S8 (SiLU) -> PW_S8 -> PROTO_S8 (100 classes, 4 prototypes each)
  "neon-fp32": GEMV_S8 of the whole window (K = M K0) -> 100 logits
Metadata records of every type: text, integers, a bool, a double, bytes.
"""
import numpy as np

from bnneon import netbuild

M, K0, K1, K2, NC, PPC = 32, 40, 136, 48, 100, 4
LABELS = b"".join(b"Species %03d_Common name %03d\n" % (i, i) for i in range(NC))


def build(pkg):
    """Adds the fixture's metadata, tensors and paths to pkg; returns the two netbuild.Net objects."""
    rng = np.random.default_rng(20241202)
    w1 = rng.standard_normal((K1, K0)).astype(np.float32) * 0.3
    b1 = rng.standard_normal(K1).astype(np.float32) * 0.1
    w2 = rng.standard_normal((K2, K1)).astype(np.float32) * 0.1
    b2 = rng.standard_normal(K2).astype(np.float32) * 0.1
    protos = rng.standard_normal((NC * PPC, K2)).astype(np.float32)
    clsw = rng.uniform(0.5, 1.5, NC * PPC).astype(np.float32)
    clsb = rng.standard_normal(NC).astype(np.float32)
    wl = rng.standard_normal((NC, M * K0)).astype(np.float32) * 0.02
    bl = rng.standard_normal(NC).astype(np.float32)

    a = netbuild.Net(pkg, prefix="a/")
    ib = a.buf(netbuild.F32, M, 1, K0)
    h1 = a.pw_s8(ib, w1, b1, act="silu")
    h2 = a.pw_s8(h1, w2, b2)
    a.proto_s8(h2, protos, clsw, clsb)
    a.add_to("neon-int8", 0, in_buf=ib)

    b = netbuild.Net(pkg, prefix="b/")
    jb = b.buf(netbuild.F32, 1, 1, M * K0)
    b.gemv_s8(jb, wl, bl)
    b.add_to("neon-fp32", 0, in_buf=jb)

    netbuild.standard_meta(pkg, M * K0, NC, labels=LABELS, model_id="golden_two_paths")
    pkg.set("logit_scale", 0.75)
    pkg.set("calibrated", True)
    pkg.set("note", "written by the reference compiler's package writer")
    pkg.set("src_nodes/neon-int8", "'/pw1/Conv'\n'/pw2/Conv'\n'/proto/MatMul'\n")
    return a, b
