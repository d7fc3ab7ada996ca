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


# ---------------------------------------------------------------- three paths, fastest first
H3, W3, C3 = 32, 40, 24     # the window as a 32 x 40 image; 24-channel cells


def build3(pkg):
    """pkg_three_paths.bnpk: a Perch-like prototype head on three paths over one window of H3 x W3 floats, stored
    fastest first as the reference compiler stores them (src/bnneon.c:79-89):
      "neon-fp16" (fp16 requirement): STEM 5x5 (fp32 math, fp16 out, 24 ch) -> PROTO variant 1 over 28 x 36 cells
      "neon-fp32": PW fp32 (40 -> 24, SiLU) over the 32 rows -> PROTO variant 0
      "neon-int8": PW_S8 (40 -> 24, SiLU) over the 32 rows -> PROTO_S8
    Returns the three netbuild.Net objects and their input buffers."""
    rng = np.random.default_rng(20261202)
    ws = rng.standard_normal((C3, 25)).astype(np.float32) / 5
    bs = rng.standard_normal(C3).astype(np.float32) * 0.1
    wp = rng.standard_normal((C3, W3)).astype(np.float32) * 0.3
    bp = rng.standard_normal(C3).astype(np.float32) * 0.1
    protos = rng.standard_normal((NC * PPC, C3)).astype(np.float32)
    clsw = rng.uniform(0.5, 1.5, NC * PPC).astype(np.float32)
    clsb = rng.standard_normal(NC).astype(np.float32)

    h = netbuild.Net(pkg, prefix="h/")
    ih = h.buf(netbuild.F32, H3, W3, 1)
    cells = h.stem_f16(ih, ws, bs, 5, 1, ldo=C3)
    h.proto_fp(cells, protos, clsw, clsb, kind="f16")
    h.add_to("neon-fp16", netbuild.HW_FP16, in_buf=ih)

    f = netbuild.Net(pkg, prefix="f/")
    i_f = f.buf(netbuild.F32, H3, 1, W3)
    rows = f.pw(i_f, wp, bp, act="silu")
    f.proto_fp(rows, protos, clsw, clsb, kind="f32")
    f.add_to("neon-fp32", 0, in_buf=i_f)

    q = netbuild.Net(pkg, prefix="q/")
    iq = q.buf(netbuild.F32, H3, 1, W3)
    rq = q.pw_s8(iq, wp, bp, act="silu")
    q.proto_s8(rq, protos, clsw, clsb)
    q.add_to("neon-int8", 0, in_buf=iq)

    netbuild.standard_meta(pkg, H3 * W3, NC, labels=LABELS, model_id="golden_three_paths")
    pkg.set("note", "written by the reference compiler's package writer")
    return (h, ih), (f, i_f), (q, iq)
