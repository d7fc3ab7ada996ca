"""The .bnpk boundary on the CPU: the package writer / reader, bnn_probe and
its metadata, label verification, and the loader's refusals of corrupt files
(the reference's error contract: src/rt_pkg.c:30-102, src/bnneon.c:147-190,
332-363; tests/test_errors.py mutates packages the same way)."""
import hashlib
import os
import struct

import numpy as np
import pytest

from bnneon import binding, netbuild, pkgfmt

LABELS = b"Turdus merula_Eurasian Blackbird\nErithacus rubecula_European Robin\n"


def small_package(path, n_classes=2):
    rng = np.random.default_rng(0)
    pkg = pkgfmt.Package()
    net = netbuild.Net(pkg)
    K, N = 40, n_classes
    ib = net.buf(netbuild.F32, 1, 1, K)
    net.gemv_s8(ib, rng.standard_normal((N, K)), rng.standard_normal(N))
    net.add_to("neon-int8", 0, in_buf=ib)
    netbuild.standard_meta(pkg, K, N, labels=LABELS, model_id="tiny_gemv")
    pkg.write(path)
    return path


def test_writer_reader_roundtrip(tmp_path):
    p = small_package(str(tmp_path / "t.bnpk"))
    r = pkgfmt.read(p)
    assert r["meta"]["n_samples"] == 40 and r["meta"]["model_id"] == "tiny_gemv"
    assert [t[0].split(".")[0] for t in r["tensors"]] == ["s8n/lin"] * 4
    assert r["paths"][0]["name"] == "neon-int8" and r["paths"][0]["ops"][0][0] == 23
    data = open(p, "rb").read()
    for name, arr, nb in r["tensors"]:
        off = data.index(arr.tobytes()) if arr.nbytes else 0
        assert off % 64 == 0


def test_probe_and_meta(tmp_path):
    p = small_package(str(tmp_path / "t.bnpk"))
    info = binding.probe(p)
    assert info.format_version == 1 and info.n_samples == 40 and info.n_classes == 2
    assert info.model_id == b"tiny_gemv" and info.path == b"neon-int8"
    assert info.has_labels_sha and bytes(info.labels_sha256) == hashlib.sha256(LABELS).digest()
    assert binding.probe_meta(p, "license").startswith("synthetic")
    assert binding.probe_meta(p, "licence") == binding.probe_meta(p, "license")
    assert binding.probe_meta(p, "n_classes") == "2"
    assert binding.probe_meta(p, "labels", raw=True) == LABELS
    assert binding.probe_meta(p, "nope") is None


def test_verify_labels(tmp_path):
    p = small_package(str(tmp_path / "t.bnpk"))
    good = tmp_path / "labels.txt"
    good.write_bytes(LABELS)
    L = binding.load_library()
    assert L.bnn_verify_labels(p.encode(), str(good).encode()) == 0
    bad = tmp_path / "other.txt"
    bad.write_bytes(LABELS + b"x\n")
    assert L.bnn_verify_labels(p.encode(), str(bad).encode()) == -1
    msg = L.bnn_last_error().decode()
    assert "is not the label file" in msg and "3 lines" in msg
    assert binding.ERR_KINDS[L.bnn_last_error_kind()] == "labels"


def mutate(path, dst, off, fmt, value):
    data = bytearray(open(path, "rb").read())
    struct.pack_into(fmt, data, off, value)
    open(dst, "wb").write(data)
    return dst


@pytest.mark.parametrize("what,off,fmt,value,expect", [
    ("magic", 0, "<8s", b"BNNPKG99", "not a bnneon weights file"),
    ("bom", 8, "<I", 0x04030201, "byte-order mark"),
    ("reader", 14, "<H", 7, "needs reader version 7"),
    ("paths", 24, "<I", 9, "corrupt header"),
    ("size", 56, "<Q", 1 << 40, "package truncated"),
])
def test_corrupt_headers_are_refused(tmp_path, what, off, fmt, value, expect):
    p = small_package(str(tmp_path / "t.bnpk"))
    bad = mutate(p, str(tmp_path / f"bad_{what}.bnpk"), off, fmt, value)
    with pytest.raises(binding.BnnError) as e:
        binding.probe(bad)
    assert expect in str(e.value) and e.value.kind == "package"


def test_truncated_and_tensor_outside(tmp_path):
    p = small_package(str(tmp_path / "t.bnpk"))
    data = open(p, "rb").read()
    short = tmp_path / "short.bnpk"
    short.write_bytes(data[:40])
    with pytest.raises(binding.BnnError, match="smaller than a package header"):
        binding.probe(str(short))
    cut = tmp_path / "cut.bnpk"
    cut.write_bytes(data[:-64])
    with pytest.raises(binding.BnnError, match="truncated"):
        binding.probe(str(cut))
    r = pkgfmt.read(p)
    toff = struct.unpack_from("<Q", data, 40)[0]
    bad = mutate(p, str(tmp_path / "tout.bnpk"), toff + 72, "<Q", len(data) + 4096)
    with pytest.raises(binding.BnnError, match="lies outside the file"):
        binding.probe(bad)


def test_legacy_files_refused(tmp_path):
    f = tmp_path / "old.bn24"
    f.write_bytes(b"BN24ENG1" + bytes(64))
    with pytest.raises(binding.BnnError, match="legacy BirdNET v2.4"):
        binding.probe(str(f))


def test_init_mode_and_device_errors(tmp_path):
    p = small_package(str(tmp_path / "t.bnpk"))
    with pytest.raises(binding.BnnError) as e:
        binding.Model(p, binding.MODE_REFERENCE)
    assert e.value.kind == "usage"
    L = binding.load_library()
    if L.bnh_device_count() == 0:
        with pytest.raises(binding.BnnError) as e:
            binding.Model(p)
        assert e.value.kind == "cpu" and "no HIP device" in str(e.value)


def test_api_version_and_threads_symbol():
    L = binding.load_library()
    assert L.bnn_api_version() == 2
    assert L.bnn_set_threads(None, 2) == -1


def test_mode0_passes_over_unserved_paths(tmp_path):
    """Mode 0 takes the first path (packages store them fastest first, src/bnneon.c:79-89) whose every op this
    library serves: a neon-fp16 path whose first op is the v3.0 front end FE_DBIMG (not served on the GPU) is passed
    over for the neon-int8 path behind it; a package of that path alone still names it, so init names the op."""
    rng = np.random.default_rng(4)
    K, N = 40, 3
    pkg = pkgfmt.Package()
    a = netbuild.Net(pkg, prefix="a/")
    ia = a.buf(netbuild.F32, 1, 1, K)
    oa = a.buf(netbuild.F32, 1, 1, N)
    a.emit(16, [ia, oa], [], [K, N])   # FE_DBIMG
    a.add_to("neon-fp16", netbuild.HW_FP16, in_buf=ia, out_buf=oa)
    b = netbuild.Net(pkg, prefix="b/")
    ib = b.buf(netbuild.F32, 1, 1, K)
    b.gemv_s8(ib, rng.standard_normal((N, K)), rng.standard_normal(N))
    b.add_to("neon-int8", 0, in_buf=ib)
    netbuild.standard_meta(pkg, K, N, model_id="two_paths_one_served")
    p = str(tmp_path / "t.bnpk")
    pkg.write(p)
    assert binding.probe(p).path == b"neon-int8"

    pkg = pkgfmt.Package()
    a = netbuild.Net(pkg)
    ia = a.buf(netbuild.F32, 1, 1, K)
    oa = a.buf(netbuild.F32, 1, 1, N)
    a.emit(16, [ia, oa], [], [K, N])
    a.add_to("neon-fp16", netbuild.HW_FP16, in_buf=ia, out_buf=oa)
    netbuild.standard_meta(pkg, K, N, model_id="one_unserved_path")
    p = str(tmp_path / "u.bnpk")
    pkg.write(p)
    assert binding.probe(p).path == b"neon-fp16"
