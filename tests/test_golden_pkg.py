"""The .bnpk byte layout against a package written by the reference
compiler's own writer (tests/golden/pkg_two_paths.bnpk, made by
tests/golden/make_golden.py from golden_pkg.build): this library's writer
must produce the same bytes from the same records, its C loader must read
the reference-written file (metadata of every type, both paths, source-node
lines), and on the GPU both paths must score windows as the oracle does."""
import os
import sys

import numpy as np
import pytest

from bnneon import binding, pkgfmt

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
sys.path.insert(0, GOLDEN)
import golden_pkg  # noqa: E402  (tests/golden/golden_pkg.py)

FIXTURE = os.path.join(GOLDEN, "pkg_two_paths.bnpk")


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn])


def test_writer_reproduces_reference_bytes():
    pkg = pkgfmt.Package()
    golden_pkg.build(pkg)
    ours = pkg.to_bytes()
    ref = open(FIXTURE, "rb").read()
    assert len(ours) == len(ref)
    if ours != ref:
        first = next(i for i in range(len(ref)) if ours[i] != ref[i])
        pytest.fail(f"first differing byte at offset {first}")


def test_reader_parses_reference_package():
    r = pkgfmt.read(FIXTURE)
    m = r["meta"]
    assert m["model_id"] == "golden_two_paths" and m["n_samples"] == golden_pkg.M * golden_pkg.K0
    assert m["logit_scale"] == 0.75 and m["calibrated"] == 1 and m["labels"] == golden_pkg.LABELS
    assert [p["name"] for p in r["paths"]] == ["neon-int8", "neon-fp32"]
    assert [op[0] for op in r["paths"][0]["ops"]] == [22, 22, 35] and r["paths"][1]["ops"][0][0] == 23


def test_c_loader_reads_reference_package(tmp_path):
    info = binding.probe(FIXTURE)
    assert info.format_version == 1 and info.n_samples == golden_pkg.M * golden_pkg.K0
    assert info.n_classes == golden_pkg.NC and info.logit_scale == 0.75
    assert info.model_id == b"golden_two_paths" and info.path == b"neon-int8" and info.has_labels_sha
    assert binding.probe_meta(FIXTURE, "calibrated") == "1"
    assert binding.probe_meta(FIXTURE, "logit_scale") == "0.75"
    assert binding.probe_meta(FIXTURE, "licence").startswith("synthetic")
    assert binding.probe_meta(FIXTURE, "labels", raw=True) == golden_pkg.LABELS
    L = binding.load_library()
    lab = tmp_path / "labels.txt"
    lab.write_bytes(golden_pkg.LABELS)
    assert L.bnn_verify_labels(FIXTURE.encode(), str(lab).encode()) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("mode,path", [(binding.MODE_INT8, "neon-int8"), (binding.MODE_FP32, "neon-fp32")])
def test_reference_package_scores_as_the_oracle(hip, mode, path):
    import oracle_net
    pkg = pkgfmt.Package()
    nets = golden_pkg.build(pkg)
    net = nets[0] if path == "neon-int8" else nets[1]
    on = oracle_net.OracleNet(net, 0, net.last)
    rng = np.random.default_rng(5)
    pcm = rng.standard_normal((40, golden_pkg.M * golden_pkg.K0)).astype(np.float32)
    print("golden package", path, flush=True)
    with binding.Model(FIXTURE, mode) as m:
        assert m.info.path == path.encode()
        out, _, status = m.infer_batch(pcm)
        assert not status.any()
        for w in (0, 17, 39):
            ref, _, _ = on.run(pcm[w])
            assert same(out[w], ref[:golden_pkg.NC]), w


FIXTURE3 = os.path.join(GOLDEN, "pkg_three_paths.bnpk")


def test_three_path_fixture_bytes_and_mode0():
    """pkg_three_paths.bnpk (fp16, fp32, int8 paths, fastest first): this library's writer gives the same bytes; the
    reader sees the paths in order with their prototype-head opcodes; mode 0 (bnn_probe's choice) takes the first
    path, whose every op the GPU serves"""
    pkg = pkgfmt.Package()
    golden_pkg.build3(pkg)
    assert pkg.to_bytes() == open(FIXTURE3, "rb").read()
    r = pkgfmt.read(FIXTURE3)
    assert [p["name"] for p in r["paths"]] == ["neon-fp16", "neon-fp32", "neon-int8"]
    assert [op[0] for op in r["paths"][0]["ops"]] == [9 | 1 << 8, 13 | 1 << 8]
    assert [op[0] for op in r["paths"][1]["ops"]] == [3, 13]
    assert [op[0] for op in r["paths"][2]["ops"]] == [22, 35]
    assert binding.probe(FIXTURE3).path == b"neon-fp16"


@pytest.mark.gpu
@pytest.mark.parametrize("mode,path", [(binding.MODE_DEFAULT, "neon-fp16"), (binding.MODE_FP16, "neon-fp16"),
                                       (binding.MODE_FP32, "neon-fp32"), (binding.MODE_INT8, "neon-int8")])
def test_three_path_package_scores_as_the_oracle(hip, mode, path):
    import oracle_net
    pkg = pkgfmt.Package()
    nets = dict(zip(("neon-fp16", "neon-fp32", "neon-int8"), golden_pkg.build3(pkg)))
    net, ib = nets[path]
    on = oracle_net.OracleNet(net, ib, net.last)
    rng = np.random.default_rng(6)
    pcm = rng.standard_normal((70, golden_pkg.H3 * golden_pkg.W3)).astype(np.float32)
    print("golden three-path package", mode, path, flush=True)
    with binding.Model(FIXTURE3, mode) as m:
        assert m.info.path == path.encode()
        out, _, status = m.infer_batch(pcm)
        assert not status.any()
        for w in (0, 35, 69):
            ref, _, _ = on.run(pcm[w])
            assert same(out[w], ref[:golden_pkg.NC]), w
