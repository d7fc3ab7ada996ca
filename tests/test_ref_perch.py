"""The Perch-shaped nets against the reference's own scalar fp32 oracle (src/perch_ref.c), on the CPU.

oracle/_ref/libperchref.so is the reference's perch_ref.c and perch_model.c compiled from the reference checkout
(`make -C oracle ref`); the nets' float weights are written in the reference's .bnp2 layout
(src/perch_model.c:43-141) and scored by pc_ref_infer (src/perch_ref.c:382): exact double FFT front end, the
graph in NHWC fp32, the ProtoPNet head. The same weights as a package run op by op on this repository's oracle,
which the GPU matches bit for bit (tests/test_gpu_perch.py, tests/test_gpu_fproto.py).

Two geometries:
  * SHALLOW: 6 blocks (k 3 / 5, four stride-2 blocks, two residual ones) to the 16 x 4 x 384 body output the loader
    requires, unit-gain projections: the embedding follows its input (another window moves it by ~2 %, a transposed
    stem by ~2 %, a 1e-7 relative change of the pcm by ~2e-7), so a layout, pad or wiring slip shows;
  * FULL: the benched net's 26 blocks at its own scaling (a deep random stack that keeps little of its input, so it
    pins the whole geometry chain: every block's shapes, pads and residual flag, checked by the reference's loader).
Stated tolerances:
  * neon-fp32 packages (fp32 1x1 convs, fp32 prototype head): the sides differ only in roundings (fp32 radix FFT
    against the exact double FFT, the engine's SiLU against x / (1 + expf(-x)), summation orders):
    |d emb| <= 2e-5 max|emb| and |d logit| <= 1e-5 (1 + max|logit|) (measured 4e-6 and 2e-6 / 1e-7);
  * a neon-int8 package (int8 1x1 convs and prototype head) against the fp32 oracle, the quantisation of every 1x1
    conv input and weight: embedding within 3 % in L2 (cosine >= 0.999), logits within 2 % of their range, the
    same top class (measured 0.9 %, 0.99996, 0.3 %).
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [os.path.join(ROOT, "oracle", "ref")]

import perchref  # noqa: E402
from bnneon import perchnet  # noqa: E402
import oracle_net  # noqa: E402

pytestmark = pytest.mark.skipif(not perchref.available(),
                                 reason="oracle/_ref/libperchref.so not built (needs the reference checkout)")
NC, PPC = 16, 2
SHALLOW = [(1, 3, 2, 24, 1), (6, 5, 2, 48, 2), (6, 3, 2, 96, 2), (6, 5, 2, 384, 1)]


def ref_run(pn, path, pcm):
    perchref.write_bnp2(path, pn)
    m = perchref.Model(path)
    try:
        return m.infer(pcm)
    finally:
        m.close()


def ours(pn, pcm):
    lg, emb, _ = oracle_net.OracleNet(pn.net, 0, pn.net.last, pn.emb_buf).run(pcm)
    return lg[:NC], emb[:perchref.EMB]


def fp32_close(lg_o, emb_o, lg_r, emb_r):
    return (np.abs(emb_o - emb_r).max() <= 2e-5 * np.abs(emb_r).max() and
            np.abs(lg_o - lg_r).max() <= 1e-5 * (1 + np.abs(lg_r).max()))


@pytest.mark.parametrize("geometry", ["shallow", "full"])
def test_fp32_net_matches_reference_oracle(tmp_path, geometry):
    kw = dict(stages=SHALLOW, pj_gain=1.0) if geometry == "shallow" else {}
    pn = perchnet.PerchNet(seed=5, n_classes=NC, kind="f32", head="proto", ppc=PPC, **kw)
    pcm = perchnet.signal(np.random.default_rng(11))
    lg_r, emb_r = ref_run(pn, str(tmp_path / "f32.bnp2"), pcm)
    lg_o, emb_o = ours(pn, pcm)
    assert np.abs(emb_r).max() > 0.05 and np.ptp(lg_r) > 0.05  # not a comparison of near-zero vectors
    assert fp32_close(lg_o, emb_o, lg_r, emb_r), (float(np.abs(emb_o - emb_r).max() / np.abs(emb_r).max()),
                                                   float(np.abs(lg_o - lg_r).max()))


def test_int8_net_within_quantisation_tolerance(tmp_path):
    pn = perchnet.PerchNet(seed=5, n_classes=NC, kind="int8", head="proto", ppc=PPC, stages=SHALLOW, pj_gain=1.0)
    pcm = perchnet.signal(np.random.default_rng(12))
    lg_r, emb_r = ref_run(pn, str(tmp_path / "i8.bnp2"), pcm)
    lg_o, emb_o = ours(pn, pcm)
    rel = np.linalg.norm(emb_o - emb_r) / np.linalg.norm(emb_r)
    cos = float(emb_o @ emb_r) / float(np.linalg.norm(emb_o) * np.linalg.norm(emb_r))
    assert rel <= 0.03 and cos >= 0.999, (rel, cos)
    assert np.abs(lg_o - lg_r).max() <= 0.02 * np.ptp(lg_r)
    assert np.argmax(lg_o) == np.argmax(lg_r)


def test_a_layout_slip_is_seen(tmp_path):
    """The fp32 comparison discriminates: the stem's 3 x 3 taps transposed in the reference's file (a row / column
    slip of the kind a layout mistake makes) fall far outside the bound."""
    pn = perchnet.PerchNet(seed=5, n_classes=NC, kind="f32", head="proto", ppc=PPC, stages=SHALLOW, pj_gain=1.0)
    pcm = perchnet.signal(np.random.default_rng(11))
    lg_o, emb_o = ours(pn, pcm)
    w = dict(pn.fw)["stem.w"]
    w[:] = w.reshape(-1, 3, 3).transpose(0, 2, 1).reshape(w.shape)
    lg_r, emb_r = ref_run(pn, str(tmp_path / "slip.bnp2"), pcm)
    assert np.abs(emb_o - emb_r).max() > 100 * 2e-5 * np.abs(emb_r).max()
    assert not fp32_close(lg_o, emb_o, lg_r, emb_r)
