"""The BirdNET-v2.4-shaped fp16 network end to end on the GPU (bnn_init /
bnn_infer_batch on a .bnpk built by bnneon.v24net, path neon-fp16):
FE_LOGMEL, STEM (fp16 output), PW (the exact fp16 GEMM: SiLU into zero-haloed
buffers, residual adds, the ReLU head conv), DW3 fp16 with TF-same offsets, SE
fp16, MEAN fp16 and the fp16-weight GEMV over 16 MBConv blocks. Every op
computes in the reference's own arithmetic, so the logits and embeddings are
bit-identical to the oracle's op-by-op run of the same package (a tolerance
would be max |logit error| <= 0 and top-1 agreement 100 %), and identical
whatever the batch size."""
import numpy as np
import pytest

from bnneon import binding, v24net

import oracle_net  # oracle/oracle_net.py

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn])


@pytest.fixture(scope="module")
def v24(tmp_path_factory):
    vn = v24net.V24Net(seed=5)
    path = vn.write(str(tmp_path_factory.mktemp("v24") / "v24_f16.bnpk"))
    return vn, path


def test_v24_batch_bit_exact(hip, v24):
    vn, path = v24
    rng = np.random.default_rng(6)
    B = 5
    pcm = np.stack([v24net.signal(rng) for _ in range(B)])
    pcm[1] = 0.0                 # silence: every frame at the log floor
    pcm[2, 777] = 0.95           # a click
    on = oracle_net.OracleNet(vn.net, 0, vn.net.last, vn.emb_buf)
    say("v24 batch", B)
    with binding.Model(path) as m:
        assert m.info.n_classes == v24net.N_CLASSES and m.info.emb_dim == v24net.EMB
        out, emb, status = m.infer_batch(pcm)
        assert not status.any()
        for w in (0, 1, 2):
            ref, ref_emb, _ = on.run(pcm[w])
            say("window", w)
            assert same(out[w], ref[:v24net.N_CLASSES]), w
            assert same(emb[w], ref_emb[:v24net.EMB]), w
        o1, e1, s1 = m.infer_batch(pcm[4:5])
        assert not s1.any() and same(o1[0], out[4]) and same(e1[0], emb[4])
        o2, e2, s2 = m.infer_batch(pcm[1:4])
        assert not s2.any() and same(o2, out[1:4]) and same(e2, emb[1:4])


def test_v24_two_stream_batch(hip, v24):
    """72 windows run as two halves on two streams (the split-K GEMM workspaces and SE scratch offset per half):
    the bytes of the same windows in batches of 24 (one stream)."""
    vn, path = v24
    rng = np.random.default_rng(10)
    pcm = np.stack([v24net.signal(rng) for _ in range(72)])
    say("v24 two-stream batch 72")
    with binding.Model(path) as m:
        out, emb, status = m.infer_batch(pcm)
        assert not status.any()
        for lo in (0, 24, 48):
            o, e, s = m.infer_batch(pcm[lo:lo + 24])
            assert not s.any() and same(o, out[lo:lo + 24]) and same(e, emb[lo:lo + 24]), lo


def test_v24_se_gates_in_the_gemm(hip, v24, monkeypatch, capfd):
    """Each of the 16 SEs computes its gates only and the projection after it applies them as it loads its rows (the
    scaled activations never written), giving the bytes of the op list run as written (BNH_FUSE=0)."""
    vn, path = v24
    rng = np.random.default_rng(12)
    pcm = np.stack([v24net.signal(rng) for _ in range(8)])
    say("v24 fused vs op by op")
    monkeypatch.setenv("BNN_PROF", "2")
    with binding.Model(path) as m:
        out, emb, status = m.infer_batch(pcm)
    err = capfd.readouterr().err
    assert err.count("[fused: applies op") == 16 and err.count("[gates only]") == 16, err[-2000:]
    monkeypatch.delenv("BNN_PROF")
    monkeypatch.setenv("BNH_FUSE", "0")
    with binding.Model(path) as m:
        o2, e2, s2 = m.infer_batch(pcm)
    assert not status.any() and not s2.any()
    assert same(out, o2) and same(emb, e2)


def test_v24_fp16_mfma_within_tolerance(hip, v24, monkeypatch):
    """BNH_F16_MFMA=1 runs every fp16 1x1 conv on fp16 MFMA with fp32 accumulation (the SE gates still applied as
    the rows load) instead of the reference's fp16 FMA chains. Over 64 windows, against the exact path: the largest
    logit error stays within 2 % of the logits' range and the top-1 class agrees on at least 62 of 64 windows."""
    vn, path = v24
    rng = np.random.default_rng(21)
    pcm = np.stack([v24net.signal(rng) for _ in range(64)])
    say("v24 fp16 MFMA vs exact, 64 windows")
    with binding.Model(path) as m:
        ref, ref_emb, s0 = m.infer_batch(pcm)
    monkeypatch.setenv("BNH_F16_MFMA", "1")
    with binding.Model(path) as m:
        got, emb, s1 = m.infer_batch(pcm)
    assert not s0.any() and not s1.any()
    d = np.abs(got.astype(np.float64) - ref)
    span = float(ref.max() - ref.min())
    top1 = int((got.argmax(1) == ref.argmax(1)).sum())
    de = float(np.abs(emb.astype(np.float64) - ref_emb).max())
    say(f"max |dlogit| {d.max():.4g} (logit range {span:.4g}, mean |dlogit| {d.mean():.3g}); top-1 agreement "
        f"{top1}/64; max |demb| {de:.4g}")
    assert not same(got, ref)   # the MFMA form really ran
    assert d.max() <= 0.02 * span, (d.max(), span)
    assert top1 >= 62, top1
