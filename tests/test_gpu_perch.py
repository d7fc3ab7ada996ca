"""The Perch-v2-shaped int8 network end to end on the GPU (bnn_init /
bnn_infer_batch on a .bnpk built by bnneon.perchnet): FE_LOGMEL, STEM,
DW3 / DWK, SE_GATE, PW_S8 (gated, residual), PAD, MEAN and GEMV_S8 over 26
MBConv blocks, logits and embeddings bit-identical to the oracle's op-by-op
run of the same package, and identical whatever the batch size."""
import numpy as np
import pytest

from bnneon import binding, perchnet

import oracle_net  # oracle/oracle_net.py

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn])


@pytest.fixture(scope="module")
def perch(tmp_path_factory):
    pn = perchnet.PerchNet(seed=3)
    path = pn.write(str(tmp_path_factory.mktemp("perch") / "perch_s8.bnpk"))
    return pn, path


def test_perch_batch_bit_exact(hip, perch):
    pn, path = perch
    rng = np.random.default_rng(4)
    B = 6
    pcm = np.stack([perchnet.signal(rng) for _ in range(B)])
    pcm[1] = 0.0                 # silence: every frame at the log floor
    pcm[2, 1000] = 0.9           # a click
    on = oracle_net.OracleNet(pn.net, 0, pn.net.last, pn.emb_buf)
    say("perch batch", B)
    with binding.Model(path) as m:
        assert m.info.n_classes == perchnet.N_CLASSES and m.info.emb_dim == perchnet.EMB
        out, emb, status = m.infer_batch(pcm)
        assert not status.any()
        for w in (0, 1, 2):
            ref, ref_emb, _ = on.run(pcm[w])
            say("window", w)
            assert same(out[w], ref[:perchnet.N_CLASSES]), w
            assert same(emb[w], ref_emb[:perchnet.EMB]), w
        # the same windows one at a time and in another batch split
        for w in (3, 5):
            o1, e1, s1 = m.infer_batch(pcm[w:w + 1])
            assert not s1.any() and same(o1[0], out[w]) and same(e1[0], emb[w])
        o2, e2, s2 = m.infer_batch(pcm[2:6])
        assert not s2.any() and same(o2, out[2:6]) and same(e2, emb[2:6])


def test_perch_two_stream_batch(hip, perch):
    """72 windows run as two halves on two streams: the bytes of the same windows in batches of 24 (one stream)."""
    pn, path = perch
    rng = np.random.default_rng(9)
    pcm = np.stack([perchnet.signal(rng) for _ in range(72)])
    say("perch two-stream batch 72")
    with binding.Model(path) as m:
        out, emb, status = m.infer_batch(pcm)
        assert not status.any()
        for lo in (0, 24, 48):
            o, e, s = m.infer_batch(pcm[lo:lo + 24])
            assert not s.any() and same(o, out[lo:lo + 24]) and same(e, emb[lo:lo + 24]), lo
        # the same 72 windows read from device memory where the caller keeps them (stride n_samples)
        dp = hip.DeviceArray.from_host(pcm)
        do = hip.DeviceArray.zeros((72, m.info.n_classes), np.float32)
        de = hip.DeviceArray.zeros((72, m.info.emb_dim), np.float32)
        st = np.zeros(72, np.int32)
        r = m.L.bnn_infer_batch_device(m.ctx, dp.ptr, 72, do.ptr, de.ptr, st.ctypes.data_as(binding._IP), None)
        assert r == 0 and not st.any()
        assert same(do.numpy(), out) and same(de.numpy(), emb)


def test_perch_fused_expansions(hip, perch, monkeypatch, capfd):
    """Each of the 24 expansions runs inside its depthwise conv (one kernel, the expanded tensor never stored), and
    the outputs are the bytes of the op list run as written (BNH_FUSE=0)."""
    pn, path = perch
    rng = np.random.default_rng(11)
    pcm = np.stack([perchnet.signal(rng) for _ in range(8)])
    say("perch fused vs op by op")
    monkeypatch.setenv("BNN_PROF", "2")
    with binding.Model(path) as m:
        out, emb, status = m.infer_batch(pcm)
    err = capfd.readouterr().err
    assert err.count("[fused: computes op") == 24 and err.count("[quantizes only]") == 24, err[-2000:]
    monkeypatch.delenv("BNN_PROF")
    monkeypatch.setenv("BNH_FUSE", "0")
    with binding.Model(path) as m:
        o2, e2, s2 = m.infer_batch(pcm)
    assert not status.any() and not s2.any()
    assert same(out, o2) and same(emb, e2)
