"""The drop-in boundary on the GPU: .bnpk packages through bnn_init /
bnn_infer / bnn_infer_batch on libbnneon_hip, every output compared bit for
bit with the oracle's op-by-op restatement of the reference library, plus the
load-time refusals and failed-window reporting of the reference's contract."""
import numpy as np
import pytest

import pyoracle as O
from bnneon import binding, hip, netbuild, pkgfmt, s8pack

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


class Spec:
    """A synthetic int8 net: rows [M][K0] -> PW_S8 (SiLU) -> PW_S8 -> PROTO_S8."""

    def __init__(self, seed=0, M=64, K0=40, K1=136, K2=48, nc=100, ppc=4):
        rng = np.random.default_rng(seed)
        self.M, self.K0, self.nc, self.ppc = M, K0, nc, ppc
        self.w1 = rng.standard_normal((K1, K0)).astype(np.float32) * 0.3
        self.b1 = rng.standard_normal(K1).astype(np.float32) * 0.1
        self.w2 = rng.standard_normal((K2, K1)).astype(np.float32) * 0.1
        self.b2 = rng.standard_normal(K2).astype(np.float32) * 0.1
        self.protos = rng.standard_normal((nc * ppc, K2)).astype(np.float32)
        self.clsw = rng.uniform(0.5, 1.5, nc * ppc).astype(np.float32)
        self.clsb = rng.standard_normal(nc).astype(np.float32)
        self.pk1 = s8pack.pack_s8(self.w1, self.b1)
        self.pk2 = s8pack.pack_s8(self.w2, self.b2)

    def package(self, path, n4=None):
        pkg = pkgfmt.Package()
        net = netbuild.Net(pkg)
        ib = net.buf(netbuild.F32, self.M, 1, self.K0)
        h1 = net.pw_s8(ib, self.w1, self.b1, act="silu")
        h2 = net.pw_s8(h1, self.w2, self.b2)
        net.proto_s8(h2, self.protos, self.clsw, self.clsb, n4=n4)
        net.add_to("neon-int8", 0, in_buf=ib)
        netbuild.standard_meta(pkg, self.M * self.K0, self.nc, model_id="synthetic_int8_proto")
        pkg.write(path)
        return path

    def oracle(self, pcm):
        x = pcm.reshape(self.M, self.K0)
        h1, *_ = O.pw_s8(x, self.pk1, act=1)
        h2, *_ = O.pw_s8(h1, self.pk2)
        N, K = self.protos.shape
        Kp, Np = s8pack.r16(K), (N + 3) // 4 * 4
        q, sw = s8pack.quant_rows_s8(self.protos)
        qp = np.zeros((Np, Kp), np.int8)
        qp[:N, :K] = q
        swp = np.zeros(Np, np.float32)
        swp[:N] = sw
        rc, lg, _, _ = O.proto_s8(h2, K, 1e-5, s8pack.pack_panels(qp), swp, Np, Kp, self.clsw, self.clsb,
                                  self.nc, self.ppc)
        return rc, lg


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return np.array_equal(an, bn) and np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn])


def test_batch_of_windows_bit_exact(hip, tmp_path):
    spec = Spec(1)
    path = spec.package(str(tmp_path / "net.bnpk"))
    rng = np.random.default_rng(2)
    pcm = (rng.standard_normal((37, spec.M * spec.K0)) * 0.5).astype(np.float32)
    say("runtime batch 37")
    with binding.Model(path) as m:
        assert m.info.path == b"neon-int8" and m.info.precision == b"int8 GEMMs, fp32 elsewhere"
        out, _, status = m.infer_batch(pcm)
        assert not status.any()
        for w in range(37):
            rc, ref = spec.oracle(pcm[w])
            assert rc == 0 and same(out[w], ref), w
        # one window at a time gives the same bytes; a smaller batch after a larger one too
        single, _ = m.infer(pcm[5])
        assert same(single, out[5])
        out2, _, _ = m.infer_batch(pcm[:3])
        assert same(out2, out[:3])


def test_failed_window_is_reported(hip, tmp_path):
    spec = Spec(3)
    path = spec.package(str(tmp_path / "net.bnpk"))
    rng = np.random.default_rng(4)
    pcm = rng.standard_normal((6, spec.M * spec.K0)).astype(np.float32)
    # an inf or NaN in the input is washed out by the next layer's quantization
    # (a NaN row quantizes to its bias); values near fp32's limit are not:
    # the dequantized layer-1 row overflows to +-inf, the layer-2 row to NaN,
    # and the prototype cells and logits follow
    pcm[4] = np.where(np.arange(pcm.shape[1]) % 2, -1.5e38, 1.5e38)
    ref_rc = [spec.oracle(p)[0] for p in pcm]
    assert ref_rc[4] == -2 and ref_rc.count(0) == 5
    say("runtime failed window", ref_rc)
    with binding.Model(path) as m:
        out, _, status = m.infer_batch(pcm, check=False)
        assert [int(s != 0) for s in status] == [int(r != 0) for r in ref_rc]
        assert status[4] == 3           # 1 + the index of PROTO_S8 in the op list
        with pytest.raises(binding.BnnError) as e:
            m.infer_batch(pcm)
        assert e.value.kind == "window" and "op 2 proto_s8n" in str(e.value) and "window 4 of 6" in str(e.value)
        for w in range(6):
            assert same(out[w], spec.oracle(pcm[w])[1])


def test_large_batch_two_streams(hip, tmp_path):
    """From 64 windows up a batch runs as two halves on two streams: the same bytes and failure flags as batches
    too small to split, a failing window in either half reported against its own index."""
    spec = Spec(5)
    path = spec.package(str(tmp_path / "net.bnpk"))
    rng = np.random.default_rng(6)
    B = 101
    pcm = (rng.standard_normal((B, spec.M * spec.K0)) * 0.5).astype(np.float32)
    bad = np.where(np.arange(pcm.shape[1]) % 2, -1.5e38, 1.5e38)
    pcm[7] = bad                 # first half (windows 0..50)
    pcm[77] = bad                # second half
    say("runtime two-stream batch", B)
    with binding.Model(path) as m:
        out, _, status = m.infer_batch(pcm, check=False)
        assert [w for w in range(B) if status[w]] == [7, 77] and status[77] == 3
        for lo in range(0, B, 30):       # 30 windows: one stream
            o, _, st = m.infer_batch(pcm[lo:lo + 30], check=False)
            assert same(o, out[lo:lo + 30]) and np.array_equal(st, status[lo:lo + 30]), lo
        for w in (0, 50, 51, 77, 100):
            rc, ref = spec.oracle(pcm[w])
            assert (rc != 0) == (w in (7, 77)) and same(out[w], ref), w
        with pytest.raises(binding.BnnError) as e:
            m.infer_batch(pcm)
        assert e.value.kind == "window" and "window 7 of 101" in str(e.value)


@pytest.mark.parametrize("n", [9, 72])
def test_device_resident_batch(hip, tmp_path, n):
    """Windows read where the caller keeps them (stride n_samples) give the host path's bytes; 72 windows run as two
    sub-batches, the second of which starts at window 36 of the caller's buffer."""
    spec = Spec(5)
    path = spec.package(str(tmp_path / "net.bnpk"))
    rng = np.random.default_rng(6)
    pcm = rng.standard_normal((n, spec.M * spec.K0)).astype(np.float32)
    say("runtime device batch", n)
    with binding.Model(path) as m:
        dp = hip.DeviceArray.from_host(pcm)
        do = hip.DeviceArray.zeros((n, spec.nc), np.float32)
        st = np.zeros(n, np.int32)
        r = m.L.bnn_infer_batch_device(m.ctx, dp.ptr, n, do.ptr, None, st.ctypes.data_as(binding._IP), None)
        assert r == 0
        host, _, _ = m.infer_batch(pcm)
        assert same(do.numpy(), host)
        for w in (0, n // 2, n - 1):
            _, ref = spec.oracle(pcm[w])
            assert same(host[w], ref), w


def test_forged_n4_flags_are_refused(hip, tmp_path):
    spec = Spec(7, K2=64)
    # prototype 9 gets 4 full-scale weights in one int16 lane (bytes 3, 11,
    # 19, 27 of a 32-byte step): 4 x 127 > 258, so its panel is not n4-safe
    for k in (3, 11, 19, 27):
        spec.protos[9, k] = 50.0
    q, _ = s8pack.quant_rows_s8(spec.protos)
    true_flags = s8pack.n4_panel_flags(q)
    assert true_flags[2] == 0
    first_bad = int(np.argmin(true_flags))
    path = spec.package(str(tmp_path / "forged.bnpk"), n4=np.ones_like(true_flags))
    say("runtime forged n4")
    with pytest.raises(binding.BnnError) as e:
        binding.Model(path)
    assert e.value.kind == "package" and f"prototype panel {first_bad} is flagged" in str(e.value)
    assert "op 2 proto_s8n" in str(e.value)
    # the compiler's own flags load
    ok = spec.package(str(tmp_path / "honest.bnpk"))
    binding.Model(ok).close()


def test_contract_violations_are_refused(hip, tmp_path):
    spec = Spec(8)
    path = spec.package(str(tmp_path / "net.bnpk"))
    r = pkgfmt.read(path)
    data = bytearray(open(path, "rb").read())
    # op 0 (PW_S8): its Np parameter (int param 3) no longer matches N rounded up to 8
    import struct
    poff = struct.unpack_from("<Q", data, 48)[0]
    ops_off = struct.unpack_from("<Q", data, poff + 64)[0]
    code, rb, nb, nt, ni, _ = struct.unpack_from("<6H", data, ops_off)
    struct.pack_into("<i", data, ops_off + 12 + 4 * (nb + nt + 3), 1000)
    bad = tmp_path / "bad_np.bnpk"
    bad.write_bytes(bytes(data))
    say("runtime bad Np")
    with pytest.raises(binding.BnnError) as e:
        binding.Model(str(bad))
    assert "int8 GEMM shape" in str(e.value) and "op 0 pw_s8n" in str(e.value)
    assert r["paths"][0]["ops"][0][0] == 22


@pytest.mark.parametrize("form,k,s", [("dwk", 5, 2), ("dwk", 3, 1), ("dwk", 7, 1), ("dw3", 3, 1), ("dw3", 3, 2)])
def test_pw_s8_into_depthwise(hip, tmp_path, form, k, s):
    """PW_S8 writing a zero-haloed output, then the fp32 depthwise op reading it:
    the depthwise output and its channel sums (as the embedding) bit for bit."""
    rng = np.random.default_rng(k * 10 + s)
    H, W, K0, N = 10, 13, 40, 24
    h = (k - 1) // 2
    w1 = rng.standard_normal((N, K0)).astype(np.float32) * 0.3
    b1 = rng.standard_normal(N).astype(np.float32) * 0.1
    wd = (rng.standard_normal((k * k, N)) * 0.4).astype(np.float32)
    bd = (rng.standard_normal(N) * 0.1).astype(np.float32)
    pkg = pkgfmt.Package()
    net = netbuild.Net(pkg)
    ib = net.buf(netbuild.F32, H * W, 1, K0)
    h1 = net.pw_s8(ib, w1, b1, act="silu", H=H, W=W, opad=h)
    if form == "dwk":
        ob, cb = net.dwk(h1, wd, bd, k, s)
    else:
        ob, cb = net.dw3(h1, wd, bd, s)
    _, Ho, Wo = net.bufs[ob][:3]
    net.add_to("neon-int8", 0, in_buf=ib, out_buf=ob, emb_buf=cb)
    netbuild.standard_meta(pkg, H * W * K0, Ho * Wo * N, model_id="synthetic_dw", emb_dim=N)
    path = str(tmp_path / "dw.bnpk")
    pkg.write(path)
    pcm = rng.standard_normal((5, H * W * K0)).astype(np.float32)
    say("runtime", form, k, s)
    pk = s8pack.pack_s8(w1, b1)
    with binding.Model(path) as m:
        out, emb, status = m.infer_batch(pcm)
        assert not status.any()
    for i in range(5):
        xp, *_ = O.pw_s8(pcm[i].reshape(H * W, K0), pk, act=1, ow=W, opad=h)
        xp = xp.reshape(H + 2 * h, W + 2 * h, N)
        if form == "dwk":
            pt = max((Ho - 1) * s + k - H, 0) // 2
            pl = max((Wo - 1) * s + k - W, 0) // 2
            ro, rc = O.dwk_f32(xp, H, W, N, k, s, pt, pl, wd, bd, 1, Ho, Wo)
        else:
            ro, rc = O.dw3_f32(xp, H, W, N, s, wd, bd, Ho, Wo)
        assert same(out[i], ro.reshape(-1)), i
        assert same(emb[i], rc), i


def test_host_batch_staged_chunks(hip, tmp_path):
    """300 windows from host buffers run in pinned chunks of 128 (the last one partial), each uploaded while the
    previous one runs: the same bits as calls of 37 windows (one chunk each) and as the oracle; a window of extreme
    input in the second chunk fails alone, with its status and the message"""
    spec = Spec(3)
    path = spec.package(str(tmp_path / "net.bnpk"))
    rng = np.random.default_rng(8)
    n = 300
    pcm = (rng.standard_normal((n, spec.M * spec.K0)) * 0.5).astype(np.float32)
    pcm[170] = np.where(np.arange(pcm.shape[1]) % 2, -1.5e38, 1.5e38)   # overflows to non-finite logits
    say("runtime staged host batch", n)
    with binding.Model(path) as m:
        out, _, status = m.infer_batch(pcm, check=False)
        assert [w for w in range(n) if status[w]] == [170] and status[170] == 3
        with pytest.raises(binding.BnnError) as e:
            m.infer_batch(pcm)
        assert e.value.kind == "window" and "window 170 of 300" in str(e.value)
        small = np.concatenate([m.infer_batch(pcm[i:i + 37], check=False)[0] for i in range(0, n, 37)])
    ok = [w for w in range(n) if w != 170]
    assert same(out[ok], small[ok])
    for w in (0, 127, 128, 255, 256, 299):
        rc, ref = spec.oracle(pcm[w])
        assert rc == 0 and same(out[w], ref), w


def test_stream_split_choice_keeps_bits(hip, tmp_path):
    """A context times its first batches of one size split over two streams and on one stream, then keeps the faster:
    seven calls of the same 130 windows from host buffers (the first five in the measuring order: one untimed and two
    split, then two on one stream) give bit-identical logits, equal to the oracle's"""
    spec = Spec(3)
    path = spec.package(str(tmp_path / "net.bnpk"))
    rng = np.random.default_rng(9)
    n = 130
    pcm = (rng.standard_normal((n, spec.M * spec.K0)) * 0.5).astype(np.float32)
    say("runtime split choice", n)
    with binding.Model(path) as m:
        outs = [m.infer_batch(pcm)[0] for _ in range(7)]
    for o in outs[1:]:
        assert same(o, outs[0])
    for w in (0, 64, 129):
        rc, ref = spec.oracle(pcm[w])
        assert rc == 0 and same(outs[0][w], ref), w
