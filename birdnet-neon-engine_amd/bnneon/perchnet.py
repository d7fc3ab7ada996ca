"""A Perch-v2-shaped int8 network as a .bnpk package, with random weights.

The geometry follows Perch v2's EfficientNet-B3 body (the layer table of
results/perch_mac_table.txt:14-77 in the reference): a 500 x 128 log-mel
front end of 5 s at 32 kHz (frame 640, hop 320, pad 160, FFT 1024), a 3 x 3
stride-2 stem to 249 x 63 x 40, 26 MBConv blocks (expand 1x1, depthwise 3x3 or
5x5 with SiLU, squeeze-excitation, project 1x1, residual when the shape
repeats) and a 384 -> 1536 head conv, then the embedding mean and a linear
classifier over ~15k classes.

The ops are the ones libbnneon's compiler emits for the neon-int8 path with
every 1x1 conv class on int8 (--int8 pw,pwl,head,lin): FE_LOGMEL, STEM,
DW3 / DWK (fp32), SE_GATE, PW_S8 (the SE gate applied as it reads its input,
the residual added in its epilogue), PAD where a depthwise input needs a halo
its producer did not write, MEAN and GEMV_S8. Weights: per output channel
N(0, sqrt(2 / fan_in)) (projections and the classifier scaled down so that
activations stay in range through the residual stack), biases N(0, 0.1).
"""
import numpy as np

from . import netbuild, pkgfmt

SR, NSAMP, FRAME, HOP, PAD, NFFT, NMEL = 32000, 160000, 640, 320, 160, 1024, 128
N_CLASSES = 14795
EMB = 1536

# (expand ratio, k, stride, out channels, repeats): EfficientNet-B3's stages at Perch's widths
STAGES = [(1, 3, 1, 24, 2), (6, 3, 2, 32, 3), (6, 5, 2, 48, 3), (6, 3, 2, 96, 5), (6, 5, 1, 136, 5),
          (6, 5, 2, 232, 6), (6, 3, 1, 384, 2)]
STEM_C = 40


def blocks(stages=None):
    """(cin, cexp, k, stride, cout) of the 26 blocks (or of the given stages)."""
    out, cin = [], STEM_C
    for e, k, s, co, n in (STAGES if stages is None else stages):
        for i in range(n):
            out.append((cin, cin * e, k, s if i == 0 else 1, co))
            cin = co
    return out


def mel_bank(nmel=NMEL, nfft=NFFT, sr=SR, fmin=60.0, fmax=16000.0):
    """Triangular filters on the mel scale, [nmel][nfft/2 + 1]."""
    bins = nfft // 2 + 1
    hz = np.linspace(0, sr / 2, bins)
    m = lambda f: 2595 * np.log10(1 + f / 700)
    pts = 700 * (10 ** (np.linspace(m(fmin), m(fmax), nmel + 2) / 2595) - 1)
    W = np.zeros((nmel, bins), np.float32)
    for j in range(nmel):
        lo, c, hi = pts[j], pts[j + 1], pts[j + 2]
        W[j] = np.maximum(0, np.minimum((hz - lo) / (c - lo), (hi - hz) / (hi - c)))
    return W


def same_pads(h, w, k, s):
    """TF 'same' output size and (top, left) pads."""
    ho, wo = (h - 1) // s + 1, (w - 1) // s + 1
    pt = max((ho - 1) * s + k - h, 0) // 2
    pl = max((wo - 1) * s + k - w, 0) // 2
    return ho, wo, pt, pl


def signal(rng, n=NSAMP, sr=SR):
    """-30 dBFS Gaussian noise plus three random linear chirps between 1 and 10 kHz."""
    x = rng.standard_normal(n) * 10 ** (-30 / 20)
    t = np.arange(n) / sr
    for _ in range(3):
        f0, f1 = rng.uniform(1000, 10000, 2)
        t0 = rng.uniform(0, n / sr * 0.7)
        d = rng.uniform(0.2, 1.0)
        on = (t >= t0) & (t < t0 + d)
        tt = t[on] - t0
        x[on] += 0.2 * np.sin(2 * np.pi * (f0 * tt + (f1 - f0) / (2 * d) * tt ** 2))
    return x.astype(np.float32)


class PerchNet:
    """The package and the float weights it was built from.

    kind "int8": the 1x1 convs on PW_S8 (the neon-int8 path, the benched net); "f32": the same graph with every 1x1
    conv an fp32 PW op (the neon-fp32 path). head "gemv": the linear classifier (GEMV_S8 for int8, GEMV for f32);
    "proto": Perch v2's ProtoPNet head (PROTO_S8 for int8, fp32 PROTO for f32) over ppc prototypes per class. The
    float weights are kept in `fw` under the reference's .bnp2 tensor names, with the block table in `blocks_table`,
    so the same net can be written for the reference's own fp32 oracle (src/perch_ref.c)."""

    def __init__(self, seed=0, n_classes=N_CLASSES, n_blocks=None, kind="int8", head="gemv", ppc=1, eps=1e-5,
                 bias_scale=0.1, pj_gain=0.5, se_open=False, stages=None):
        """bias_scale, pj_gain, se_open (SE gates near 1: the second FC's weights x 0.1, its biases 4) keep the same
        random draws; with small biases, unit-gain projections and open gates the embedding depends strongly on the
        input (the defaults, the benched net, let a deep random stack wash most of the input out). stages: the
        (expand ratio, k, stride, out channels, repeats) list in place of EfficientNet-B3's."""
        assert kind in ("int8", "f32") and head in ("gemv", "proto")
        rng = np.random.default_rng(seed)
        self.n_classes, self.kind, self.head, self.ppc, self.eps = n_classes, kind, head, ppc, eps
        pkg = pkgfmt.Package()
        net = netbuild.Net(pkg)
        self.pkg, self.net = pkg, net
        self.fw, self.blocks_table = [], []
        nw = lambda shape, fan, g=1.0: (rng.standard_normal(shape) * g * np.sqrt(2.0 / fan)).astype(np.float32)
        bias = lambda n: (rng.standard_normal(n) * bias_scale).astype(np.float32)
        pw = net.pw_s8 if kind == "int8" else net.pw

        def keep(name, a):
            self.fw.append((name, a))
            return a
        ib = net.buf(netbuild.F32, 1, NSAMP, 1)
        window = keep("fe.window", (0.5 - 0.5 * np.cos(2 * np.pi * np.arange(FRAME) / FRAME)).astype(np.float32))
        mel = keep("fe.mel", mel_bank())
        self.log_floor, self.log_scale = 1e-3, 1.0
        spec = net.logmel(ib, NSAMP, FRAME, HOP, PAD, NFFT, window, mel, self.log_floor, self.log_scale)
        x = net.stem(spec, keep("stem.w", nw((STEM_C, 9), 9)), keep("stem.b", bias(STEM_C)), 3, 2, act="silu", opad=1,
                     ldo=STEM_C)
        H, W = net.bufs[x][1], net.bufs[x][2]
        bl = blocks(stages) if n_blocks is None else blocks(stages)[:n_blocks]
        for i, (cin, ce, k, s, co) in enumerate(bl):
            res = x if (s == 1 and cin == co) else -1
            h = (k - 1) // 2
            if ce != cin:   # expand 1x1 + SiLU straight into the depthwise conv's zero-haloed input
                d = pw(x, keep(f"m{i}.ex.w", nw((ce, cin), cin)), keep(f"m{i}.ex.b", bias(ce)), act="silu", opad=h)
            elif net.bufs[x][5] == h and net.bufs[x][4] == cin:
                d = x
            else:
                d = net.pad(x, h)
            Ho, Wo, pt, pl = same_pads(H, W, k, s)
            wdw = keep(f"m{i}.dw.w", nw((k * k, ce), k * k))
            bdw = keep(f"m{i}.dw.b", bias(ce))
            if k == 3 and pt == 1 and pl == 1:
                y, cs = net.dw3(d, wdw, bdw, s=s)
            else:
                y, cs = net.dwk(d, wdw, bdw, k, s, pt, pl)
            rd = max(1, cin // 4)
            w1, b1, w2, b2 = nw((rd, ce), ce), bias(rd), nw((ce, rd), rd), bias(ce)
            if se_open:
                w2, b2 = w2 * np.float32(0.1), np.full(ce, 4.0, np.float32)
            g = net.se_gate(cs, Ho * Wo, keep(f"m{i}.se1.w", w1), keep(f"m{i}.se1.b", b1), keep(f"m{i}.se2.w", w2),
                            keep(f"m{i}.se2.b", b2))
            x = pw(y, keep(f"m{i}.pj.w", nw((co, ce), ce, pj_gain)), keep(f"m{i}.pj.b", bias(co)), gate=g, res=res)
            pb, pr = max((Ho - 1) * s + k - H, 0) - pt, max((Wo - 1) * s + k - W, 0) - pl
            self.blocks_table.append((k, s, cin, ce if ce != cin else 0, co, rd, int(res >= 0),
                                      pt | pl << 8 | pb << 16 | pr << 24))
            H, W = Ho, Wo
        c_top = net.bufs[x][3]
        top = pw(x, keep("top.w", nw((EMB, c_top), c_top)), keep("top.b", bias(EMB)), act="silu")
        emb = net.mean(top)
        self.emb_buf = emb
        if head == "gemv":
            wl, bl_ = nw((n_classes, EMB), EMB, 0.5), bias(n_classes)
            if kind == "int8":
                net.gemv_s8(emb, wl, bl_)
            else:
                net.gemv(emb, wl, bl_)
        else:
            protos = keep("proto", nw((n_classes * ppc, EMB), EMB))
            clsw = keep("cls.w", (rng.standard_normal((n_classes, ppc)) * 0.5).astype(np.float32))
            clsb = keep("cls.b", bias(n_classes))
            if kind == "int8":
                net.proto_s8(top, protos, clsw, clsb, eps=eps)
            else:
                net.proto_fp(top, protos, clsw, clsb, eps=eps, kind="f32")
        self.H, self.W = H, W
        net.add_to("neon-int8" if kind == "int8" else "neon-fp32", 0, in_buf=ib, emb_buf=emb)
        netbuild.standard_meta(pkg, NSAMP, n_classes, sample_rate=SR, model_id="perch_v2_shaped_synthetic",
                               emb_dim=EMB)

    def write(self, path):
        self.pkg.write(path)
        return path
