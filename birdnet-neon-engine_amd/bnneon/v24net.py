"""A BirdNET-v2.4-shaped fp16 network as a .bnpk package, with random weights.

The body follows BirdNET v2.4's layer table (results/mac_table.txt in the
reference): four MBConv stages at 24 -> 36 -> 72 -> 108 -> 192 channels with
expansion to 72 / 288 / 864 / 1536 (expand 1x1 + SiLU, depthwise 3x3 + SiLU,
squeeze-excitation, project 1x1, residual when the shape repeats), on the
pixel counts of that table (6,144-ish pixels into the first block, 1,536 / 384
/ 96 / 24 after each stride-2 stage), then a 192 -> 1024 ReLU conv, the global
mean and a 6,522-class linear head whose logits take a sigmoid.

Its front end is the framed log-mel op (3 s at 48 kHz: frame 1024, hop 562,
pad 512, 96 mel bands -> 257 x 96) and a 3 x 3 stride-2 stem to 128 x 47 x 24;
BirdNET v2.4's own front end (a two-channel STFT image and a 4 x 8 stride-2
conv with pooling) and its 3 x 3 valid post conv are v2.4-specific ops that
the generic fp16 ops stand in for here, at the same channel widths.

The ops are the fp16 family's (variant 1, hwcap fp16; src/rt_ops_f16.c):
FE_LOGMEL (fp32), STEM (fp32 math, fp16 output), PW (the fp16 GEMM), DW3
(fp16, TF-same offsets), SE (fp16), MEAN (fp16 rows) and GEMV (fp16 weights).
Weights: per output channel N(0, sqrt(2 / fan_in)) (projections and the
classifier scaled down so that activations stay in range through the residual
stack), biases N(0, 0.1).
"""
import numpy as np

from . import netbuild
from . import perchnet
from . import pkgfmt

SR, NSAMP, FRAME, HOP, PAD, NFFT, NMEL = 48000, 144000, 1024, 562, 512, 1024, 96
N_CLASSES = 6522
EMB = 1024
STEM_C = 24

# (expanded channels, out channels, repeats); the first block of each stage has stride 2
STAGES = [(72, 36, 3), (288, 72, 4), (864, 108, 5), (1536, 192, 4)]


def blocks():
    """(cin, cexp, stride, cout) of the 16 blocks."""
    out, cin = [], STEM_C
    for ce, co, n in STAGES:
        for i in range(n):
            out.append((cin, ce, 2 if i == 0 else 1, co))
            cin = co
    return out


def signal(rng):
    """3 s at 48 kHz: -30 dBFS Gaussian noise plus three random chirps between 1 and 10 kHz."""
    return perchnet.signal(rng, NSAMP, SR)


class V24Net:
    """The package and the float weights it was built from."""

    def __init__(self, seed=0, n_classes=N_CLASSES, n_blocks=None):
        rng = np.random.default_rng(seed)
        self.n_classes = n_classes
        pkg = pkgfmt.Package()
        net = netbuild.Net(pkg)
        self.pkg, self.net = pkg, net
        nw = lambda shape, fan, g=1.0: (rng.standard_normal(shape) * g * np.sqrt(2.0 / fan)).astype(np.float32)
        bias = lambda n: (rng.standard_normal(n) * 0.1).astype(np.float32)
        ib = net.buf(netbuild.F32, 1, NSAMP, 1)
        window = (0.5 - 0.5 * np.cos(2 * np.pi * np.arange(FRAME) / FRAME)).astype(np.float32)
        spec = net.logmel(ib, NSAMP, FRAME, HOP, PAD, NFFT, window, perchnet.mel_bank(NMEL, NFFT, SR, 0.0, 15000.0),
                          1e-3, 1.0)
        x = net.stem_f16(spec, nw((STEM_C, 9), 9), bias(STEM_C), 3, 2, act="silu")
        H, W = net.bufs[x][1], net.bufs[x][2]
        bl = blocks() if n_blocks is None else blocks()[:n_blocks]
        for cin, ce, s, co in bl:
            res = x if (s == 1 and cin == co) else -1
            e = net.pw_f16(x, nw((ce, cin), cin), bias(ce), act="silu", opad=1)
            Ho, Wo, pt, pl = perchnet.same_pads(H, W, 3, s)
            y, cs = net.dw3(e, nw((9, ce), 9), bias(ce), s=s, pt=pt, pl=pl, fp16=True)
            rd = max(1, cin // 4)
            net.se_f16(y, cs, nw((rd, ce), ce), bias(rd), nw((ce, rd), rd), bias(ce))
            x = net.pw_f16(y, nw((co, ce), ce, 0.5), bias(co), res=res)
            H, W = Ho, Wo
        top = net.pw_f16(x, nw((EMB, net.bufs[x][3]), net.bufs[x][3]), bias(EMB), act="relu")
        emb = net.mean_f16(top)
        self.emb_buf = emb
        net.gemv(emb, nw((n_classes, EMB), EMB, 0.5), bias(n_classes), fp16=True)
        self.H, self.W = H, W
        net.add_to("neon-fp16", netbuild.HW_FP16, in_buf=ib, emb_buf=emb)
        netbuild.standard_meta(pkg, NSAMP, n_classes, sample_rate=SR, model_id="birdnet_v24_shaped_synthetic",
                               emb_dim=EMB, post=1)

    def write(self, path):
        self.pkg.write(path)
        return path
