"""Throughput of libbnneon_hip's hot path on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads (one "step" = one pass of the hot path over one batch of synthetic
windows already resident in HBM):

  perch_s8         (default) the Perch-v2-shaped int8 network end to end
                   through bnn_infer_batch_device: 5 s of 32 kHz audio per
                   window -> log-mel 500 x 128 -> stem -> 26 MBConv blocks
                   (int8 1x1 convs, fp32 depthwise, SE) -> 1536 embedding ->
                   14,795-class int8 linear head, batch 256 windows. The line
                   also carries the path's two int8 GEMMs timed on their
                   own, each checked against the oracle: "gemm_s8" (the
                   pointwise conv 1152 -> 256 below) and "gemm_s8_proto"
                   (the prototype head's column-max GEMM below).
  v24_f16          the BirdNET-v2.4-shaped fp16 network end to end through
                   bnn_infer_batch_device: 3 s of 48 kHz audio per window ->
                   log-mel 257 x 96 -> stem -> 16 MBConv blocks (exact fp16
                   1x1 convs, fp16 depthwise, fp16 SE) -> 1024 embedding ->
                   6,522-class fp16-weight linear head, batch 256 windows.
  proto_s8         the int8 prototype head (PROTO_S8) at Perch v2's shape:
                   64 cells x 1536 channels per window against 59,180
                   int8 prototypes (14,795 classes x 4), batch 256 windows.
  gemm_s8_requant  the int8 pointwise convolution 1152 -> 256 over
                   24 x 64 pixels per window, int8 NCHW activations with zero
                   point -128, per-channel Q31 requant, batch 256 windows.
  pw_s8            libbnneon's PW_S8 op (fp32 rows, per-row dynamic int8,
                   fp32 dequant + SiLU) at the same shape, batch 256.
  qpw_s8           the dotprod family's QPW (gated fp16 rows, per-row
                   asymmetric int8, fp32 FMA epilogue, fp16 SiLU out) 64 ->
                   256 over 56 x 117 pixels, batch 64 windows.
  dw_f16, dw_s8    the depthwise convolution, NHWC, C = 672, 24 x 64, k x k
                   (--k 3|5) at stride --s 1|2, 'same' padding, bias + SiLU,
                   batch 64 windows: fp16 (libbnneon's DWK fp16 kernel) or
                   int8 with per-channel Q31 requant and a SiLU table.
  wino_f16         the fp16 Winograd F(2x2,3x3) convolution 64 -> 64 channels
                   over 96 x 256, stride 1, pad 1, fp32 accumulation, bias +
                   SiLU, batch 64 windows.

The timed region is bracketed by device synchronisation; the dominant
kernel's average duration comes from HIP events recorded on the stream the
kernels are launched on. The CPU baseline times the oracle (the scalar C
restatement of the same computation) on the host cores on a bounded sample.
"""
import argparse
import concurrent.futures
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "birdnet-neon-engine_amd"))

METRIC = "windows/s at batch 256 (int8 net); int8 GEMM TOPS as % of MFMA peak"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=None,
                    help="windows per launch (256; 64 for the depthwise workloads)")
    ap.add_argument("--workload", default="perch_s8",
                    choices=["perch_s8", "v24_f16", "gemm_s8_requant", "pw_s8", "proto_s8", "qpw_s8", "dw_f16", "dw_s8",
                             "wino_f16", "copy"])
    ap.add_argument("--k", type=int, default=5, choices=[3, 5], help="depthwise kernel size")
    ap.add_argument("--s", type=int, default=1, choices=[1, 2], help="depthwise stride")
    ap.add_argument("--f16-mfma", action="store_true",
                    help="v24_f16: run the fp16 1x1 convs on fp16 MFMA with fp32 accumulation (BNH_F16_MFMA=1) "
                         "instead of the reference's exact fp16 chains")
    ap.add_argument("--no-legs", action="store_true",
                    help="default workload: skip the timed legs of configs 1-3 (depthwise, Winograd, v2.4 net)")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline leg")
    return ap.parse_args()


def config0_inputs(rng, B, N=256, K=1152, M=1536):
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    x = np.clip(np.round(rng.normal(-40, 35, (B, K, M))), -128, 127).astype(np.int8)
    bias = rng.integers(-2 ** 14, 2 ** 14 + 1, N).astype(np.int32)
    mult = rng.integers(2 ** 30, 2 ** 31, N).astype(np.int32)
    shift = rng.integers(6, 11, N).astype(np.int32)
    return w, x, bias, mult, shift


def time_steps(H, stream, launch, steps, warmup):
    """(ms per step from events on `stream`, wall seconds of the timed region)."""
    for _ in range(warmup):
        launch()
    H.sync(stream)
    ev0, ev1 = H.lib().bnh_event_new(), H.lib().bnh_event_new()
    t0 = time.perf_counter()
    H.check(H.lib().bnh_event_record(ev0, stream))
    for _ in range(steps):
        launch()
    H.check(H.lib().bnh_event_record(ev1, stream))
    H.sync(stream)
    wall = time.perf_counter() - t0
    ms = H.lib().bnh_event_ms(ev0, ev1)
    if ms < 0:
        H.check(None, "bnh_event_ms")
    H.lib().bnh_event_free(ev0)
    H.lib().bnh_event_free(ev1)
    return ms / steps, wall


def cpu_threads():
    """Worker threads of the CPU legs: every host core this process may use, at most 16 (a GPU box grants one
    GPU's job a 16-thread CPU share, whatever os.cpu_count() reports there)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def host_description():
    """The host the CPU legs ran on: core counts, CPU model and the oracle's compiler."""
    import subprocess
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        cc = subprocess.run(["gcc", "--version"], capture_output=True, text=True).stdout.splitlines()[0]
    except (OSError, IndexError):
        cc = "unknown"
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    return {"nproc": os.cpu_count(), "usable_cores": affinity, "threads_used": cpu_threads(), "cpu_model": model,
            "oracle_compiler": cc + " -O2 -ffp-contract=off"}


def cpu_baseline_gemm_s8_requant(w, bias, mult, shift, rng):
    """The oracle's requant GEMM, one window per thread, on a bounded sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O
    T = cpu_threads()
    n_win = 2 * T
    xs = [np.clip(np.round(rng.normal(-40, 35, (w.shape[1], 1536))), -128, 127).astype(np.int8)
          for _ in range(T)]
    t0 = time.perf_counter()
    with concurrent.futures.ThreadPoolExecutor(T) as ex:
        list(ex.map(lambda i: O.gemm_s8_requant(w, xs[i % T], bias, mult, shift, -128, -128),
                    range(n_win)))
    dt = time.perf_counter() - t0
    return {"value": n_win / dt, "unit": "windows/s", "cores": T, "kind": "port",
            "sample": f"{n_win} windows of the 1152->256 x 1536-pixel requant GEMM, "
                      f"one window per thread ({T} threads), scalar C oracle -O2 "
                      f"-ffp-contract=off; {dt:.2f} s wall"}


def cpu_baseline_pw_s8(pk, rng):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O
    T = cpu_threads()
    n_win = 2 * T
    xs = [rng.standard_normal((1536, 1152)).astype(np.float32) for _ in range(T)]
    t0 = time.perf_counter()
    with concurrent.futures.ThreadPoolExecutor(T) as ex:
        list(ex.map(lambda i: O.pw_s8(xs[i % T], pk, act=1), range(n_win)))
    dt = time.perf_counter() - t0
    return {"value": n_win / dt, "unit": "windows/s", "cores": T, "kind": "port",
            "sample": f"{n_win} windows of PW_S8 1152->256 x 1536 pixels (quantize + GEMM + "
                      f"dequant + SiLU), one window per thread ({T} threads), scalar C oracle; "
                      f"{dt:.2f} s wall"}


def gemm_s8_leg(H, rng, B, stream, steps, warmup, check_windows=(0, -1)):
    """The int8 pointwise GEMM of the second half of the metric: 1152 -> 256 channels over 24 x 64 pixels per window,
    int8 NCHW activations with zero point -128, per-channel Q31 requant (k_gemm_s8_requant_sr), B windows per launch,
    timed with events on `stream`; windows check_windows of the batch are compared with the oracle bit for bit."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O
    N, K, M = 256, 1152, 1536
    w, x, bias, mult, shift = config0_inputs(rng, B)
    Wq = H.Q8Weights(w, bias, mult, shift, -128, -128)
    dx = H.DeviceArray.from_host(x)
    dout = H.DeviceArray.zeros((B, N, M), np.int8)

    def launch():
        H.check(H.lib().bnh_gemm_s8_requant(Wq.h, dx.ptr, K * M, M, B, dout.ptr, N * M, stream))
    ms, _ = time_steps(H, stream, launch, steps, warmup)
    got = dout.numpy()
    ok = [bool(np.array_equal(got[i], O.gemm_s8_requant(w, x[i], bias, mult, shift, -128, -128)))
          for i in check_windows]
    nbytes = B * (K * M + N * M) + N * K + 3 * 4 * N
    ops = 2.0 * B * M * N * K
    tops = ops / (ms * 1e-3) / 1e12
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"kernel": "k_gemm_s8_requant_sr",
            "launch": f"int8 1x1 conv {K}->{N} over 24x64 px x {B} windows, NCHW, Q31 requant, int8 out",
            "ms_per_launch": round(ms, 4), "tops": round(tops, 1), "mfma_frac": round(tops / INT8_PEAK_TOPS, 4),
            "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "algorithmic_bytes_per_launch": nbytes, "ops_per_launch": int(ops),
            "parity_windows": f"{sum(ok)}/{len(ok)} bit-exact vs the oracle (windows {list(check_windows)})"}


def proto_s8_leg(H, rng, B, stream, steps, warmup):
    """The int8 prototype head's column-max GEMM (k_proto_gemm_pp) at Perch v2's shape: 64 cells x 1536 channels per
    window against 59,180 prototypes, B windows per launch, timed with events on `stream` after `warmup` launches;
    window 0's logits (cell quantization + GEMM + logits) are compared with the oracle bit for bit."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O
    from bnneon import s8pack
    P, C, nc, ppc = 64, 1536, 14795, 4
    N = nc * ppc
    protos = rng.standard_normal((N, C)).astype(np.float32)
    clsw = rng.uniform(0, 1, N).astype(np.float32)
    clsb = (rng.standard_normal(nc) * 0.1).astype(np.float32)
    Kp, Np = s8pack.r16(C), (N + 3) // 4 * 4
    q, sw = s8pack.quant_rows_s8(protos)
    qp = np.zeros((Np, Kp), np.int8)
    qp[:N, :C] = q
    swp = np.zeros(Np, np.float32)
    swp[:N] = sw
    qw = s8pack.pack_panels(qp)
    L = H.lib()
    W = L.bnh_s8p_new(Np, Kp, qw.ctypes.data, swp.ctypes.data)
    if not W:
        H.check(None, "bnh_s8p_new")
    cells = np.maximum(rng.standard_normal((B, P, C)), 0).astype(np.float32)
    dx = H.DeviceArray.from_host(cells)
    dqa = H.DeviceArray.zeros((B, P * Kp), np.int8)
    dsx = H.DeviceArray.zeros((B, P), np.float32)
    dcm = H.DeviceArray.zeros((B, Np), np.float32)
    dlg = H.DeviceArray.zeros((B, nc), np.float32)
    dcw = H.DeviceArray.from_host(clsw)
    dcb = H.DeviceArray.from_host(clsb)
    H.check(L.bnh_quant_cells(dx.ptr, P * C, P, C, C, 1e-5, dqa.ptr, P * Kp, Kp, dsx.ptr, P, B, stream))

    def colmax():
        H.check(L.bnh_proto_colmax(dqa.ptr, P * Kp, dsx.ptr, P, P, W, dcm.ptr, Np, B, stream))
    ms, _ = time_steps(H, stream, colmax, steps, warmup)
    H.check(L.bnh_proto_logits(dcm.ptr, Np, dcw.ptr, dcb.ptr, nc, ppc, dlg.ptr, nc, B, None, 7, stream))
    got = dlg.numpy()[0]
    ref = O.proto_s8(cells[0], C, 1e-5, qw, swp, Np, Kp, clsw, clsb, nc, ppc)[1]
    L.bnh_s8p_free(W)
    ops = 2.0 * B * P * C * N
    tops = ops / (ms * 1e-3) / 1e12
    return {"kernel": "k_proto_gemm_pp",
            "launch": f"int8 prototype head {B} windows x {P} cells x {C} channels against {N:,} prototypes, column "
                      "maxima per window",
            "ms_per_launch": round(ms, 4), "tops": round(tops, 1), "mfma_frac": round(tops / INT8_PEAK_TOPS, 4),
            "ops_per_launch": int(ops),
            "parity_windows": f"{int(np.array_equal(got.view(np.uint32), ref.view(np.uint32)))}/1 window's logits "
                              "bit-exact vs the oracle (window 0)"}


def same_pads(n, k, s):
    o = (n - 1) // s + 1
    return o, max((o - 1) * s + k - n, 0) // 2


def silu_lut_s8(sx, zx, sy, zy):
    """int8 -> int8 SiLU table for activations with scales / zero points."""
    q = np.arange(-128, 128, dtype=np.float64)
    x = (q - zx) * sx
    y = x / (1 + np.exp(-x))
    return np.clip(np.round(y / sy) + zy, -128, 127).astype(np.int8)


def dw_inputs(rng, B, C, H, W, k, s, kind):
    h = (k - 1) // 2
    Ho, pt = same_pads(H, k, s)
    Wo, pl = same_pads(W, k, s)
    if kind == "f16":
        x = rng.standard_normal((B, H, W, C)).astype(np.float32)
        x = x / (1 + np.exp(-x))                     # activations SiLU(N(0, 1))
        xp = np.zeros((B, H + 2 * h, W + 2 * h, C), np.float16)
        xp[:, h:h + H, h:h + W] = x
        w = (rng.standard_normal((k * k, C)) * np.sqrt(2.0 / (k * k))).astype(np.float16)
        b = (rng.standard_normal(C) * 0.1).astype(np.float16)
        return dict(x=xp, w=w, b=b, Ho=Ho, Wo=Wo, pt=pt, pl=pl)
    x = np.clip(np.round(rng.normal(-40, 35, (B, H, W, C))), -128, 127).astype(np.int8)
    w = rng.integers(-127, 128, (k * k, C)).astype(np.int8)
    bias = rng.integers(-2 ** 14, 2 ** 14 + 1, C).astype(np.int32)
    mult = rng.integers(2 ** 30, 2 ** 31, C).astype(np.int32)
    shift = rng.integers(6, 11, C).astype(np.int32)
    lut = silu_lut_s8(0.05, -128, 0.05, -128)
    return dict(x=x, w=w, bias=bias, mult=mult, shift=shift, lut=lut, Ho=Ho, Wo=Wo, pt=pt, pl=pl)


def cpu_baseline_dw(d, kind, C, H, W, k, s):
    """The oracle's depthwise kernel, one window per thread, on a bounded sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O
    T = cpu_threads()
    n_win = 2 * T
    x = d["x"]
    if kind == "f16":
        f = lambda i: O.dwk_f16(x[i % x.shape[0]], H, W, C, k, s, d["pt"], d["pl"], d["w"], d["b"], 1,
                                d["Ho"], d["Wo"])
        what = "fp16 DWK (exact fp16 arithmetic emulated in integer C)"
    else:
        f = lambda i: O.dw_s8(x[i % x.shape[0]], k, s, d["pt"], d["pl"], d["w"], d["bias"], d["mult"],
                              d["shift"], -128, -128, -128, 127, d["lut"], d["Ho"], d["Wo"])
        what = "int8 depthwise + Q31 requant + SiLU table"
    t0 = time.perf_counter()
    f(0)
    n_win = T * max(2, min(200, int(5.0 / max(time.perf_counter() - t0, 1e-3))))  # about 5 s per thread
    t0 = time.perf_counter()
    with concurrent.futures.ThreadPoolExecutor(T) as ex:
        list(ex.map(f, range(n_win)))
    dt = time.perf_counter() - t0
    return {"value": n_win / dt, "unit": "windows/s", "cores": T, "kind": "port",
            "sample": f"{n_win} windows of the {k}x{k} s{s} {what}, C={C}, {H}x{W}, one window per "
                      f"thread ({T} threads), scalar C oracle; {dt:.2f} s wall"}


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: every box here has one "
                          "MI355X and the hot path needs no collective (windows are "
                          "independent); run with --gpus 1"}))
        sys.exit(2)
    from bnneon import hip as H
    if H.lib().bnh_device_count() < 1:
        raise SystemExit("no HIP device visible")
    rng = np.random.default_rng(20240601)
    B = a.batch or (64 if a.workload.startswith(("dw_", "wino", "qpw")) else 256)
    N, K, M = 256, 1152, 1536
    stream = H.lib().bnh_stream_new()
    if a.workload == "copy":
        # calibration: a plain 1 GiB device-to-device copy (the achievable HBM
        # rate, and the reference for the FETCH_SIZE / WRITE_SIZE counters)
        nbytes = 1 << 30
        src = H.DeviceArray.zeros(nbytes, np.uint8)
        dst = H.DeviceArray.zeros(nbytes, np.uint8)
        ms, wall = time_steps(H, stream, lambda: H.check(H.lib().bnh_copy(dst.ptr, src.ptr, nbytes, stream)),
                              a.steps, a.warmup)
        print(json.dumps({"workload": "copy", "bytes_read": nbytes, "bytes_written": nbytes,
                          "ms_per_copy": round(ms, 4), "GBps": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}),
              flush=True)
        return
    if a.workload.startswith("dw_"):
        run_dw(a, H, rng, B, stream)
        return
    if a.workload == "wino_f16":
        run_wino(a, H, rng, B, stream)
        return
    if a.workload == "perch_s8":
        run_perch(a, H, rng, B, stream)
        return
    if a.workload == "v24_f16":
        run_v24(a, H, rng, B, stream)
        return
    if a.workload == "proto_s8":
        run_proto(a, H, rng, B, stream)
        return
    if a.workload == "qpw_s8":
        run_qpw(a, H, rng, B, stream)
        return
    if a.workload == "gemm_s8_requant":
        w, x, bias, mult, shift = config0_inputs(rng, B)
        Wq = H.Q8Weights(w, bias, mult, shift, -128, -128)
        dx = H.DeviceArray.from_host(x)
        dout = H.DeviceArray.zeros((B, N, M), np.int8)
        del x

        def launch():
            H.check(H.lib().bnh_gemm_s8_requant(Wq.h, dx.ptr, K * M, M, B, dout.ptr, N * M, stream))
        bytes_per_launch = B * (K * M + N * M) + N * K + 3 * 4 * N
        workload = ("int8 pointwise conv 1152->256 over 24x64 pixels per window, NCHW int8 "
                    "activations (zero point -128), per-channel Q31 requant, int8 out")
        kernel = "k_gemm_s8_requant_sr"
        dtype = "int8"
    else:
        sys.path.insert(0, os.path.join(ROOT, "birdnet-neon-engine_amd"))
        from bnneon import s8pack
        wf = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
        pk = s8pack.pack_s8(wf, rng.standard_normal(N).astype(np.float32))
        _, _, Kp, Np = pk["shape"]
        Wt = H.S8Weights(N, K, Kp, Np, pk["q"], pk["sw"], pk["cs"], pk["b"])
        dx = H.DeviceArray.from_host(rng.standard_normal((B, M, K)).astype(np.float32))
        dq = H.DeviceArray.zeros((B, M * Kp), np.int8)
        dsa = H.DeviceArray.zeros((B, M), np.float32)
        dza = H.DeviceArray.zeros((B, M), np.int32)
        dout = H.DeviceArray.zeros((B, M, Np), np.float32)
        e = H.epi32(dout, Np, act=1, out_ws=M * Np)

        def launch():
            H.check(H.lib().bnh_pw_s8(dx.ptr, M * K, K, M, None, 0, dq.ptr, M * Kp, dsa.ptr, M, dza.ptr,
                                      M, B, Wt.h, e, stream))
        # quantize (read fp32 rows, write q) + GEMM (read q, write fp32 out)
        bytes_per_launch = B * M * (4 * K + 2 * Kp + 4 * Np) + Np * Kp
        workload = ("libbnneon PW_S8 1152->256 over 24x64 pixels per window: fp32 NHWC rows, "
                    "per-row dynamic int8, fp32 dequant + SiLU epilogue")
        kernel = "k_s8n_gemm + k_s8n_quant"
        dtype = "int8"
    ms, wall = time_steps(H, stream, launch, a.steps, a.warmup)
    ops_per_launch = 2.0 * B * M * N * K
    value = B / (ms * 1e-3)
    tops = ops_per_launch / (ms * 1e-3) / 1e12
    gbs = bytes_per_launch / (ms * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "windows/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dtype, "data": "synthetic (seeded; config distributions)",
        "config": {"workload": workload, "global_batch": B, "pixels_per_window": M,
                   "cin": K, "cout": N, "parallelism": "1 GPU, windows batched per launch",
                   "wall_s_timed_region": round(wall, 4)},
        "int8_tops": round(tops, 2), "mfma_frac": round(tops / INT8_PEAK_TOPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": kernel, "algorithmic_bytes_per_launch": bytes_per_launch},
    }
    if not a.no_cpu:
        if a.workload == "gemm_s8_requant":
            line["cpu_baseline"] = cpu_baseline_gemm_s8_requant(w, bias, mult, shift, rng)
        else:
            line["cpu_baseline"] = cpu_baseline_pw_s8(pk, rng)
    print(json.dumps(line), flush=True)


def run_dw(a, H, rng, B, stream, emit=True):
    C, Hh, W, k, s = 672, 24, 64, a.k, a.s
    kind = a.workload[3:]
    d = dw_inputs(rng, B, C, Hh, W, k, s, kind)
    Ho, Wo, pt, pl = d["Ho"], d["Wo"], d["pt"], d["pl"]
    L = H.lib()
    dx = H.DeviceArray.from_host(d["x"])
    x_ws = d["x"][0].size
    o_ws = Ho * Wo * C
    dw_ = H.DeviceArray.from_host(d["w"])
    if kind == "f16":
        db = H.DeviceArray.from_host(d["b"])
        dout = H.DeviceArray.zeros((B, o_ws), np.float16)

        def launch():
            H.check(L.bnh_dwk_f16(dx.ptr, x_ws, Hh, W, C, k, s, pt, pl, dw_.ptr, db.ptr, 1, dout.ptr, o_ws,
                                  Ho, Wo, None, 0, B, stream))
        esz = 2
        workload = (f"fp16 depthwise {k}x{k} stride {s}, 'same', NHWC C=672 24x64, bias + SiLU (LUT), "
                    f"libbnneon DWK fp16 arithmetic")
        kernel = "k_dw_f16"
        dtype = "fp16"
    else:
        dbias, dm = H.DeviceArray.from_host(d["bias"]), H.DeviceArray.from_host(d["mult"])
        dsh, dl = H.DeviceArray.from_host(d["shift"]), H.DeviceArray.from_host(d["lut"])
        dout = H.DeviceArray.zeros((B, o_ws), np.int8)

        def launch():
            H.check(L.bnh_dw_s8(dx.ptr, x_ws, Hh, W, C, k, s, pt, pl, dw_.ptr, dbias.ptr, dm.ptr, dsh.ptr,
                                -128, -128, -128, 127, dl.ptr, dout.ptr, o_ws, Ho, Wo, B, stream))
        esz = 1
        workload = (f"int8 depthwise {k}x{k} stride {s}, 'same', NHWC C=672 24x64, per-channel Q31 requant "
                    f"+ SiLU table")
        kernel = "k_dw_s8"
        dtype = "int8"
    ms, wall = time_steps(H, stream, launch, a.steps, a.warmup)
    bytes_per_launch = B * (x_ws + o_ws) * esz + k * k * C * esz
    gbs = bytes_per_launch / (ms * 1e-3) / 1e9
    line = {
        "metric": "windows/s (depthwise layer, batch 64)", "value": round(B / (ms * 1e-3), 1),
        "unit": "windows/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": dtype, "data": "synthetic (seeded; config distributions)",
        "config": {"workload": workload, "global_batch": B, "channels": C, "height": Hh, "width": W,
                   "k": k, "stride": s, "parallelism": "1 GPU, windows batched per launch",
                   "wall_s_timed_region": round(wall, 4)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": kernel,
                     "algorithmic_bytes_per_launch": bytes_per_launch},
    }
    line["parity_windows"] = dw_parity(dout.numpy(), d, kind, C, Hh, W, k, s, (0, B - 1))
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline_dw(d, kind, C, Hh, W, k, s)
    if not emit:
        return line
    print(json.dumps(line), flush=True)


def dw_parity(got, d, kind, C, H, W, k, s, wins):
    """The batch's outputs of windows `wins` against the oracle's depthwise kernel, bit for bit."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O
    ok = []
    for i in wins:
        if kind == "f16":
            ref = O.dwk_f16(d["x"][i], H, W, C, k, s, d["pt"], d["pl"], d["w"], d["b"], 1, d["Ho"], d["Wo"])[0]
            ok.append(bool(np.array_equal(got[i].view(np.uint16), ref.reshape(-1).view(np.uint16))))
        else:
            ref = O.dw_s8(d["x"][i], k, s, d["pt"], d["pl"], d["w"], d["bias"], d["mult"], d["shift"], -128, -128,
                          -128, 127, d["lut"], d["Ho"], d["Wo"])
            ok.append(bool(np.array_equal(got[i], ref.reshape(-1))))
    return f"{sum(ok)}/{len(ok)} bit-exact vs the oracle (windows {list(wins)})"


def cpu_baseline_wino(xp, w, b):
    """float64 direct convolution (numpy), the comparison oracle, on a bounded sample of windows."""
    T = 1
    t0 = time.perf_counter()
    n = 0
    while n == 0 or time.perf_counter() - t0 < 5.0:
        x = xp[n % xp.shape[0]].astype(np.float64)
        H, W = x.shape[0] - 2, x.shape[1] - 2
        cols = np.stack([x[ky:ky + H, kx:kx + W] for ky in range(3) for kx in range(3)], axis=2)
        y = cols.reshape(H * W, -1) @ w.reshape(w.shape[0], -1).T.astype(np.float64) + b
        y = y / (1 + np.exp(-y))
        n += 1
    dt = time.perf_counter() - t0
    return {"value": n / dt, "unit": "windows/s", "cores": T, "kind": "port",
            "sample": f"{n} windows of the 64->64 3x3 conv over 96x256 as a float64 im2col GEMM + SiLU "
                      f"(numpy, BLAS threads as configured), {dt:.2f} s wall"}


def run_wino(a, H, rng, B, stream, emit=True):
    Hh, W, C, K = 96, 256, 64, 64
    xp = np.zeros((B, Hh + 2, W + 2, C), np.float16)
    xp[:, 1:-1, 1:-1] = rng.standard_normal((B, Hh, W, C))
    w = (rng.standard_normal((K, 3, 3, C)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    b = (rng.standard_normal(K) * 0.1).astype(np.float32)
    L = H.lib()
    P = L.bnh_wino16_new(C, K, w.ctypes.data, b.ctypes.data)
    if not P:
        H.check(None, "bnh_wino16_new")
    x_ws = (Hh + 2) * (W + 2) * C
    o_ws = Hh * W * K
    dx = H.DeviceArray.from_host(xp)
    dout = H.DeviceArray.zeros((B, o_ws), np.float16)

    def launch():
        H.check(L.bnh_wino_f16(dx.ptr, x_ws, Hh, W, C, P, 1, dout.ptr, o_ws, K, 0, None, 0, 0, 0, B, stream))
    ms, wall = time_steps(H, stream, launch, a.steps, a.warmup)
    bytes_per_launch = B * (x_ws + o_ws) * 2 + 16 * K * C * 2
    gbs = bytes_per_launch / (ms * 1e-3) / 1e9
    flops_direct = 2.0 * B * Hh * W * K * C * 9
    line = {
        "metric": "windows/s (fp16 Winograd conv, batch 64)", "value": round(B / (ms * 1e-3), 1),
        "unit": "windows/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic (seeded; config distributions)",
        "config": {"workload": "fp16 Winograd F(2x2,3x3) conv 64->64 over 96x256, stride 1, pad 1, fp32 "
                               "accumulation on fp16 MFMA, bias + SiLU, NHWC",
                   "global_batch": B, "channels_in": C, "channels_out": K, "height": Hh, "width": W,
                   "parallelism": "1 GPU, windows batched per launch", "wall_s_timed_region": round(wall, 4)},
        "direct_equivalent_tflops": round(flops_direct / (ms * 1e-3) / 1e12, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "k_wino_f16r",
                     "algorithmic_bytes_per_launch": bytes_per_launch},
    }
    got = dout.numpy().reshape(B, Hh, W, K).astype(np.float64)
    u = 2.0 ** -11
    worst = 0.0
    for i in (0, B - 1):
        x64 = xp[i].astype(np.float64)
        cols = np.stack([x64[ky:ky + Hh, kx:kx + W] for ky in range(3) for kx in range(3)], axis=2)
        y = (cols.reshape(Hh * W, -1) @ w.reshape(K, -1).T.astype(np.float64) + b).reshape(Hh, W, K)
        y = y / (1 + np.exp(-y))
        worst = max(worst, float(np.abs(got[i] - y).max() / (8 * u * np.abs(y).max())))
    line["parity_windows"] = (f"windows [0, {B - 1}] against a float64 direct conv + SiLU: max |error| = "
                              f"{worst:.3f} x the stated whole-output bound 8 u max|y| (u = 2^-11)"
                              + (" (within)" if worst <= 1.0 else " (EXCEEDED)"))
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline_wino(xp, w, b)
    L.bnh_wino16_free(P)
    if not emit:
        return line
    print(json.dumps(line), flush=True)



def run_qpw(a, H, rng, B, stream):
    """The dotprod family's QPW (src/rt_ops_dot.c:326-339) at a BirdNET-v3.0-like MBConv expansion: per window
    fp16 rows of 56 x 117 pixels x 64 channels, gated by an SE's fp16 gates, quantised per row to int8 (k_qd_quant),
    the int8 MFMA GEMM to 256 channels with the fp32 FMA epilogue, fp16 + table SiLU into a zero-haloed buffer
    (k_qd_gemm). Timed: both kernels per step; the GEMM also alone, for the roofline."""
    import ctypes
    Hh, W, K, N = 56, 117, 64, 256
    M, Kp = Hh * W, 64
    L = H.lib()
    w = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    Wq = L.bnh_qdw_new(w.ctypes.data, bias.ctypes.data, N, K, N)
    if not Wq:
        H.check(None, "bnh_qdw_new")
    x = (rng.standard_normal((B, M * K)) * 2).astype(np.float16)
    g = rng.uniform(0, 1, (B, K)).astype(np.float16)
    dx, dg = H.DeviceArray.from_host(x), H.DeviceArray.from_host(g)
    a_ws, rq_ws = (M + 4) * Kp, 2 * (M + 4)
    rows_out = (Hh + 2) * (W + 2)
    o_ws = rows_out * N
    da = H.DeviceArray.zeros((B, a_ws), np.int8)
    dr = H.DeviceArray.zeros((B, rq_ws), np.float32)
    do = H.DeviceArray.zeros((B, o_ws), np.float16)
    e = H.QdEpi(1, 1, do.ptr, o_ws, N, W, 1, None, 0)

    def quant():
        H.check(L.bnh_qd_quant_rows(dx.ptr, 1, M * K, K, M, K, dg.ptr, K, da.ptr, a_ws, dr.ptr, rq_ws, B, stream))

    def gemm():
        H.check(L.bnh_qd_gemm(da.ptr, a_ws, Kp, dr.ptr, rq_ws, 0, M, Wq, ctypes.byref(e), B, stream))

    def launch():
        quant()
        gemm()
    ms, wall = time_steps(H, stream, launch, a.steps, a.warmup)
    ms_g, _ = time_steps(H, stream, gemm, max(10, a.steps), 3)
    op_bytes = B * (M * K * 2 + K * 2 + M * N * 2) + N * Kp + 12 * N   # the op's own inputs and outputs
    gemm_bytes = B * (M * Kp + 8 * M + rows_out * N * 2) + N * Kp + 12 * N
    gbs = gemm_bytes / (ms_g * 1e-3) / 1e9
    line = {
        "metric": "windows/s (dotprod QPW, batch 64)", "value": round(B / (ms * 1e-3), 1), "unit": "windows/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded normal rows, uniform gates, random weights)",
        "config": {"workload": "dotprod QPW 64->256 over 56x117 px per window: gated fp16 rows, per-row asymmetric "
                               "int8, int8 MFMA GEMM, fp32 FMA epilogue, fp16 table SiLU into a zero-haloed buffer",
                   "global_batch": B, "channels_in": K, "channels_out": N, "pixels": M,
                   "parallelism": "1 GPU, windows batched per launch", "wall_s_timed_region": round(wall, 4),
                   "op_bytes_per_step": op_bytes},
        "int8_tops": round(2.0 * B * M * N * K / (ms_g * 1e-3) / 1e12, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "k_qd_gemm",
                     "ms_per_launch": round(ms_g, 4), "algorithmic_bytes_per_launch": gemm_bytes},
    }
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline_qpw(x, g, w, bias, Hh, W)
    L.bnh_qdw_free(Wq)
    print(json.dumps(line), flush=True)


def cpu_baseline_qpw(x, g, w, bias, Hh, W):
    """The oracle's QPW (quantisation + int8 GEMM + epilogue, scalar C) on a bounded sample of windows."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O
    K = w.shape[1]
    pk = O.qd_wpack(w, bias)
    t0 = time.perf_counter()
    n = 0
    while n == 0 or time.perf_counter() - t0 < 5.0:
        O.qpw(x[n % x.shape[0]].reshape(Hh * W, K), pk, act=1, out16=True, ow=W, opad=1, gate=g[n % g.shape[0]])
        n += 1
    dt = time.perf_counter() - t0
    return {"value": n / dt, "unit": "windows/s", "cores": 1, "kind": "port",
            "sample": f"{n} windows of the oracle's QPW (scalar C, 1 thread), {dt:.2f} s wall"}


def run_proto(a, H, rng, B, stream):
    """The int8 prototype head (PROTO_S8) at Perch v2's shape: per window 64 cells of 1536 channels (fp32, as the
    body leaves them) against 14,795 classes x 4 prototypes. Timed: cell quantization + column-max GEMM + logits per
    step; the column-max GEMM (k_proto_gemm_pp, the MFMA-bound kernel) also alone, for the roofline."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O
    from bnneon import s8pack
    P, C, nc, ppc = 64, 1536, 14795, 4
    N = nc * ppc
    protos = rng.standard_normal((N, C)).astype(np.float32)
    clsw = rng.uniform(0, 1, N).astype(np.float32)
    clsb = (rng.standard_normal(nc) * 0.1).astype(np.float32)
    Kp, Np = s8pack.r16(C), (N + 3) // 4 * 4
    q, sw = s8pack.quant_rows_s8(protos)
    qp = np.zeros((Np, Kp), np.int8)
    qp[:N, :C] = q
    swp = np.zeros(Np, np.float32)
    swp[:N] = sw
    qw = s8pack.pack_panels(qp)
    L = H.lib()
    W = L.bnh_s8p_new(Np, Kp, qw.ctypes.data, swp.ctypes.data)
    if not W:
        H.check(None, "bnh_s8p_new")
    n_distinct = min(B, 2 * cpu_threads())
    cells = [np.maximum(rng.standard_normal((P, C)), 0).astype(np.float32) for _ in range(n_distinct)]
    dx = H.DeviceArray.from_host(np.stack([cells[i % n_distinct] for i in range(B)]))
    dqa = H.DeviceArray.zeros((B, P * Kp), np.int8)
    dsx = H.DeviceArray.zeros((B, P), np.float32)
    dcm = H.DeviceArray.zeros((B, Np), np.float32)
    dlg = H.DeviceArray.zeros((B, nc), np.float32)
    dcw = H.DeviceArray.from_host(clsw)
    dcb = H.DeviceArray.from_host(clsb)

    def quant():
        H.check(L.bnh_quant_cells(dx.ptr, P * C, P, C, C, 1e-5, dqa.ptr, P * Kp, Kp, dsx.ptr, P, B, stream))

    def colmax():
        H.check(L.bnh_proto_colmax(dqa.ptr, P * Kp, dsx.ptr, P, P, W, dcm.ptr, Np, B, stream))

    def head():
        quant()
        colmax()
        H.check(L.bnh_proto_logits(dcm.ptr, Np, dcw.ptr, dcb.ptr, nc, ppc, dlg.ptr, nc, B, None, 7, stream))
    ms, wall = time_steps(H, stream, head, a.steps, a.warmup)
    logits = dlg.numpy()
    ms_gemm, _ = time_steps(H, stream, colmax, max(10, a.steps), 3)
    ops = 2.0 * B * P * C * N
    tops = ops / (ms_gemm * 1e-3) / 1e12
    line = {
        "metric": "windows/s (int8 prototype head, batch 256)", "value": round(B / (ms * 1e-3), 1),
        "unit": "windows/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: ReLU(N(0,1)) cells, N(0,1) prototypes quantized per row",
        "config": {"workload": "PROTO_S8 at Perch v2's head: 64 cells x 1536 channels per window, 14,795 classes x "
                               "4 prototypes (59,180 x 1536 int8), cell quantization + column maxima + logits",
                   "global_batch": B, "parallelism": "1 GPU, windows batched per launch",
                   "wall_s_timed_region": round(wall, 4)},
        "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                     "frac": round(tops / INT8_PEAK_TOPS, 4), "traffic": None, "kernel": "k_proto_gemm_pp",
                     "ms_per_launch": round(ms_gemm, 4), "ops_per_launch": int(ops),
                     "algorithmic_bytes_per_launch": B * P * (Kp + 4) + Np * (Kp + 4) + B * Np * 4},
    }
    if not a.no_cpu:
        T = cpu_threads()
        t0 = time.perf_counter()
        with concurrent.futures.ThreadPoolExecutor(T) as ex:
            ref = list(ex.map(lambda c: O.proto_s8(c, C, 1e-5, qw, swp, Np, Kp, clsw, clsb, nc, ppc)[1], cells))
        dt = time.perf_counter() - t0
        line["cpu_baseline"] = {"value": round(n_distinct / dt, 3), "unit": "windows/s", "cores": T, "kind": "port",
                                "sample": f"{n_distinct} windows of the head through the scalar C oracle, one window "
                                          f"per thread ({T} threads); {dt:.2f} s wall", "host": host_description()}
        same = [bool(np.array_equal(logits[w].view(np.uint32), ref[w % n_distinct].view(np.uint32))) for w in range(B)]
        line["parity_windows"] = f"{sum(same)}/{B} windows' logits bit-identical to the oracle's"
    L.bnh_s8p_free(W)
    print(json.dumps(line), flush=True)


def perch_counts(net):
    """(int8 GEMM ops per window, the PW_S8 op record with the most output) of a netbuild net."""
    ops, big = 0, None
    for code, b, t, p in net.ops:
        if code & 0xff == 22:   # PW_S8: N K Kp Np M ...
            ops += 2 * p[0] * p[1] * p[4]
            if big is None or p[0] * p[4] > big[3][0] * big[3][4]:
                big = (code, b, t, p)
        elif code & 0xff == 23:  # GEMV_S8
            ops += 2 * p[0] * p[1]
    return ops, big


def cpu_baseline_perch(pn, pcms, n_one=6):
    """The oracle's op-by-op run of the same package on the host cores: len(pcms) windows one per thread on
    cpu_threads() threads (about 10 s), then n_one of them on one thread. Returns (baseline dict, the oracle's
    logits of every window in pcms)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_net
    T = cpu_threads()
    on = oracle_net.OracleNet(pn.net, 0, pn.net.last, pn.emb_buf)
    t0 = time.perf_counter()
    with concurrent.futures.ThreadPoolExecutor(T) as ex:
        outs = list(ex.map(lambda p: on.run(p)[0].copy(), pcms))
    dt = time.perf_counter() - t0
    t1 = time.perf_counter()
    for p in pcms[:n_one]:
        on.run(p)
    dt1 = time.perf_counter() - t1
    base = {"value": round(len(pcms) / dt, 3), "unit": "windows/s", "cores": T, "kind": "port",
            "sample": f"{len(pcms)} windows of the same package through the scalar C oracle's op-by-op restatement "
                      f"(log-mel, stem, 26 blocks, head), one window per thread ({T} threads); {dt:.2f} s wall",
            "one_thread": {"value": round(n_one / dt1, 3), "unit": "windows/s", "cores": 1,
                           "sample": f"{n_one} of those windows on one thread; {dt1:.2f} s wall"},
            "host": host_description()}
    return base, outs


def cpu_baseline_reference(pn, pcms, n_one=2):
    """The reference's own scalar fp32 Perch v2 oracle (src/perch_ref.c, built from the reference checkout into
    oracle/_ref) on the bench net's float weights, written as a .bnp2 file: len(pcms) windows one per thread on
    cpu_threads() threads, then n_one on one thread. Returns (baseline dict, its embeddings of pcms), or None where
    the library was not built."""
    sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "oracle", "ref")]
    import perchref
    if not perchref.available():
        return None
    import tempfile
    T = cpu_threads()
    tmp = tempfile.mkdtemp(prefix="bnn_ref_")
    path = os.path.join(tmp, "bench_net.bnp2")
    perchref.write_bnp2(path, pn)
    m = perchref.Model(path)
    try:
        t0 = time.perf_counter()
        with concurrent.futures.ThreadPoolExecutor(T) as ex:
            embs = list(ex.map(lambda p: m.infer(p)[1], pcms))
        dt = time.perf_counter() - t0
        t1 = time.perf_counter()
        for p in pcms[:n_one]:
            m.infer(p)
        dt1 = time.perf_counter() - t1
    finally:
        m.close()
        os.unlink(path)
        os.rmdir(tmp)
    base = {"value": round(len(pcms) / dt, 3), "unit": "windows/s", "cores": T, "kind": "reference",
            "sample": f"{len(pcms)} windows through the reference's own scalar fp32 Perch v2 oracle (src/perch_ref.c "
                      f"pc_ref_infer, clang -O2 -ffp-contract=off) on the bench net's float weights: exact FFT "
                      f"front end, stem, 26 blocks, head conv and embedding, a one-prototype head in place of the "
                      f"linear one (1.8 % of the net's MACs); one window per thread ({T} threads), {dt:.2f} s wall",
            "one_thread": {"value": round(n_one / dt1, 3), "unit": "windows/s", "cores": 1,
                           "sample": f"{n_one} of those windows on one thread; {dt1:.2f} s wall"}}
    return base, embs


def run_perch(a, H, rng, B, stream):
    import tempfile
    from bnneon import binding, perchnet
    pn = perchnet.PerchNet(seed=7)
    tmp = tempfile.mkdtemp(prefix="bnn_bench_")
    path = pn.write(os.path.join(tmp, "perch_v2_shaped_s8.bnpk"))
    L = binding.load_library()
    m = binding.Model(path)
    nc, ne, ns = m.info.n_classes, m.info.emb_dim, m.info.n_samples
    # the batch: n_distinct synthetic windows, repeated; the CPU leg scores the same windows on the oracle and the
    # GPU's logits of every window of the batch (both sub-batches) are compared with them bit for bit
    n_distinct = min(B, 8 * cpu_threads())
    pcms = [perchnet.signal(rng) for _ in range(n_distinct)]
    pcm = np.stack([pcms[i % n_distinct] for i in range(B)])
    dx = H.DeviceArray.from_host(pcm)
    dout = H.DeviceArray.zeros((B, nc), np.float32)
    demb = H.DeviceArray.zeros((B, ne), np.float32)
    status = np.zeros(B, np.int32)
    sp = status.ctypes.data_as(binding._IP)

    def launch():
        r = L.bnn_infer_batch_device(m.ctx, dx.ptr, B, dout.ptr, demb.ptr, sp, stream)
        if r != 0:
            raise RuntimeError(f"bnn_infer_batch_device returned {r}: {L.bnn_last_error()}")
    ms, wall = time_steps(H, stream, launch, a.steps, a.warmup)
    logits = dout.numpy()
    ops_win, _ = perch_counts(pn.net)
    value = B / (ms * 1e-3)
    tops = ops_win * B / (ms * 1e-3) / 1e12
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "windows/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: -30 dBFS noise + 3 chirps 1-10 kHz per window; random weights",
        "config": {"workload": "Perch-v2-shaped int8 net (log-mel 500x128, stem 3x3/2 -> 40, 26 MBConv blocks "
                               "with SE, 1x1 convs on PW_S8, fp32 depthwise, 384->1536 head conv, mean, "
                               "14,795-class GEMV_S8), 160,000 samples @ 32 kHz per window",
                   "global_batch": B, "n_samples": ns, "n_classes": nc,
                   "parallelism": "1 GPU, windows batched per launch",
                   "wall_s_timed_region": round(wall, 4)},
        "int8_tops": round(tops, 3), "mfma_frac": round(tops / INT8_PEAK_TOPS, 5),
        "int8_tops_scope": "the whole net: its int8 GEMM operations per step over the step's time (most of a step is "
                           "depthwise, SE and quantisation work); the int8 GEMMs timed on their own are under "
                           "gemm_s8 and gemm_s8_proto",
    }
    line["roofline"] = perch_roofline(H, pn, B, stream, a)
    m.close()
    line["host_buffers"] = host_buffers_leg(L, path, pcm, a)
    os.unlink(path)
    os.rmdir(tmp)
    # the GEMM takes ~0.15 ms: 200 untimed launches (~30 ms) bring the clocks back up after the host-side input
    # generation, and 300 timed ones average over ~45 ms
    line["gemm_s8"] = gemm_s8_leg(H, rng, B, stream, max(300, a.steps), 200)
    # the other int8 GEMM of the path, the prototype head (~1.1 ms a launch): 60 warmup launches, 100 timed
    line["gemm_s8_proto"] = proto_s8_leg(H, rng, B, stream, max(100, a.steps), 60)
    if not a.no_legs:
        line.update(config_legs(a, H, rng, stream))
    if not a.no_cpu:
        port, ref = cpu_baseline_perch(pn, pcms)
        same = [bool(np.array_equal(logits[w].view(np.uint32), ref[w % n_distinct][:nc].view(np.uint32)))
                for w in range(B)]
        line["parity_windows"] = f"{sum(same)}/{B} windows' logits bit-identical to the oracle's"
        rb = cpu_baseline_reference(pn, pcms[:2 * cpu_threads()])
        if rb is None:
            line["cpu_baseline"] = port
        else:
            base, embs = rb
            host = port.pop("host")
            line["cpu_baseline"] = dict(base, port=port, host=host)
            gemb = demb.numpy()
            rel = [float(np.linalg.norm(gemb[w] - e) / np.linalg.norm(e)) for w, e in enumerate(embs)]
            line["vs_reference_fp32"] = {
                "windows": len(embs), "emb_rel_l2_max": round(max(rel), 5),
                "note": "the GPU's int8 embeddings against the reference's fp32 oracle on the same float weights: the "
                        "int8 quantisation of every 1x1 conv (tests/test_ref_perch.py states the bounds)"}
    print(json.dumps(line), flush=True)


def host_buffers_leg(L, path, pcm, a):
    """The Perch-shaped batch scored from host buffers through bnn_infer_batch (a fresh context): the PCIe copies of
    the windows in and of the logits and embeddings out are inside the timed region. Reported beside the
    device-resident rate, never as the value."""
    from bnneon import binding
    m = binding.Model(path)
    B = pcm.shape[0]
    out = np.empty((B, m.info.n_classes), np.float32)
    emb = np.empty((B, m.info.emb_dim), np.float32)
    status = np.zeros(B, np.int32)
    pin = np.ascontiguousarray(pcm, np.float32)

    def once():
        r = m.L.bnn_infer_batch(m.ctx, binding._fp(pin), B, binding._fp(out), binding._fp(emb),
                                status.ctypes.data_as(binding._IP))
        if r != 0:
            raise RuntimeError(f"bnn_infer_batch returned {r}")
    for _ in range(5):   # the context settles its stream split on its first five batches
        once()
    n = max(5, a.steps // 2)
    times = []
    for _ in range(n):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    dt = sum(times) / n
    m.close()
    return {"value": round(B / dt, 1), "unit": "windows/s", "ms_per_batch": round(dt * 1e3, 3), "batches": n,
            "ms_per_batch_min_max": [round(min(times) * 1e3, 3), round(max(times) * 1e3, 3)],
            "note": "bnn_infer_batch from pageable host buffers (copies in and out included, host clock around "
                    "each call); the line's value is the device-resident rate"}


def compact_leg(line):
    """The fields of a workload line that the default line carries for it."""
    keep = ("value", "unit", "ms_per_step", "dtype", "parity_windows", "fp16_tflops", "direct_equivalent_tflops")
    out = {k: line[k] for k in keep if k in line}
    out["workload"] = line["config"]["workload"]
    out["global_batch"] = line["config"]["global_batch"]
    rf = line["roofline"]
    out["roofline"] = {k: rf[k] for k in ("bound", "achieved", "peak", "unit", "frac", "kernel", "ms_per_launch")
                       if k in rf}
    return out


def config_legs(a, H, rng, stream):
    """The other configurations, each timed on its own, with its roofline fraction and its parity windows against
    the oracle: config 1 (the depthwise convs at 5x5 stride 1, fp16 and int8, batch 64), config 2 (the fp16
    Winograd conv, batch 64), config 3 (the v2.4-shaped fp16 net, batch 256: its exact fp16 path, and its fp16
    1x1 convs on fp16 MFMA within the stated tolerance)."""
    legs = {}
    # each leg follows host work (input generation, the previous leg's oracle check) during which the GPU's clocks
    # fall; a few hundred untimed launches (~30 ms of load) bring them back up before the timed ones
    for kind in ("f16", "s8"):
        b = argparse.Namespace(**vars(a))
        b.workload, b.k, b.s, b.no_cpu, b.steps, b.warmup = "dw_" + kind, 5, 1, True, max(200, a.steps), 400
        legs[f"config1_dw_{kind}"] = compact_leg(run_dw(b, H, rng, 64, stream, emit=False))
    b = argparse.Namespace(**vars(a))
    b.workload, b.no_cpu, b.steps, b.warmup = "wino_f16", True, max(200, a.steps), 200
    legs["config2_wino_f16"] = compact_leg(run_wino(b, H, rng, 64, stream, emit=False))
    b = argparse.Namespace(**vars(a))
    b.workload, b.no_cpu, b.steps, b.warmup = "v24_f16", True, max(20, a.steps), 10
    legs["config3_v24_f16"] = compact_leg(run_v24(b, H, rng, 256, stream, emit=False))
    # the same net with its fp16 1x1 convs on fp16 MFMA (fp32 accumulation): within the configuration's stated
    # fp16 tolerance against the exact path, not bit-identical; priced against the fp16 MFMA peak
    b = argparse.Namespace(**vars(a))
    b.workload, b.no_cpu, b.steps, b.warmup, b.f16_mfma = "v24_f16", True, max(20, a.steps), 10, True
    try:
        legs["config3_v24_f16_mfma"] = compact_leg(run_v24(b, H, rng, 256, stream, emit=False))
    finally:
        os.environ.pop("BNH_F16_MFMA", None)   # read by bnn_init: the exact path for any later context
    return legs


# Counter figures of the fused kernel's launch below (24 -> 144 expansion into the 3 x 3 stride-2 depthwise,
# 249 x 63 -> 125 x 32 pixels, 256 windows), from rocprofv3 --pmc runs of this bench, named with their source:
# HBM bytes per launch (FETCH_SIZE x 2 + WRITE_SIZE, the copy-kernel calibration) and the VALU wave instructions per
# launch. The VALU issue share is computed in the run from the instruction count and this run's launch time: a wave64
# VALU instruction occupies a 16-lane SIMD for 4 cycles; the chip has 1,024 SIMDs at 2.4 GHz.
PERCH_PWDW_PROFILE = "profiles/k_pwdw_f32_24to144_dw3s2_249x63_b256.md"
PERCH_PWDW_TRAFFIC = 775128064
PERCH_PWDW_VALU_INSTS = 486559744
SIMDS, SCLK_HZ = 1024, 2.4e9


def perch_pairs(net):
    """The (PW_S8 expansion, depthwise) op pairs the runtime fuses into k_pwdw_f32: a PW_S8 with a zero-haloed output
    that the next op, a DW3 / DWK, reads."""
    out = []
    for x, y in zip(net.ops, net.ops[1:]):
        if x[0] & 0xff == 22 and x[3][9] > 0 and y[0] & 0xff in (4, 10) and y[1][0] == x[1][1]:
            out.append((x, y))
    return out


def perch_roofline(H, pn, B, stream, a):
    """The dominant kernel of the net is the int8 expansion fused into its depthwise conv (k_pwdw_f32, the largest
    share of the step); its largest launch, block 2's 24 -> 144 expansion into the 3 x 3 stride-2 depthwise over
    249 x 63 pixels, is replayed with the net's own weights and shape on `stream` and timed with events. Algorithmic
    bytes per launch: the int8 rows and their scales and zero points read (B x M x (Kp + 8)), the depthwise outputs
    written (B x Ho x Wo x C x 4) and the weights. The kernel recomputes the expansion instead of storing it, so it
    is bound by VALU issue (dequantisation and the exact SiLU of every expanded value), not by HBM: valu_busy is the
    measured share of the SIMDs' issue cycles its VALU instructions take."""
    # the launch with the most expansion work: pixels x expanded channels
    (pc, pbf, ptn, pp), (dc, dbf, dtn, dp) = max(perch_pairs(pn.net), key=lambda pr: pr[0][3][4] * pr[0][3][0])
    N, K, Kp, Np, M, lda, act, ldo, ow, opad, ldr = pp
    if dc & 0xff == 4:  # DW3: H W C s Ho Wo, pads 1, SiLU
        Hh, Wd, C, s, Ho, Wo = dp[:6]
        k, pt, pl, form, dact = 3, 1, 1, 2, 1
    else:               # DWK: H W C k s pt pl Ho Wo act
        Hh, Wd, C, k, s, pt, pl, Ho, Wo, dact = dp
        form = 0
    T = [arr for (_, arr, _) in pn.pkg.tensors]
    Wt = H.S8Weights(N, K, Kp, Np, T[ptn[0]], T[ptn[1]], T[ptn[2]], T[ptn[3]])
    dw = H.DeviceArray.from_host(np.asarray(T[dtn[0]], np.float32))
    db = H.DeviceArray.from_host(np.asarray(T[dtn[1]], np.float32))
    rng = np.random.default_rng(5)
    dq = H.DeviceArray.from_host(rng.integers(-127, 128, (B, M * Kp)).astype(np.int8))
    dsa = H.DeviceArray.from_host(rng.uniform(0.005, 0.02, (B, M)).astype(np.float32))
    dza = H.DeviceArray.from_host(rng.integers(-20, 20, (B, M)).astype(np.int32))
    o_ws = Ho * Wo * C
    dout = H.DeviceArray.zeros((B, o_ws), np.float32)

    def launch():
        H.check(H.lib().bnh_pwdw_f32(dq.ptr, M * Kp, dsa.ptr, M, dza.ptr, M, Hh, Wd, Wt.h, act, k, s, pt, pl, form,
                                     dw.ptr, db.ptr, dact, dout.ptr, o_ws, Ho, Wo, None, 0, B, stream), "pwdw_f32")
    ms, _ = time_steps(H, stream, launch, max(10, a.steps), 3)
    nbytes = B * M * (Kp + 8) + B * o_ws * 4 + Np * Kp + 12 * Np + (k * k + 1) * C * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    # the profile counted one launch over 256 windows; every window runs the same instructions
    insts = PERCH_PWDW_VALU_INSTS * B / 256
    issue = insts / (ms * 1e-3) / 1e9                      # G wave-instructions / s
    peak_issue = SIMDS * SCLK_HZ / 4 / 1e9                  # a wave64 VALU instruction holds a SIMD 4 cycles
    return {"bound": "valu", "achieved": round(issue, 1), "peak": round(peak_issue, 1),
            "unit": "G VALU wave-instructions/s", "frac": round(issue / peak_issue, 4),
            "traffic": PERCH_PWDW_TRAFFIC if B == 256 else None,
            "kernel": "k_pwdw_f32",
            "launch": f"PW_S8 {K}->{N} expansion fused into the {k}x{k}/{s} depthwise, {Hh}x{Wd} -> {Ho}x{Wo} px "
                      f"x {B} windows",
            "ms_per_launch": round(ms, 4), "valu_wave_insts_per_launch": int(insts),
            "algorithmic_bytes_per_launch": nbytes,
            "hbm": {"achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gbs / HBM_PEAK_GBS, 4)},
            "note": "the kernel recomputes each expanded value (dequantisation + exact SiLU) instead of storing it, "
                    "so VALU issue binds it, not HBM: frac = its VALU wave instructions x 4 cycles / (this run's "
                    "launch time x 2.4 GHz x 1,024 SIMDs); instruction count and traffic from " + PERCH_PWDW_PROFILE}


def v24_counts(net):
    """(fp16 FLOPs per window of the 1x1 convs and the head, the PW op record with the most FLOPs)."""
    flops, big = 0, None
    for code, b, t, p in net.ops:
        if code == 3 | 1 << 8:   # PW f16: N K Kp Np M ...
            flops += 2 * p[0] * p[1] * p[4]
            if big is None or p[0] * p[1] * p[4] > big[3][0] * big[3][1] * big[3][4]:
                big = (code, b, t, p)
        elif code == 15 | 1 << 8:   # GEMV, fp16 weights
            flops += 2 * p[0] * p[1]
    return flops, big


def cpu_baseline_v24(vn, rng):
    """The oracle's op-by-op run of the same package, one window per thread, on a bounded sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_net
    from bnneon import v24net
    T = cpu_threads()
    n_win = 2 * T   # about 20 s of the host's cores
    on = oracle_net.OracleNet(vn.net, 0, vn.net.last, vn.emb_buf)
    pcms = [v24net.signal(rng) for _ in range(n_win)]
    t0 = time.perf_counter()
    with concurrent.futures.ThreadPoolExecutor(T) as ex:
        list(ex.map(lambda i: on.run(pcms[i]), range(n_win)))
    dt = time.perf_counter() - t0
    return {"value": round(n_win / dt, 3), "unit": "windows/s", "cores": T, "kind": "port",
            "sample": f"{n_win} windows of the same package through the scalar C oracle's op-by-op "
                      f"restatement (log-mel, stem, 16 blocks, head), one window per thread ({T} threads), "
                      f"-O2 -ffp-contract=off; {dt:.2f} s wall"}


def run_v24(a, H, rng, B, stream, emit=True):
    import tempfile
    from bnneon import binding, v24net
    vn = v24net.V24Net(seed=7)
    tmp = tempfile.mkdtemp(prefix="bnn_bench_")
    path = vn.write(os.path.join(tmp, "birdnet_v24_shaped_f16.bnpk"))
    L = binding.load_library()
    if a.f16_mfma:
        os.environ["BNH_F16_MFMA"] = "1"   # read by bnn_init
    m = binding.Model(path)
    os.unlink(path)
    os.rmdir(tmp)
    nc, ne, ns = m.info.n_classes, m.info.emb_dim, m.info.n_samples
    pcm = np.stack([v24net.signal(rng) for _ in range(min(B, 16))])
    pcm = np.concatenate([pcm] * ((B + len(pcm) - 1) // len(pcm)))[:B]
    dx = H.DeviceArray.from_host(pcm)
    dout = H.DeviceArray.zeros((B, nc), np.float32)
    demb = H.DeviceArray.zeros((B, ne), np.float32)
    status = np.zeros(B, np.int32)
    sp = status.ctypes.data_as(binding._IP)

    def launch():
        r = L.bnn_infer_batch_device(m.ctx, dx.ptr, B, dout.ptr, demb.ptr, sp, stream)
        if r != 0:
            raise RuntimeError(f"bnn_infer_batch_device returned {r}: {L.bnn_last_error()}")
    ms, wall = time_steps(H, stream, launch, a.steps, a.warmup)
    flops_win, _ = v24_counts(vn.net)
    line = {
        "metric": METRIC, "value": round(B / (ms * 1e-3), 1), "unit": "windows/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: -30 dBFS noise + 3 chirps 1-10 kHz per window; random weights",
        "config": {"workload": "BirdNET-v2.4-shaped fp16 net (log-mel 257x96, stem 3x3/2 -> 24, 16 MBConv blocks "
                               "24-36-72-108-192 with SE, exact fp16 1x1 convs, fp16 depthwise, 192->1024 head "
                               "conv, mean, 6,522-class fp16 GEMV), 144,000 samples @ 48 kHz per window",
                   "global_batch": B, "n_samples": ns, "n_classes": nc,
                   "parallelism": "1 GPU, windows batched per launch",
                   "fp16_gemm": ("fp16 MFMA, fp32 accumulation (within the fp16 accumulation bound)" if a.f16_mfma
                                 else "the reference's exact fp16 FMA chains (bit-identical)"),
                   "wall_s_timed_region": round(wall, 4)},
        "fp16_tflops": round(flops_win * B / (ms * 1e-3) / 1e12, 3),
    }
    if a.f16_mfma:
        line["config"]["workload"] = line["config"]["workload"].replace("exact fp16 1x1 convs",
                                                                      "fp16-MFMA 1x1 convs")
    line["roofline"] = v24_roofline(H, vn, B, stream, a)
    m.close()
    line["parity_windows"] = v24_parity(vn, pcm, dout.numpy(), nc, (0, B - 1), a.f16_mfma)
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline_v24(vn, rng)
    if not emit:
        return line
    print(json.dumps(line), flush=True)


def v24_parity(vn, pcm, logits, nc, wins, f16_mfma):
    """The batch's logits of windows `wins` against the oracle's op-by-op run of the package: bit for bit for the
    exact path; for the fp16-MFMA form, the largest logit difference and top-1 agreement."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_net
    on = oracle_net.OracleNet(vn.net, 0, vn.net.last, vn.emb_buf)
    with concurrent.futures.ThreadPoolExecutor(len(wins)) as ex:   # one window per thread
        refs = list(ex.map(lambda i: on.run(pcm[i])[0][:nc].copy(), wins))
    if not f16_mfma:
        same = sum(bool(np.array_equal(logits[i].view(np.uint32), r.view(np.uint32))) for i, r in zip(wins, refs))
        return f"{same}/{len(wins)} windows' logits bit-identical to the oracle's (windows {list(wins)})"
    d = max(float(np.abs(logits[i] - r).max()) for i, r in zip(wins, refs))
    top = sum(int(np.argmax(logits[i]) == np.argmax(r)) for i, r in zip(wins, refs))
    rng_ = max(float(r.max() - r.min()) for r in refs)
    return (f"windows {list(wins)} against the oracle's exact path: max |logit difference| {d:.3g} of a "
            f"{rng_:.3g} logit range, top-1 {top}/{len(wins)}")


FP16_MFMA_PEAK_TFLOPS = 2500.0
# HBM bytes per launch of the replayed fp16 GEMM (72 -> 864 channels, 384 px, 256 windows): FETCH_SIZE x 2 +
# WRITE_SIZE from rocprofv3 --pmc runs of this bench (profiles/k_gemm_f16e_pw_f16_72to864_24x16_b256.md)
V24_GEMM_TRAFFIC = 185333824
FP16_VALU_PEAK_TFLOPS = 157.3


def v24_roofline(H, vn, B, stream, a):
    """The net's largest fp16 1x1 conv (by FLOPs) replayed through bnh_gemm_f16 with the net's own weights and
    shape on `stream`, timed with events. The exact GEMM keeps the reference's fp16 accumulation, so it runs on
    packed fp16 VALU FMAs, not MFMA: the roofline is priced against the packed-fp16 VALU peak that bounds it, with
    the fp16 MFMA pricing beside it (the MFMA form, --f16-mfma, is priced against MFMA)."""
    import ctypes
    _, big = v24_counts(vn.net)
    code, b, t, p = big
    N, K, Kp, Np, M, lda, act, ldo, ow, opad, ldr = p
    T = [arr for (_, arr, _) in vn.pkg.tensors]
    w, b32, b16 = (np.ascontiguousarray(T[i]) for i in t)
    hw = H.lib().bnh_h16w_new(N, K, Kp, Np, w.ctypes.data, b32.ctypes.data, b16.ctypes.data)
    if not hw:
        H.check(None, "bnh_h16w_new")
    rng = np.random.default_rng(5)
    dA = H.DeviceArray.from_host(rng.standard_normal((B, M * lda)).astype(np.float16))
    Hh = M // ow if opad else M
    rows = (Hh + 2 * opad) * (ow + 2 * opad) if opad else M
    dout = H.DeviceArray.zeros((B, rows * ldo), np.float16)
    e = H.Epi16(act, dout.ptr, rows * ldo, ldo, ow if opad else 0, opad, None, 0, 0)

    def launch():   # the GEMM kernel alone: the halo was zeroed once (as the net's arena slots keep it)
        if a.f16_mfma:
            H.check(H.lib().bnh_gemm_f16_mfma(dA.ptr, M * lda, lda, M, B, hw, ctypes.byref(e), stream))
        else:
            H.check(H.lib().bnh_gemm_f16_body(dA.ptr, M * lda, lda, M, B, hw, ctypes.byref(e), stream))
    H.check(H.lib().bnh_gemm_f16(dA.ptr, M * lda, lda, M, B, hw, ctypes.byref(e), stream))
    ms, _ = time_steps(H, stream, launch, max(10, a.steps), 3)
    H.lib().bnh_h16w_free(hw)
    tf = 2.0 * M * N * K * B / (ms * 1e-3) / 1e12
    hbm_bytes = B * (M * lda + rows * ldo) * 2 + Np * Kp * 2   # fp16 rows in and out, the weights once
    gbps = hbm_bytes / (ms * 1e-3) / 1e9
    r = {"bound": "mfma", "achieved": round(tf, 2), "peak": FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
         "frac": round(tf / FP16_MFMA_PEAK_TFLOPS, 4), "traffic": V24_GEMM_TRAFFIC,
         "kernel": "k_gemm_f16" if a.f16_mfma else "k_gemm_f16e",
         "launch": f"PW f16 GEMM {K}->{N} over {M} px x {B} windows, act {act}, halo-{opad} output",
         "ms_per_launch": round(ms, 4), "algorithmic_flops_per_launch": 2 * M * N * K * B,
         "algorithmic_bytes_per_launch": hbm_bytes, "hbm_GBps": round(gbps, 1), "hbm_frac": round(gbps / 8000.0, 4)}
    if not a.f16_mfma:
        # the exact GEMM's binding resource is the packed fp16 VALU (the matrix cores cannot keep fp16 sums):
        # the roofline is priced against it, with the MFMA pricing beside it
        r.update({"bound": "valu", "peak": FP16_VALU_PEAK_TFLOPS, "frac": round(tf / FP16_VALU_PEAK_TFLOPS, 4),
                  "mfma": {"peak": FP16_MFMA_PEAK_TFLOPS, "frac": round(tf / FP16_MFMA_PEAK_TFLOPS, 4)}})
    return r


if __name__ == "__main__":
    main()
