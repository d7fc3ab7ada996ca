"""GPU parity of the int8 pointwise GEMMs against the CPU oracle: bit-exact.

libbnneon_hip (through its C ABI) vs oracle/s8n.c on the same seeded inputs:
the device numerics (FRECPE, SiLU, ReLU) on exhaustive / adversarial inputs,
per-row quantization (every K tail form, constant / zero / huge-offset / NaN
rows, the SE gate), the whole PW_S8 op (activations, residual, zero-haloed
output, batches of windows with padded strides) and the Q31-requantised NCHW
GEMM at the 1152 -> 256, 24 x 64 pixel shape.
"""
import numpy as np
import pytest

import pyoracle as O
from bnneon import s8pack

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same_f32(a, b):
    """Bit equality, any NaN equal to any NaN."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    an, bn = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(an, bn) and
                np.array_equal(a.view(np.uint32)[~an], b.view(np.uint32)[~bn]))


def adversarial_floats(rng, n):
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45,
                        1.17e-38, 2.0 ** -127, 2.0 ** -128, 2.0 ** -129,
                        3.4e38, -3.4e38, 41.6, 41.59, -41.6, 60.0, -60.0,
                        86.5, -87.3, 1.0, -1.0, 0.5], np.float32)
    bitsr = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([special, bitsr.view(np.float32),
                           rng.standard_normal(n).astype(np.float32) * 8])


def run_eval(H, f, x):
    d = H.DeviceArray.from_host(x)
    y = H.DeviceArray.zeros(x.shape, np.float32)
    H.check(H.lib().bnh_eval_f32(f, d.ptr, y.ptr, x.size, None), "eval")
    H.sync()
    return y.numpy()


def test_frecpe_every_significand_and_exponent(hip):
    # all 2^23 significands of [1, 2) and a spread of exponents incl. denormals
    sig = np.arange(2 ** 23, dtype=np.uint32) | np.uint32(127 << 23)
    xs = [sig.view(np.float32)]
    rng = np.random.default_rng(0)
    for e in list(range(0, 255, 3)) + [1, 2, 253, 254]:
        s = rng.integers(0, 2 ** 23, 4096, dtype=np.uint64).astype(np.uint32)
        xs.append(((s | np.uint32(e << 23)) | np.uint32(rng.integers(0, 2) << 31)).view(np.float32))
    x = np.concatenate(xs + [adversarial_floats(rng, 4096)])
    say("frecpe", x.size)
    assert same_f32(run_eval(hip, 0, x), O.eval_f32(0, x))


@pytest.mark.parametrize("f", [1, 2])
def test_silu_relu_bit_exact(hip, f):
    rng = np.random.default_rng(1)
    x = np.concatenate([adversarial_floats(rng, 200000),
                        np.linspace(-100, 100, 200001).astype(np.float32)])
    say("eval", f, x.size)
    assert same_f32(run_eval(hip, f, x), O.eval_f32(f, x))


def test_silu_dense(hip):
    """every 16th float of both signs with |x| in [2^-27, 2^34) (past +-41.6 the clamp saturates), NaNs and
    infinities: the epilogue SiLU's divisor covers its whole range; both device forms (with and without the LDS
    estimate table)."""
    e = np.arange(100, 161, dtype=np.uint32)
    m = np.arange(0, 2 ** 23, 16, dtype=np.uint32)
    bits = (e[:, None] << np.uint32(23)) | m[None, :]
    bits = np.concatenate([bits.ravel(), bits.ravel() | np.uint32(0x80000000),
                           np.array([0x7f800000, 0xff800000, 0x7fc00000, 0xffc00001, 0x7f800001], np.uint32)])
    x = bits.view(np.float32)
    say("silu dense", x.size)
    want = O.eval_f32(1, x)
    assert same_f32(run_eval(hip, 1, x), want)   # the LDS-table form the epilogues use
    assert same_f32(run_eval(hip, 3, x), want)   # the form without the table


def quant_case(hip, x, K, Kp, gate=None, B=1):
    """x [B][M][ld]; returns True when q, sa, za match the oracle."""
    H = hip
    B, M, ld = x.shape
    M4 = (M + 3) // 4 * 4
    q_ws = M4 * Kp + 64          # padded per-window strides
    s_ws = M4 + 8
    x_ws = M * ld + 32
    xh = np.zeros((B, x_ws), np.float32)
    xh[:, :M * ld] = x.reshape(B, -1)
    dx = H.DeviceArray.from_host(xh)
    dq = H.DeviceArray.zeros((B, q_ws), np.int8)
    dsa = H.DeviceArray.zeros((B, s_ws), np.float32)
    dza = H.DeviceArray.zeros((B, s_ws), np.int32)
    dg, g_ws = None, 0
    if gate is not None:
        g_ws = K + 4
        gh = np.zeros((B, g_ws), np.float32)
        gh[:, :K] = gate
        dg = H.DeviceArray.from_host(gh)
    H.check(H.lib().bnh_s8n_quant_rows(dx.ptr, x_ws, ld, M, K, Kp, H.ptr(dg), g_ws,
                                       dq.ptr, q_ws, dsa.ptr, s_ws, dza.ptr, s_ws, B, None), "quant")
    H.sync()
    q, sa, za = dq.numpy(), dsa.numpy(), dza.numpy()
    ok = True
    for b in range(B):
        oq, osa, oza = O.quant_rows(x[b], K, Kp, None if gate is None else gate[b])
        ok &= np.array_equal(q[b, :M * Kp].reshape(M, Kp), oq)
        ok &= same_f32(sa[b, :M], osa) and np.array_equal(za[b, :M], oza)
    return ok


@pytest.mark.parametrize("K", [1, 3, 4, 7, 8, 13, 24, 40, 144, 816, 1152, 1392])
def test_quant_rows_random(hip, K):
    rng = np.random.default_rng(K)
    Kp = s8pack.r16(K)
    B, M = 3, 37
    ld = K + (K % 3)
    x = (rng.standard_normal((B, M, ld)) * rng.uniform(1e-3, 1e3, (B, M, 1))
         + rng.uniform(-10, 10, (B, M, 1))).astype(np.float32)
    say("quant K", K)
    assert quant_case(hip, x, K, Kp)


def test_quant_rows_edge_rows(hip):
    rng = np.random.default_rng(11)
    K, Kp, M = 21, 32, 12   # K % 4 = 1 and K % 8 = 5: both tail forms
    x = rng.standard_normal((1, M, K)).astype(np.float32)
    x[0, 0] = 3.25                      # constant row
    x[0, 1] = 0.0                       # zero row
    x[0, 2] = 1e10 + rng.uniform(0, 1e3, K)   # far offset: out-of-range conversions
    x[0, 3, 5] = np.nan                 # NaN in the 4-lane part
    x[0, 4, 20] = np.nan                # NaN in the scalar tail
    x[0, 5, 2] = np.inf
    x[0, 6] = -1e-40                    # denormal constant row
    x[0, 7, :] = rng.standard_normal(K) * 1e-38
    x[0, 8, 0] = -3e38
    x[0, 8, 1] = 3e38                   # range overflows to inf
    say("quant edge rows")
    assert quant_case(hip, x, K, Kp)


def test_quant_rows_gate(hip):
    rng = np.random.default_rng(12)
    K, Kp, M, B = 96, 96, 29, 2
    x = rng.standard_normal((B, M, K)).astype(np.float32)
    g = rng.uniform(0, 1, (B, K)).astype(np.float32)
    say("quant gate")
    assert quant_case(hip, x, K, Kp, gate=g)


def pw_case(hip, B, H_, W_, K, N, act, opad=0, res=False, lda_extra=0, seed=0, gate=False, ldo_extra=8, rpad=0,
            wins=None):
    H = hip
    rng = np.random.default_rng(seed)
    M = H_ * W_
    lda = K + lda_extra
    w = (rng.standard_normal((N, K)) * rng.uniform(0.01, 1, (N, 1))).astype(np.float32)
    w[0] = 0                                  # an all-zero channel
    b = rng.standard_normal(N).astype(np.float32)
    pk = s8pack.pack_s8(w, b)
    N_, K_, Kp, Np = pk["shape"]
    x = (rng.standard_normal((B, M, lda)) * 2).astype(np.float32)
    gt = rng.uniform(0, 1, (B, K)).astype(np.float32) if gate else None
    ldo = Np + ldo_extra
    out_rows = M if not opad else (H_ + 2 * opad) * (W_ + 2 * opad)
    rrows = (H_ + 2 * rpad) * (W_ + 2 * rpad) if rpad else M
    rs = rng.standard_normal((B, rrows, Np)).astype(np.float32) if res else None
    if res and rpad:  # a zero-haloed residual buffer, as the runtime's haloed activations
        rs.reshape(B, H_ + 2 * rpad, W_ + 2 * rpad, Np)[:, :rpad] = 0
        rs.reshape(B, H_ + 2 * rpad, W_ + 2 * rpad, Np)[:, -rpad:] = 0
        rs.reshape(B, H_ + 2 * rpad, W_ + 2 * rpad, Np)[:, :, :rpad] = 0
        rs.reshape(B, H_ + 2 * rpad, W_ + 2 * rpad, Np)[:, :, -rpad:] = 0
    M4 = (M + 3) // 4 * 4
    Wt = H.S8Weights(N_, K_, Kp, Np, pk["q"], pk["sw"], pk["cs"], pk["b"])
    dx = H.DeviceArray.from_host(x)
    dg = H.DeviceArray.from_host(gt) if gate else None
    dq = H.DeviceArray.zeros((B, M4 * Kp), np.int8)
    dsa = H.DeviceArray.zeros((B, M4), np.float32)
    dza = H.DeviceArray.zeros((B, M4), np.int32)
    # the output starts as garbage: the halo must be zeroed by the op
    dout = H.DeviceArray.from_host(np.full((B, out_rows * ldo), 7.0, np.float32))
    dres = H.DeviceArray.from_host(rs) if res else None
    e = H.epi32(dout, ldo, act=act, ow=W_ if opad else 0, opad=opad, res=dres,
                ldr=Np if res else 0, rpad=rpad, rw=W_ if rpad else 0, out_ws=out_rows * ldo, res_ws=rrows * Np)
    say(f"pw_s8 B{B} {H_}x{W_} K{K} N{N} act{act} opad{opad} res{res} gate{gate}")
    H.check(H.lib().bnh_pw_s8(dx.ptr, M * lda, lda, M, H.ptr(dg), K if gate else 0, dq.ptr, M4 * Kp,
                              dsa.ptr, M4, dza.ptr, M4, B, Wt.h, e, None), "pw_s8")
    H.sync()
    out = dout.numpy().reshape(B, out_rows, ldo)
    q = dq.numpy().reshape(B, M4, Kp)
    ok = True
    for bi in (range(B) if wins is None else wins):
        ref_out, rq, rsa, rza = O.pw_s8(x[bi], pk, act=act, ldo=ldo, ow=W_ if opad else 0, opad=opad,
                                        res=None if rs is None else rs[bi], ldr=Np if res else 0,
                                        rpad=rpad, rw=W_ if rpad else 0, gate=None if gt is None else gt[bi])
        got = out[bi].copy()
        # columns [Np, ldo) are never written: the garbage stays, as in the reference
        ok &= same_f32(got[:, :Np], ref_out[:, :Np])
        ok &= np.array_equal(q[bi, :M], rq[:M])
    return ok


@pytest.mark.parametrize("act", [0, 1, 2])
def test_pw_s8_perch_shapes(hip, act):
    for (H_, W_, K, N) in ((25, 13, 40, 24), (13, 8, 144, 32), (8, 8, 1392, 232), (4, 4, 232, 1392)):
        assert pw_case(hip, 2, H_, W_, K, N, act, seed=H_ * K + act)


def test_pw_s8_config0_shape(hip):
    assert pw_case(hip, 2, 24, 64, 1152, 256, 1, seed=5)


def test_pw_s8_large_k_tile_kernel(hip):
    """Kp >= 256 with rows for 1024+ tiles: the LDS-staged tile GEMM (k_s8n_gemm_lds). 128 x 256 tiles at config 0's
    1152 -> 256 (86 windows); 256 x 128 tiles with a residual from a zero-haloed buffer into a haloed output
    (N = 100); ldo odd (values stored one by one) with a gate; windows at both ends and the middle checked"""
    assert pw_case(hip, 86, 24, 64, 1152, 256, 1, seed=41, wins=(0, 43, 85))
    assert pw_case(hip, 128, 32, 64, 320, 100, 2, opad=1, res=True, rpad=1, seed=42, wins=(0, 77, 127))
    assert pw_case(hip, 86, 24, 64, 256, 200, 0, seed=43, gate=True, ldo_extra=1, wins=(0, 85))


def test_pw_s8_residual_halo_gate(hip):
    assert pw_case(hip, 3, 7, 9, 48, 40, 1, opad=2, res=True, lda_extra=5, seed=9)
    assert pw_case(hip, 2, 5, 6, 96, 136, 2, opad=1, seed=10, gate=True)
    assert pw_case(hip, 1, 1, 1, 24, 8, 0, seed=11)   # a single row (GEMV-like)


def test_pw_s8_residual_quads_split_groups(hip):
    """The residual epilogue's 16-byte-quad form (ldo and ldr multiples of 4) with three 64-channel groups, the last
    one partial (N = 136), the groups split over blocks (few rows: gsplit > 1), and zero-haloed residual and output
    buffers (rpad 1, opad 1), as well as an unhaloed residual into a haloed output."""
    assert pw_case(hip, 3, 7, 9, 48, 136, 1, opad=1, res=True, rpad=1, seed=14)
    assert pw_case(hip, 2, 6, 11, 96, 136, 0, opad=2, res=True, rpad=0, seed=15)
    assert pw_case(hip, 2, 5, 5, 232, 200, 2, opad=0, res=True, rpad=2, seed=16, gate=True)


def test_pw_s8_unaligned_output_rows(hip):
    # output rows 4-byte aligned only (ldo odd): the epilogue's one-value-per-access form; with a residual and ldo a
    # multiple of 4 (above) the GEMM takes the 16-byte-quad form through LDS
    assert pw_case(hip, 2, 9, 11, 144, 24, 0, res=True, seed=12, ldo_extra=3)
    assert pw_case(hip, 2, 7, 5, 40, 136, 1, opad=1, seed=13, ldo_extra=1)


def test_gemm_requant_config0(hip):
    H = hip
    rng = np.random.default_rng(2024)
    N, K, M, B = 256, 1152, 1536, 2
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    x = np.clip(np.round(rng.normal(-40, 35, (B, K, M))), -128, 127).astype(np.int8)
    bias = rng.integers(-2 ** 14, 2 ** 14 + 1, N).astype(np.int32)
    mult = rng.integers(2 ** 30, 2 ** 31, N).astype(np.int32)
    shift = rng.integers(6, 11, N).astype(np.int32)
    Wq = H.Q8Weights(w, bias, mult, shift, -128, -128)
    dx = H.DeviceArray.from_host(x)
    dout = H.DeviceArray.zeros((B, N, M), np.int8)
    say("requant gemm config0 B2")
    H.check(H.lib().bnh_gemm_s8_requant(Wq.h, dx.ptr, K * M, M, B, dout.ptr, N * M, None), "requant")
    H.sync()
    got = dout.numpy()
    for b in range(B):
        ref = O.gemm_s8_requant(w, x[b], bias, mult, shift, -128, -128)
        assert np.array_equal(got[b], ref), (b, np.argwhere(got[b] != ref)[:5])


def test_gemm_requant_small_shapes(hip):
    H = hip
    rng = np.random.default_rng(7)
    for (N, K, M) in ((8, 16, 4), (24, 48, 68), (136, 144, 132), (300, 80, 256)):
        w = rng.integers(-127, 128, (N, K)).astype(np.int8)
        x = rng.integers(-128, 128, (1, K, M)).astype(np.int8)
        bias = rng.integers(-2 ** 20, 2 ** 20, N).astype(np.int32)
        mult = rng.integers(2 ** 30, 2 ** 31, N).astype(np.int32)
        shift = rng.integers(0, 16, N).astype(np.int32)
        Wq = H.Q8Weights(w, bias, mult, shift, 3, -5, -100, 90)
        dx = H.DeviceArray.from_host(x)
        dout = H.DeviceArray.zeros((N, M), np.int8)
        say("requant", N, K, M)
        H.check(H.lib().bnh_gemm_s8_requant(Wq.h, dx.ptr, K * M, M, 1, dout.ptr, N * M, None), "requant")
        H.sync()
        assert np.array_equal(dout.numpy(), O.gemm_s8_requant(w, x[0], bias, mult, shift, 3, -5, -100, 90))


def test_gemm_requant_ring_kernel_shapes(hip):
    """Pixel counts that are multiples of 16 (the direct-to-LDS kernel): a
    single 16-pixel column, a partial last pixel tile, one K step, a K tail
    inside the last step, channel counts past one 256-channel block, and
    windows at padded (16-byte multiple) strides."""
    H = hip
    rng = np.random.default_rng(77)
    for (N, K, M, B, slack) in ((8, 16, 16, 1, 0), (24, 48, 144, 3, 16), (256, 64, 272, 2, 48),
                                (520, 208, 128, 2, 0), (40, 1152, 1536, 3, 4096)):
        w = rng.integers(-127, 128, (N, K)).astype(np.int8)
        x = rng.integers(-128, 128, (B, K, M)).astype(np.int8)
        bias = rng.integers(-2 ** 20, 2 ** 20, N).astype(np.int32)
        mult = rng.integers(2 ** 30, 2 ** 31, N).astype(np.int32)
        shift = rng.integers(0, 16, N).astype(np.int32)
        Wq = H.Q8Weights(w, bias, mult, shift, -7, 4, -120, 127)
        x_ws = K * M + slack
        xs = np.zeros((B, x_ws), np.int8)
        xs[:, :K * M] = x.reshape(B, -1)
        o_ws = N * M + 32
        dx = H.DeviceArray.from_host(xs)
        dout = H.DeviceArray.zeros((B, o_ws), np.int8)
        say("requant ring", N, K, M, B)
        H.check(H.lib().bnh_gemm_s8_requant(Wq.h, dx.ptr, x_ws, M, B, dout.ptr, o_ws, None), "requant")
        H.sync()
        got = dout.numpy()
        for b in range(B):
            ref = O.gemm_s8_requant(w, x[b], bias, mult, shift, -7, 4, -120, 127)
            assert np.array_equal(got[b, :N * M].reshape(N, M), ref), (N, K, M, b)
            assert not got[b, N * M:].any()   # nothing written past the window's output


def test_gemm_requant_output_rows_4_byte_aligned(hip):
    """Window output strides that are multiples of 4 but not of 16: the ring kernel whose epilogue stages the tile in
    LDS and stores whole rows (the ping-pong kernel stores 16 bytes per lane and needs 16-byte aligned rows)."""
    H = hip
    rng = np.random.default_rng(78)
    for (N, K, M, B) in ((24, 48, 144, 3), (256, 1152, 512, 2)):
        w = rng.integers(-127, 128, (N, K)).astype(np.int8)
        x = rng.integers(-128, 128, (B, K, M)).astype(np.int8)
        bias = rng.integers(-2 ** 20, 2 ** 20, N).astype(np.int32)
        mult = rng.integers(2 ** 30, 2 ** 31, N).astype(np.int32)
        shift = rng.integers(1, 16, N).astype(np.int32)
        Wq = H.Q8Weights(w, bias, mult, shift, -7, 4, -120, 127)
        o_ws = N * M + 4
        dx = H.DeviceArray.from_host(x)
        dout = H.DeviceArray.zeros((B, o_ws), np.int8)
        say("requant 4-byte rows", N, K, M, B)
        H.check(H.lib().bnh_gemm_s8_requant(Wq.h, dx.ptr, K * M, M, B, dout.ptr, o_ws, None), "requant")
        H.sync()
        got = dout.numpy()
        for b in range(B):
            ref = O.gemm_s8_requant(w, x[b], bias, mult, shift, -7, 4, -120, 127)
            assert np.array_equal(got[b, :N * M].reshape(N, M), ref), (N, K, M, b)
            assert not got[b, N * M:].any()


def test_gemm_requant_short_epilogue(hip):
    """Output zero points at or below the clamp's low end (zy <= lo) with every shift in 1..31 and bias_eff small
    enough that acc + bias_eff cannot wrap: the kernel folds bias, rounding and the zero point into one 64-bit
    multiply-add per output and adds zy bytewise. Covers shifts 1 and 31, negative, zero and extreme multipliers,
    zy = lo (config 0), zy < lo, zy >= 0 (a bytewise add with no wrap), partial tiles and K tails; then the same data
    with bias_eff one past the bound, which must take the general path and agree as well."""
    H = hip
    rng = np.random.default_rng(31)
    K_BOUND = 16384
    cases = ((256, 1152, 1536, 2, -128, -128, 127), (40, 208, 272, 3, -20, -10, 100), (300, 64, 256, 1, -128, -100, 90),
             (24, 48, 144, 2, 0, 0, 127), (136, 1152, 512, 2, 5, 5, 127),
             # zy far below lo: hi - zy = 327 does not fit a byte, so the general epilogue must run
             (64, 208, 272, 2, -200, -128, 127), (32, 64, 144, 1, -129, -128, 127))
    for (N, K, M, B, zy, lo, hi) in cases:
        zx = -128 if zy == -128 else -3
        w = rng.integers(-128, 128, (N, K)).astype(np.int8)
        x = rng.integers(-128, 128, (B, K, M)).astype(np.int8)
        mult = rng.integers(-2 ** 31, 2 ** 31, N).astype(np.int64)
        mult[:6] = [2 ** 31 - 1, -2 ** 31, 0, 1, -1, 2 ** 30]
        mult = mult.astype(np.int32)
        shift = rng.integers(1, 32, N).astype(np.int32)
        shift[:4] = [1, 31, 1, 31]
        cs = w.astype(np.int64).sum(1)
        room = 2 ** 31 - 1 - K * K_BOUND           # |bias_eff| must stay below this
        for over in (False, True):
            be = rng.integers(-room + 1, room, N).astype(np.int64)
            if over:
                be[N // 2] = room + 1               # one channel past the bound: the general epilogue
            bias = (be + zx * cs).astype(np.int64)
            bias = ((bias + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int32)   # bias_eff = bias - zx cs, wrapping
            Wq = H.Q8Weights(w, bias, mult, shift, zx, zy, lo, hi)
            dx = H.DeviceArray.from_host(x)
            dout = H.DeviceArray.zeros((B, N * M), np.int8)
            say("requant short epilogue", N, K, M, B, zy, lo, hi, "over" if over else "")
            H.check(H.lib().bnh_gemm_s8_requant(Wq.h, dx.ptr, K * M, M, B, dout.ptr, N * M, None), "requant")
            H.sync()
            got = dout.numpy()
            for b in range(B):
                ref = O.gemm_s8_requant(w, x[b], bias, mult, shift, zx, zy, lo, hi)
                assert np.array_equal(got[b].reshape(N, M), ref), (N, K, M, zy, lo, hi, over, b,
                                                                   np.argwhere(got[b].reshape(N, M) != ref)[:4])


def test_requant_arithmetic_edges(hip):
    """The device's closed-form Q31 requantisation against the oracle's
    textbook SaturatingRoundingDoublingHighMul + RoundingDivideByPOT on the
    extremes (INT32_MIN x INT32_MIN saturation, INT32_MAX products), exact
    rounding ties at every shift, negative multipliers and random values."""
    H = hip
    L = O.lib()
    rng = np.random.default_rng(99)
    I32 = np.iinfo(np.int32)
    edge = np.array([I32.min, I32.min + 1, -1, 0, 1, I32.max - 1, I32.max, 1 << 30, -(1 << 30)], np.int64)
    acc, mult, shift = [], [], []
    for a in edge:
        for m in edge:
            for s in (0, 1, 5, 30, 31):
                acc.append(a), mult.append(m), shift.append(s)
    # ties of RoundingDivideByPOT: x = (2q + 1) 2^(s-1) exactly, through mult = 2^30 (SRDHM(a, 2^30) = a / 2 rounded)
    for s in range(1, 32):
        for q in (-3, -2, -1, 0, 1, 2):
            x = (2 * q + 1) * (1 << (s - 1))
            if I32.min <= 2 * x <= I32.max:
                acc.append(2 * x), mult.append(1 << 30), shift.append(s)
    n = 200000
    acc += list(rng.integers(I32.min, I32.max, n, endpoint=True))
    mult += list(rng.integers(I32.min, I32.max, n, endpoint=True))
    shift += list(rng.integers(0, 32, n))
    acc, mult, shift = (np.array(v, np.int32) for v in (acc, mult, shift))
    for zy, lo, hi in ((0, -128, 127), (-128, -128, 127), (5, -100, 90)):
        da, dm, ds = H.DeviceArray.from_host(acc), H.DeviceArray.from_host(mult), H.DeviceArray.from_host(shift)
        dy = H.DeviceArray.zeros(acc.size, np.int32)
        H.check(H.lib().bnh_eval_requant(da.ptr, dm.ptr, ds.ptr, zy, lo, hi, dy.ptr, acc.size, None), "requant")
        H.sync()
        got = dy.numpy()
        want = np.array([L.orc_requant(int(a), int(m), int(s), zy, lo, hi) for a, m, s in zip(acc, mult, shift)],
                        np.int32)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, [(int(acc[i]), int(mult[i]), int(shift[i]), int(got[i]), int(want[i])) for i in bad[:5]]
