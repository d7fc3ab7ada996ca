"""GPU parity of the fp16 pointwise GEMM (libbnneon's gemm_f16 / PW f16 op).

bnh_gemm_f16 computes in the reference's own arithmetic (fp16 FMA chains over
its K blocks, fp32 sums across blocks, its bias and epilogue): bit-identical to
the oracle (oracle/f16gemm.c) on random data, overflow to infinity, NaN inputs,
every epilogue form, one and several K blocks, the 8-channel tail panel and the
package's own fp16 bias.

bnh_gemm_f16_mfma accumulates on fp16 MFMA in fp32 instead. Stated tolerance,
per output before the activation: |gpu - oracle| <= (n + 2) 2^-11 S +
2^-10 |oracle| + 2^-24, n = the reference's K-block length, S = sum_k |a_k w_k|
+ |b| (the recursive-summation bound of the reference's fp16 chain plus one
rounding of each result); with small-integer operands every operation of both
is exact and the outputs are bit-identical.
"""
import numpy as np
import pytest

import pyoracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def hpack(W, Kp):
    """hp_pack's panel layout (src/gemm_f16.c:18-40) of fp16 weights W [N][K]."""
    N, K = W.shape
    Np = (N + 7) // 8 * 8
    n16 = Np // 16
    out = np.zeros(Np * Kp, np.float16)
    for o in range(N):
        nb, j = o // 16, o % 16
        idx = (nb * Kp + np.arange(K)) * 16 + j if nb < n16 else n16 * Kp * 16 + np.arange(K) * 8 + j
        out[idx] = W[o, :K]
    return out


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    an, bn = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(an, bn) and np.array_equal(a.view(np.uint16)[~an], b.view(np.uint16)[~bn]))


def run_gpu(hip, A, W, b32, act=0, ow=0, opad=0, res=None, Kp=None, b16=None, fn="bnh_gemm_f16", ldo=None,
            o_slack=32, gh=None):
    """A [B][M][lda] fp16 -> out [B][rows][ldo] fp16 through fn (bnh_gemm_f16 or bnh_gemm_f16_mfma; with
    fn = bnh_gemm_f16_ws and gates gh [B][Kp] fp16, bnh_gemm_f16_gated_ws)."""
    H = hip
    Bw, M, lda = A.shape
    N, K = W.shape
    Kp = Kp or (K + 7) // 8 * 8
    Np = (N + 7) // 8 * 8
    Wp = np.zeros((N, Kp), np.float16)
    Wp[:, :K] = W
    bpad = np.zeros(Np + 16, np.float32)
    bpad[:N] = b32
    b16p = None
    if b16 is not None:
        b16p = np.zeros(Np + 16, np.float16)
        b16p[:N] = b16
    hp = hpack(Wp, Kp)   # kept alive across the call (a temporary's buffer could be freed before it runs)
    hw = H.lib().bnh_h16w_new(N, K, Kp, Np, hp.ctypes.data, bpad.ctypes.data,
                              None if b16p is None else b16p.ctypes.data)
    if not hw:
        H.check(None, "bnh_h16w_new")
    try:
        rows = M if not opad else (M // ow + 2 * opad) * (ow + 2 * opad)
        ldo = ldo or Np
        a_ws = M * lda + 64
        ah = np.zeros((Bw, a_ws), np.float16)
        ah[:, :M * lda] = A.reshape(Bw, -1)
        o_ws = rows * ldo + o_slack
        dA = H.DeviceArray.from_host(ah)
        dO = H.DeviceArray.from_host(np.full((Bw, o_ws), np.float16(7.0)))   # garbage that the halo zeroing clears
        dR = None
        r_ws = 0
        if res is not None:
            ldr = res.shape[2]
            r_ws = M * ldr
            dR = H.DeviceArray.from_host(res.reshape(Bw, -1))
        e = H.Epi16(act, dO.ptr, o_ws, ldo, ow, opad, dR.ptr if dR else None, r_ws, res.shape[2] if res is not None else 0)
        if fn == "bnh_gemm_f16_ws":   # the split form (no halo zeroing: the output starts at zero here)
            wsb = H.lib().bnh_gemm_f16_ws_bytes(M, Bw, hw)
            dW = H.DeviceArray.zeros(max(int(wsb), 16), np.uint8)
            dO = H.DeviceArray.zeros((Bw, o_ws), np.float16)
            e = H.Epi16(act, dO.ptr, o_ws, ldo, ow, opad, dR.ptr if dR else None, r_ws,
                        res.shape[2] if res is not None else 0)
            if gh is None:
                H.check(H.lib().bnh_gemm_f16_ws(dA.ptr, a_ws, lda, M, Bw, hw, e, dW.ptr, wsb, None), fn)
            else:
                dG = H.DeviceArray.from_host(np.ascontiguousarray(gh, np.float16))
                H.check(H.lib().bnh_gemm_f16_gated_ws(dA.ptr, a_ws, lda, M, Bw, hw, e, dG.ptr, gh.shape[1], dW.ptr,
                                                      wsb, None), "bnh_gemm_f16_gated_ws")
            H.sync()
            return dO.numpy()[:, :rows * ldo].reshape(Bw, rows, ldo), Wp
        if fn == "bnh_gemm_f16_mfma_gated":
            dG = H.DeviceArray.from_host(np.ascontiguousarray(gh, np.float16))
            H.check(H.lib().bnh_gemm_f16_mfma_gated(dA.ptr, a_ws, lda, M, Bw, hw, e, dG.ptr, gh.shape[1], None), fn)
        else:
            H.check(getattr(H.lib(), fn)(dA.ptr, a_ws, lda, M, Bw, hw, e, None), fn)
        H.sync()
        out = dO.numpy()
        assert (out[:, rows * ldo:] == 7.0).all()   # nothing past each window's output
        return out[:, :rows * ldo].reshape(Bw, rows, ldo), Wp
    finally:
        H.lib().bnh_h16w_free(hw)


@pytest.mark.parametrize("act", [0, 1, 2])
def test_small_integers_bit_exact(hip, act):
    rng = np.random.default_rng(act)
    B, M, N, K = 3, 40, 24, 136      # K 136 -> Kp 136: two reference K blocks (72 + 64)
    A = rng.integers(-3, 4, (B, M, K)).astype(np.float16)
    W = rng.integers(-2, 3, (N, K)).astype(np.float16)
    b = rng.integers(-9, 10, N).astype(np.float32)
    res = rng.integers(-4, 5, (B, M, 24)).astype(np.float16)
    for fn in ("bnh_gemm_f16", "bnh_gemm_f16_mfma"):
        say("f16 gemm ints act", act, fn)
        out, Wp = run_gpu(hip, A, W, b, act=act, res=res, fn=fn)
        for i in range(B):
            ref = O.gemm_f16(A[i], Wp, b, act=act, res=res[i])
            assert np.array_equal(out[i].view(np.uint16), ref.view(np.uint16)), (fn, i)


# (K, N, M, B): one K block (K <= 128), two (136: 72 + 64), three (300 -> 104 + 104 + 92), the v2.4 expansion
# and projection shapes (36 -> 288 etc.), N with an 8-channel tail panel, M not a multiple of 64
@pytest.mark.parametrize("K,N,M,B", [(64, 48, 100, 2), (200, 136, 64, 2), (1152, 256, 70, 2), (24, 8, 7, 3),
                                     (300, 200, 129, 2), (36, 288, 64 * 24, 2), (864, 108, 383, 2), (128, 1024, 96, 2)])
@pytest.mark.parametrize("act", [0, 1])
def test_random_bit_exact(hip, K, N, M, B, act):
    rng = np.random.default_rng(K + N + act)
    Kp = (K + 7) // 8 * 8
    A = np.zeros((B, M, Kp), np.float16)
    A[:, :, :K] = rng.standard_normal((B, M, K))
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    Np = (N + 7) // 8 * 8
    res = rng.standard_normal((B, M, Np)).astype(np.float16) if act == 0 else None
    say("f16 gemm random", K, N, M, B, act)
    out, Wp = run_gpu(hip, A, W, b, act=act, res=res)
    for i in range(B):
        ref = O.gemm_f16(A[i], Wp, b, act=act, res=None if res is None else res[i])
        assert same_bits(out[i], ref), i


@pytest.mark.parametrize("K,N,ldo,slack", [(72, 36, 44, 3), (300, 200, 204, 32), (40, 72, 76, 1)])
def test_unaligned_output_strides(hip, K, N, ldo, slack):
    """Output rows and window strides that are not multiples of 8 halves: the element-wise store path."""
    rng = np.random.default_rng(K + ldo)
    B, M = 3, 77
    A = rng.standard_normal((B, M, (K + 7) // 8 * 8)).astype(np.float16)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    res = rng.standard_normal((B, M, ldo)).astype(np.float16)
    say("f16 gemm unaligned", K, N, ldo, slack)
    out, Wp = run_gpu(hip, A, W, b, act=1, res=res, ldo=ldo, o_slack=slack)
    for i in range(B):
        ref = O.gemm_f16(A[i], Wp, b, act=1, ldo=ldo, res=res[i])
        Np = (N + 7) // 8 * 8
        assert same_bits(out[i][:, :Np], ref[:, :Np]), i
        assert (out[i][:, Np:] == 7.0).all()


@pytest.mark.parametrize("K", [96, 264])
def test_package_fp16_bias_overflow_and_nan(hip, K):
    """The package's own fp16 bias (used alone by a single K block, the fp32 one by several), fp16 overflow to
    +-inf inside a chain, a NaN operand."""
    rng = np.random.default_rng(K)
    B, M, N = 2, 72, 40
    A = rng.standard_normal((B, M, K)).astype(np.float16)
    A[0, 3, :] = 200.0           # 200 * 100 * K overflows the fp16 chain
    A[1, 5, 7] = np.nan
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float16)
    W[2, :] = 100.0
    W[3, :] = -100.0
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    b16 = (b * 3 + 0.25).astype(np.float16)   # deliberately not b32 rounded
    say("f16 gemm bias/overflow", K)
    out, Wp = run_gpu(hip, A, W, b, act=2, b16=b16)
    for i in range(B):
        ref = O.gemm_f16(A[i], Wp, b, act=2, b16=np.pad(b16, (0, 8)))
        assert same_bits(out[i], ref), i
    assert np.isinf(out[0, 3, 2]) and np.isnan(out[1, 5]).any()


@pytest.mark.parametrize("K,N,M", [(64, 48, 100), (200, 136, 64), (1152, 256, 256), (24, 8, 7)])
def test_mfma_within_stated_tolerance(hip, K, N, M):
    rng = np.random.default_rng(K + N)
    B = 2
    Kp = (K + 7) // 8 * 8
    A = np.zeros((B, M, Kp), np.float16)
    A[:, :, :K] = rng.standard_normal((B, M, K))
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    say("f16 gemm mfma random", K, N, M)
    out, Wp = run_gpu(hip, A, W, b, fn="bnh_gemm_f16_mfma")
    nblk = (Kp + 127) // 128
    n = ((Kp + nblk - 1) // nblk + 7) // 8 * 8
    for i in range(B):
        ref = O.gemm_f16(A[i], Wp, b).astype(np.float64)
        g = out[i].astype(np.float64)
        S = np.abs(A[i].astype(np.float64)) @ np.abs(Wp.astype(np.float64)).T + np.abs(np.pad(b, (0, Wp.shape[0] - N)))
        Np = (N + 7) // 8 * 8
        S = np.pad(S, ((0, 0), (0, Np - S.shape[1])))
        tol = (n + 2) * 2.0 ** -11 * S + 2.0 ** -10 * np.abs(ref) + 2.0 ** -24
        assert (np.abs(g - ref) <= tol).all(), np.max(np.abs(g - ref) / tol)
        # and closer to the exact product than the reference's fp16 chain is allowed to be
        exact = A[i].astype(np.float64) @ Wp.astype(np.float64).T + np.pad(b, (0, Np - N))
        assert (np.abs(g - exact) <= 2.0 ** -10 * np.abs(exact) + 2.0 ** -24 + Kp * 2.0 ** -24 * S).all()


@pytest.mark.parametrize("fn", ["bnh_gemm_f16", "bnh_gemm_f16_mfma"])
def test_padded_output_and_silu(hip, fn):
    rng = np.random.default_rng(5)
    B, M, N, K, ow = 2, 48, 32, 64, 8
    A = rng.integers(-2, 3, (B, M, K)).astype(np.float16)
    W = rng.integers(-2, 3, (N, K)).astype(np.float16)
    b = rng.integers(-3, 4, N).astype(np.float32)
    say("f16 gemm padded", fn)
    out, Wp = run_gpu(hip, A, W, b, act=1, ow=ow, opad=2, fn=fn)
    for i in range(B):
        ref = O.gemm_f16(A[i], Wp, b, act=1, ow=ow, opad=2)
        assert np.array_equal(out[i].view(np.uint16), ref.view(np.uint16))


def test_padded_random_bit_exact(hip):
    rng = np.random.default_rng(6)
    B, ow, oh, N, K = 3, 64, 24, 72, 36
    M = ow * oh
    A = rng.standard_normal((B, M, 40)).astype(np.float16)   # K 36 -> Kp 40 = lda
    W = (rng.standard_normal((N, K)) / 6).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    say("f16 gemm padded random")
    out, Wp = run_gpu(hip, A, W, b, act=1, ow=ow, opad=1)
    for i in range(B):
        assert same_bits(out[i], O.gemm_f16(A[i], Wp, b, act=1, ow=ow, opad=1)), i


def test_bad_params_refused(hip):
    H = hip
    w, b = np.zeros(256, np.float16), np.zeros(32, np.float32)
    assert not H.lib().bnh_h16w_new(10, 16, 16, 10, w.ctypes.data, b.ctypes.data, None)
    assert b"Np = N rounded up to 8" in H.lib().bnh_last_error()


def test_silu_epilogue_every_fp16_input(hip):
    """The GEMM's packed SiLU on every fp16 bit pattern: W picks k = 0, so the pre-activation of row m is the fp16
    value with bits m (-0 becomes +0 through the chain's +0 start), and the outputs must equal the oracle's fp16 LUT
    SiLU (src/silu_lut.h:28-42) bit for bit, NaNs as NaNs; ReLU the same way."""
    M, K, N = 65536, 8, 16
    A = np.zeros((1, M, K), np.float16)
    A[0, :, 0] = np.arange(M, dtype=np.uint32).astype(np.uint16).view(np.float16)
    W = np.zeros((N, K), np.float16)
    W[:, 0] = 1.0
    b = np.zeros(N, np.float32)
    for act in (1, 2):
        say("f16 gemm every input, act", act)
        out, Wp = run_gpu(hip, A, W, b, act=act)
        ref = O.gemm_f16(A[0], Wp, b, act=act)
        assert same_bits(out[0], ref)
        # the NaN patterns stay NaN; the LUT SiLU of +inf is inf - inf = NaN as well (the reference's formula)
        assert np.isnan(out[0][:, 0]).sum() == 2 * 1023 + (act == 1)


# K blocks run as separate blocks and a combining kernel when rows are few (the v2.4 head shapes 1536 -> 192 and
# 864 -> 108 at 24 / 96 pixels per window), with residual, SiLU, a padded output and unaligned rows
@pytest.mark.parametrize("K,N,M,B,act,opad,ldo", [(1536, 192, 24, 8, 0, 0, None), (864, 108, 96, 4, 1, 1, None),
                                                  (300, 200, 33, 3, 2, 0, None), (1536, 192, 24, 5, 1, 0, 196)])
def test_split_k_blocks_bit_exact(hip, K, N, M, B, act, opad, ldo):
    rng = np.random.default_rng(K + N + M)
    Kp = (K + 7) // 8 * 8
    A = np.zeros((B, M, Kp), np.float16)
    A[:, :, :K] = rng.standard_normal((B, M, K))
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    Np = (N + 7) // 8 * 8
    ow = 8 if opad else 0
    res = rng.standard_normal((B, M, ldo or Np)).astype(np.float16) if not opad else None
    say("f16 gemm split", K, N, M, B, act, opad, ldo)
    out, Wp = run_gpu(hip, A, W, b, act=act, ow=ow, opad=opad, res=res, fn="bnh_gemm_f16_ws", ldo=ldo)
    for i in range(B):
        ref = O.gemm_f16(A[i], Wp, b, act=act, ldo=ldo, ow=ow, opad=opad, res=None if res is None else res[i])
        assert same_bits(out[i][:, :Np], ref[:, :Np]), i


# The fp16 SE's gates applied in the A-load (bnh_gemm_f16_gated_ws): the bytes the plain exact GEMM gives on the rows
# scaled in place by the same fp16 products (the fp16 SE, src/rt_ops_f32.c:256-327), per-window gates, the split
# K-block form, residual, padded output; rows holding inf / NaN and gates of 0 and 1; and the oracle on the scaled rows
@pytest.mark.parametrize("K,N,M,B,act,opad", [(72, 288, 96, 3, 1, 1), (288, 72, 96, 3, 0, 0), (1536, 192, 24, 5, 2, 0),
                                              (864, 108, 96, 4, 1, 0)])
def test_gated_rows_bit_exact(hip, K, N, M, B, act, opad):
    rng = np.random.default_rng(K + 7 * N + M)
    A = rng.standard_normal((B, M, K)).astype(np.float16)
    A[0, 0, :3] = [np.inf, -np.inf, np.nan]
    gh = rng.uniform(0, 1, (B, K)).astype(np.float16)
    gh[0, :4] = [0.0, 1.0, 0.5, 0.0]
    scaled = (A.astype(np.float32) * gh[:, None, :].astype(np.float32)).astype(np.float16)  # one rounding each
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    Np = (N + 7) // 8 * 8
    ow = 8 if opad else 0
    res = rng.standard_normal((B, M, Np)).astype(np.float16) if not opad else None
    say("f16 gemm gated", K, N, M, B, act, opad)
    got, Wp = run_gpu(hip, A, W, b, act=act, ow=ow, opad=opad, res=res, fn="bnh_gemm_f16_ws", gh=gh)
    want, _ = run_gpu(hip, scaled, W, b, act=act, ow=ow, opad=opad, res=res, fn="bnh_gemm_f16_ws")
    assert same_bits(got, want)
    ref = O.gemm_f16(scaled[1], Wp, b, act=act, ow=ow, opad=opad, res=None if res is None else res[1])
    assert same_bits(got[1][:, :Np], ref[:, :Np])


@pytest.mark.parametrize("K,N,M,ldo,opad", [(72, 864, 384, None, 1), (136, 40, 100, 44, 0), (48, 24, 64, None, 0)])
def test_mfma_gated_equals_pregated(hip, K, N, M, ldo, opad):
    """the gated MFMA form multiplies each loaded value by its channel's fp16 gate, one rounding, so it equals the
    ungated MFMA form on A * gate rounded to fp16 (numpy), bit for bit: SiLU, residual, halo, the vector epilogue
    (ldo % 8 == 0) and the scalar one (ldo 44)"""
    rng = np.random.default_rng(K + N + M)
    B, ow = 3, 16
    Kp = (K + 7) // 8 * 8
    A = np.zeros((B, M, Kp), np.float16)
    A[:, :, :K] = rng.standard_normal((B, M, K))
    g = np.zeros((B, Kp), np.float16)
    g[:, :K] = rng.uniform(0, 1, (B, K))
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    res = None if opad else rng.standard_normal((B, M, ldo or (N + 7) // 8 * 8)).astype(np.float16)
    say("f16 mfma gated", K, N, M, ldo, opad)
    kw = dict(act=1, res=res, ldo=ldo, ow=ow if opad else 0, opad=opad)
    got, _ = run_gpu(hip, A, W, b, fn="bnh_gemm_f16_mfma_gated", gh=g, **kw)
    pre = (A * g[:, None, :]).astype(np.float16)
    ref, _ = run_gpu(hip, pre, W, b, fn="bnh_gemm_f16_mfma", **kw)
    assert same_bits(got, ref)
