"""Pins the fp16 GEMM oracle (oracle/f16gemm.c, restating src/gemm_f16.c):
fp32 -> fp16 conversion against numpy's (IEEE round to nearest even, with
denormals); small-integer operands, where every fp16 operation is exact, against
the integer product; the K-block structure (fp16 within blocks of <= 128 steps,
fp32 across them) against closed forms that a single fp16 chain would get wrong;
the epilogue (bias, LUT SiLU, ReLU, residual, zero-haloed store); random inputs
against a float64 GEMM within the fp16 accumulation error bound."""
import numpy as np
import pytest

import pyoracle as O


def h(a):
    return np.asarray(a, np.float16)


def test_f2h_matches_numpy():
    L = O.lib()
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, 300000, dtype=np.uint64).astype(np.uint32)
    special = np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-9,
                        np.inf, -np.inf, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11], np.float32)
    xs = np.concatenate([bits.view(np.float32), special, rng.standard_normal(100000).astype(np.float32) * 100])
    xs = xs[~np.isnan(xs)]
    got = np.array([L.orc_f2h(float(x)) for x in xs], np.uint16)
    want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_small_integers_are_exact():
    rng = np.random.default_rng(1)
    M, N, K = 13, 20, 96
    A = rng.integers(-3, 4, (M, K)).astype(np.float16)
    W = rng.integers(-3, 4, (N, K)).astype(np.float16)
    b = rng.integers(-20, 21, N).astype(np.float32)
    out = O.gemm_f16(A, W, b)
    want = A.astype(np.int64) @ W.astype(np.int64).T + b.astype(np.int64)
    assert np.array_equal(out[:, :N].astype(np.int64), want)
    assert not out[:, N:].any()   # pad channels store zero


def test_k_blocks_flush_in_fp32():
    # Kp = 256: two blocks of 128. Every product is 16; a block sums to 2048 exactly in fp16. One fp16 chain over all
    # 256 steps would stall at 2048 (2048 + 16 rounds to 2048 in fp16), the blocked sum reaches 4096.
    A = np.full((1, 256), 4.0, np.float16)
    W = np.full((1, 256), 4.0, np.float16)
    out = O.gemm_f16(A, W, np.zeros(1, np.float32))
    assert float(out[0, 0]) == 4096.0
    # one block (Kp = 128): the fp16 bias add rounds; 2048 + 1 -> 2048 (ties to even)
    out = O.gemm_f16(A[:, :128], W[:, :128], np.ones(1, np.float32))
    assert float(out[0, 0]) == 2048.0
    # Kp = 136 -> 2 balanced blocks of 72 and 64 (not 128 + 8): products 32 -> 2304 and 2048, both exact in fp16
    A2 = np.full((1, 136), 8.0, np.float16)
    W2 = np.full((1, 136), 4.0, np.float16)
    assert float(O.gemm_f16(A2, W2, np.zeros(1, np.float32))[0, 0]) == 4352.0


def test_epilogue_forms():
    rng = np.random.default_rng(2)
    M, N, K, ow = 12, 16, 32, 4
    A = h(rng.standard_normal((M, K)))
    W = h(rng.standard_normal((N, K)) * 0.2)
    b = rng.standard_normal(N).astype(np.float32)
    plain = O.gemm_f16(A, W, b)
    L = O.lib()
    silu = O.gemm_f16(A, W, b, act=1)
    want = np.array([L.orc_silu_lut_h(int(v)) for v in plain.reshape(-1).view(np.uint16)], np.uint16)
    assert np.array_equal(silu.reshape(-1).view(np.uint16), want)
    relu = O.gemm_f16(A, W, b, act=2)
    assert np.array_equal(relu, np.maximum(plain, h(0)))
    res = h(rng.standard_normal((M, N)))
    withres = O.gemm_f16(A, W, b, act=1, res=res)
    assert np.array_equal(withres, (silu.astype(np.float32) + res).astype(np.float16))  # one fp16 add
    padded = O.gemm_f16(A, W, b, act=1, ow=ow, opad=1)
    grid = padded.reshape(M // ow + 2, ow + 2, N)
    assert not grid[0].any() and not grid[-1].any() and not grid[:, 0].any() and not grid[:, -1].any()
    assert np.array_equal(grid[1:-1, 1:-1].reshape(M, N), silu)


@pytest.mark.parametrize("K", [64, 200, 1152])
def test_random_within_fp16_accumulation_bound(K):
    rng = np.random.default_rng(K)
    M, N = 16, 24
    Kp = (K + 7) // 8 * 8
    A = h(np.pad(rng.standard_normal((M, K)), ((0, 0), (0, Kp - K))))
    W = h(np.pad(rng.standard_normal((N, K)) / np.sqrt(K), ((0, 0), (0, Kp - K))))
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    out = O.gemm_f16(A, W, b).astype(np.float64)[:, :N]
    exact = A.astype(np.float64) @ W.astype(np.float64).T + b
    mag = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64)).T + np.abs(b)
    n = min(Kp, 128) + 2
    bound = n * 2.0 ** -11 * mag + 2.0 ** -11 * np.abs(exact) + 2.0 ** -24
    assert (np.abs(out - exact) <= bound).all()
