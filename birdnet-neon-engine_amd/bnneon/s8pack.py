"""Offline int8 weight quantization and packing (what bnc writes into .bnpk).

The same arithmetic as the reference compiler, so that a package from either
tool holds the same bytes:

  * pack_s8 follows s8_tensors (python/bnneon/compiler/lower.py:883-914):
    per output row, in float64, sw = max|w| / 127 (1.0 for an all-zero row),
    q = sign(w / sw) * floor(|w / sw| + 0.5) clipped to [-127, 127], the
    panels [Np/4][Kp/16][4][16], int32 column sums and the fp32 bias, with sw,
    colsum and b zero-padded to Np + 8.
  * quant_rows_s8 follows lower.py:160-177 (the prototype head's weights):
    sw = max|row| / 127 computed in float32, 0 for an all-zero row.
  * n4_panel_flags follows lower.py:180-203 (N4_LANE_LIMIT = 258, :157).
"""
import numpy as np

N4_LANE_LIMIT = 32767 // 127


def r8(n):
    return (n + 7) // 8 * 8


def r16(n):
    return (n + 15) // 16 * 16


def half_away(x):
    """Rounds half away from zero (float64 in, float64 out)."""
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def pack_panels(q):
    """int8 [Np][Kp] rows -> the kernel's panels [Np/4][Kp/16][4][16]."""
    n, k = q.shape
    assert n % 4 == 0 and k % 16 == 0, q.shape
    return np.ascontiguousarray(
        q.reshape(n // 4, 4, k // 16, 16).transpose(0, 2, 1, 3))


def unpack_panels(p, n_pad, k_pad):
    """Inverse of pack_panels: [Np/4][Kp/16][4][16] -> [Np][Kp]."""
    p = np.asarray(p).reshape(n_pad // 4, k_pad // 16, 4, 16)
    return np.ascontiguousarray(p.transpose(0, 2, 1, 3).reshape(n_pad, k_pad))


def pack_s8(w, b):
    """The int8 GEMM tensors of a [N][K] float weight and [N] bias.

    Returns:
        dict with q (panels int8 [Np/4][Kp/16][4][16]), sw (f32 [Np+8]),
        cs (i32 [Np+8]), b (f32 [Np+8]) and shape (N, K, Kp, Np).
    """
    w = np.asarray(w)
    n, k = w.shape
    n_pad, k_pad = r8(n), r16(k)
    wq = np.zeros((n_pad, k_pad), np.float64)
    wq[:n, :k] = w
    am = np.abs(wq).max(1)
    sw = np.where(am > 0, am / 127.0, 1.0)
    q = np.clip(half_away(wq / sw[:, None]), -127, 127).astype(np.int8)
    cs = q.astype(np.int64).sum(1).astype(np.int32)
    swf = np.zeros(n_pad + 8, np.float32)
    swf[:n_pad] = sw
    csp = np.zeros(n_pad + 8, np.int32)
    csp[:n_pad] = cs
    bb = np.zeros(n_pad + 8, np.float32)
    bb[:n] = b
    return {"q": pack_panels(q), "sw": swf, "cs": csp, "b": bb,
            "shape": (n, k, k_pad, n_pad)}


def quant_rows_s8(w):
    """Per-row symmetric int8 of float32 [N][K]: (q int8, sw float32 [N])."""
    w = np.asarray(w, np.float32)
    am = np.abs(w).max(1)
    sw = np.where(am > 0, am / np.float32(127.0), 0.0).astype(np.float32)
    safe = np.where(sw > 0, sw, 1).astype(np.float32)
    # float32 throughout, as the reference's numpy arithmetic on float32 rows
    ratio = np.where(sw[:, None] > 0, w / safe[:, None],
                     np.float32(0)).astype(np.float32)
    r = np.sign(ratio) * np.floor(np.abs(ratio) + np.float32(0.5))
    q = np.clip(r, -127, 127)
    return q.astype(np.int8), sw


def n4_panel_flags(q, lane_limit=N4_LANE_LIMIT):
    """1 per 4-row panel whose every int16 lane of the n=4 K loop stays exact.

    A lane of a 32-byte step takes the weights at bytes l, l + 8, l + 16,
    l + 24 of the step; the panel is safe when every such 4-weight group of its
    4 rows has sum |w| <= lane_limit. All zero when Kp % 32 != 0.
    """
    q = np.asarray(q)
    rows, kp = q.shape
    if kp % 32:
        return np.zeros(rows // 4, np.int8)
    a = np.abs(q.astype(np.int32)).reshape(rows, kp // 32, 4, 8)
    worst = a.sum(2).max(axis=(1, 2))
    return (worst.reshape(rows // 4, 4).max(1) <= lane_limit).astype(np.int8)
