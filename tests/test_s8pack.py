"""Known answers of the reference's own tests for int8 packing, applied to
bnneon.s8pack: tests/test_lower_units.py:139-160 (s8_tensors) and
tests/test_lower_s8.py:38-105 (quant_rows_s8, n4_panel_flags)."""
import numpy as np

from bnneon import s8pack


def test_s8_tensors_known_answers():
    w = np.array([[0.5, -1.0, 0.25], [0.0, 0.0, 0.0]], np.float32)
    pk = s8pack.pack_s8(w, np.array([1.0, 2.0], np.float32))
    assert pk["shape"] == (2, 3, 16, 8)
    q = pk["q"]
    assert q.shape == (2, 1, 4, 16)
    # 0.5 * 127 = 63.5 rounds away from zero to 64; 0.25 * 127 = 31.75 -> 32
    assert q[0, 0, 0, :3].tolist() == [64, -127, 32]
    assert not q[0, 0, 1].any()
    assert pk["cs"][:2].tolist() == [64 - 127 + 32, 0]
    assert np.isclose(pk["sw"][0], 1 / 127) and pk["sw"][1] == 1.0
    assert pk["sw"].size == 16 and pk["b"][:3].tolist() == [1.0, 2.0, 0.0]


def test_quant_rows_s8_known_answers():
    q, sw = s8pack.quant_rows_s8(np.array([[0.5, -0.25, 0.1, 0.0]], np.float32))
    assert q.tolist() == [[127, -64, 25, 0]] and abs(float(sw[0]) - 0.5 / 127) < 1e-9
    q, _ = s8pack.quant_rows_s8(np.array([[127.0, 0.5, -0.5, 1.5, -2.5]], np.float32))
    assert q.tolist() == [[127, 1, -1, 2, -3]]
    q, sw = s8pack.quant_rows_s8(np.zeros((2, 8), np.float32))
    assert not q.any() and sw.tolist() == [0.0, 0.0]
    rng = np.random.default_rng(0)
    q, _ = s8pack.quant_rows_s8(-np.abs(rng.standard_normal((16, 64))).astype(np.float32))
    assert int(q.min()) >= -127


def _row_with_lane(values, lane=3):
    row = [0] * 32
    for step, v in enumerate(values):
        row[lane + 8 * step] = v
    return row


def _brute_flags(q):
    out = []
    for first in range(0, q.shape[0], 4):
        worst = 0
        for row in range(first, first + 4):
            for step in range(q.shape[1] // 32):
                for lane in range(8):
                    worst = max(worst, sum(abs(int(q[row, 32 * step + lane + 8 * i])) for i in range(4)))
        out.append(int(worst <= 258))
    return out


def test_n4_panel_flags_known_answers():
    Z = [0] * 32
    assert s8pack.N4_LANE_LIMIT == 258
    assert s8pack.n4_panel_flags(np.array([_row_with_lane([127, -127, 4, 0]), Z, Z, Z], np.int8)).tolist() == [1]
    assert s8pack.n4_panel_flags(np.array([Z, Z, _row_with_lane([127, -127, 4, -1]), Z], np.int8)).tolist() == [0]
    same, other = [0] * 64, [0] * 64
    for p in (3, 11, 19, 27):
        same[p] = 100
    for p in (3, 12, 21, 30, 35):
        other[p] = 100
    z64 = Z * 2
    q = np.array([same, z64, z64, z64, other, z64, z64, z64], np.int8)
    assert s8pack.n4_panel_flags(q).tolist() == [0, 1]
    rng = np.random.default_rng(1)
    q = rng.integers(-20, 21, (8, 64)).astype(np.int8)
    q[5, 7] = q[5, 15] = q[5, 23] = q[5, 31] = 100
    assert s8pack.n4_panel_flags(q).tolist() == [1, 0]
    assert s8pack.n4_panel_flags(np.zeros((8, 48), np.int8)).tolist() == [0, 0]
    rng = np.random.default_rng(2)
    q = rng.integers(-90, 91, (64, 96)).astype(np.int8)
    exp = _brute_flags(q)
    assert s8pack.n4_panel_flags(q).tolist() == exp and 0 in exp
    assert 1 in s8pack.n4_panel_flags((q // 2).astype(np.int8)).tolist()


def test_panels_roundtrip():
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, (24, 48)).astype(np.int8)
    p = s8pack.pack_panels(q)
    assert p.shape == (6, 3, 4, 16)
    assert p[1, 2, 3, 5] == q[4 + 3, 32 + 5]
    assert np.array_equal(s8pack.unpack_panels(p, 24, 48), q)
