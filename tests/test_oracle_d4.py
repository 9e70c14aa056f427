"""Pins of the oracle's D4 restatement (coset/core/d4/lattice.py:62-146,
coset/core/base.py:134-176, d4/layers.py:46-47 with layers.py:428-463).

The reference has no tests of its core D4 lattice, so the oracle is checked
against what the mathematics fixes:
  * brute force over every D4 point near x (exact distances): with an even
    rounding, or an odd one whose worst coordinate is not the reference's
    quirk case, the projection is the nearest point; in the quirk case
    (x_k < 0 with f_k < x_k: the reference steps -1 where the nearest point
    steps +1) it is f - e_k, strictly farther than the nearest point;
  * g_x changes exactly one coordinate of custom_round(x), by +-1;
  * encode_coords(decode_coords(b)) = b for every b in [0, q)^4, and
    y - decode(encode(y)) lies in q D4 for lattice points y;
  * the layer quantizer fixes D4 points at beta = 1 and respects the clip.
"""
import itertools

import numpy as np
import pytest

from oracle import oracle as orc


def _nearest(x):
    """Nearest even-sum integer point by enumeration, with its squared
    distance and whether the minimum is shared (a tie)."""
    base = np.floor(x).astype(np.int64)
    best, best_d, second = None, np.inf, np.inf
    for off in itertools.product(range(-1, 3), repeat=4):
        p = base + np.array(off)
        if p.sum() % 2:
            continue
        d = float(((x.astype(np.float64) - p) ** 2).sum())
        if d < best_d:
            best, best_d, second = p, d, best_d
        elif d < second:
            second = d
    return best, best_d, second - best_d < 1e-9


def test_projection_against_brute_force():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((6000, 4)) * 2.0).astype(np.float32)
    x[:500] = np.round(x[:500] * 4) / 4          # quarter grid: ties of the rounding and of the argmax
    y = orc.d4_projection(x)
    f = orc.custom_round(x)
    counts = {"even": 0, "odd": 0, "quirk": 0}
    for i in range(x.shape[0]):
        p, d, tie = _nearest(x[i])
        assert int(y[i].sum()) % 2 == 0
        if int(f[i].sum()) % 2 == 0:
            assert np.array_equal(y[i], f[i])
            if not tie:
                assert np.array_equal(y[i], p), (x[i], y[i], p)
                counts["even"] += 1
            continue
        delta = np.abs(x[i].astype(np.float64) - f[i])
        k = int(np.argmax(delta))
        if x[i, k] < 0 and f[i, k] < x[i, k]:
            want = f[i].copy()
            want[k] -= 1
            assert np.array_equal(y[i], want)
            if not tie:
                dy = float(((x[i].astype(np.float64) - y[i]) ** 2).sum())
                assert dy > d
                counts["quirk"] += 1
        elif not tie and np.sum(delta == delta[k]) == 1:
            assert np.array_equal(y[i], p), (x[i], y[i], p)
            counts["odd"] += 1
    assert min(counts.values()) > 300, counts


def test_g_x_moves_one_coordinate():
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((2000, 4)) * 3).astype(np.float32)
    g = orc.d4_g_x(x)
    f = orc.custom_round(x)
    diff = g - f
    assert np.all((diff != 0).sum(axis=1) == 1)
    assert np.all(np.abs(diff).sum(axis=1) == 1)


@pytest.mark.parametrize("q", [2, 3, 4, 5])
def test_encode_decode_coords(q):
    b = np.array(list(itertools.product(range(q), repeat=4)), dtype=np.int32)
    y = orc.d4_decode_coords(b)
    assert np.all(y.sum(axis=1).astype(np.int64) % 2 == 0)      # G b is in D4
    assert np.array_equal(orc.d4_encode_coords(y, q), b)
    rng = np.random.default_rng(q)
    pts = rng.integers(-50, 50, size=(3000, 4))
    pts[:, 3] += pts.sum(axis=1) % 2                             # even sum
    yy = pts.astype(np.float32)
    r = (yy - orc.d4_decode_coords(orc.d4_encode_coords(yy, q))) / q
    assert np.array_equal(r, np.round(r)) and np.all(r.sum(axis=1).astype(np.int64) % 2 == 0)


def test_layer_quant_fixed_points_and_clip():
    rng = np.random.default_rng(9)
    pts = rng.integers(-3, 4, size=(6, 8))
    pts[:, 3] += pts[:, :4].sum(axis=1) % 2
    pts[:, 7] += pts[:, 4:].sum(axis=1) % 2
    W = pts.astype(np.float32)
    assert np.array_equal(orc.d4_layer_quant(W, np.ones(6, np.float32), 2, 100.0), W)
    Wr = (rng.standard_normal((6, 8)) * 2).astype(np.float32)
    Wq = orc.d4_layer_quant(Wr, np.full(6, 0.5, np.float32), 2, 1.0)
    assert np.abs(Wq).max() <= 1.0
    Wq1 = orc.d4_layer_quant(Wr, np.full(12, 0.5, np.float32), 1, 100.0)   # block tiling, same beta
    assert np.array_equal(Wq1, orc.d4_layer_quant(Wr, np.full(6, 0.5, np.float32), 2, 100.0))
