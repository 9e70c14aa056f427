"""The CPU oracle against the reference's own outputs (tests/golden/*.npz,
written by tests/golden/make_goldens.py from the mlsquare/coset tree) and
against what the mathematics fixes.  No GPU."""
import itertools

import numpy as np
import pytest

from oracle import oracle as O

G = np.array([[2, 0, 0, 0, 0, 0, 0, 0], [-1, 1, 0, 0, 0, 0, 0, 0], [0, -1, 1, 0, 0, 0, 0, 0],
              [0, 0, -1, 1, 0, 0, 0, 0], [0, 0, 0, -1, 1, 0, 0, 0], [0, 0, 0, 0, -1, 1, 0, 0],
              [0, 0, 0, 0, 0, -1, 1, 0], [0.5] * 8], dtype=np.float64).T

CODEC_CASES = [("q4M2_b1", 4, 2, 1.0), ("q4M2_b025", 4, 2, 0.25), ("q4M2_b03", 4, 2, 0.3),
               ("q4M2_b002", 4, 2, 0.02), ("q16M3_b1", 16, 3, 1.0), ("q3M2_b1", 3, 2, 1.0),
               ("q8M2_b05", 8, 2, 0.5), ("q2M4_b1", 2, 4, 1.0)]


def test_projection_matches_reference(golden):
    P = golden("projection")
    np.testing.assert_array_equal(O.projection(P["x"]), P["projection"])


def test_custom_round_and_g_x_match_reference(golden):
    P = golden("projection")
    np.testing.assert_array_equal(O.custom_round(P["x"][:2000]), P["custom_round"][:2000])
    np.testing.assert_array_equal(O.g_x(P["x"][:2000]), P["g_x"][:2000])


def test_legacy_q_matches_reference(golden):
    P = golden("projection")
    np.testing.assert_array_equal(O.projection(P["legacy_x"], legacy=True), P["legacy_q"])


def test_custom_round_special_cases():
    # tests/legacy/test_lattices.py:113-123: exact +-0.5 round toward zero
    assert list(O.custom_round(np.array([0.5, -0.5, 1.5, -1.5], np.float32))) == [0, 0, 1, -1]
    # for |x| >= 2 the 2^-23 nudge is absorbed: ties go half-up
    assert list(O.custom_round(np.array([2.5, -2.5, 3.5, -3.5], np.float32))) == [3, -2, 4, -3]


@pytest.mark.parametrize("q", [2, 3, 4])
def test_exhaustive_residual_table(golden, q):
    R = golden("residual_tables")
    b = O.unpack_words(np.arange(q ** 8), q).reshape(-1, 1, 8)
    r = O.e8_decode(b, q, 1)
    np.testing.assert_array_equal(np.rint(2 * r).astype(np.int8), R[f"two_r_q{q}"])


def test_q16_residual_sample(golden):
    R = golden("residual_tables")
    r = O.e8_decode(R["b_q16"].astype(np.int32).reshape(-1, 1, 8), 16, 1)
    np.testing.assert_array_equal(r, R["r_q16"])


@pytest.mark.parametrize("name,q,M,beta", CODEC_CASES)
def test_codec_matches_reference(golden, name, q, M, beta):
    C = golden("codec")
    x = C[name + "_x"]
    codes = O.e8_encode(x, q, M, beta)
    np.testing.assert_array_equal(codes, C[name + "_codes"].astype(np.int32))
    dec = O.e8_decode(C[name + "_codes"].astype(np.int32), q, M, beta)
    np.testing.assert_array_equal(dec, C[name + "_dec"])


def test_quantize_matches_reference(golden):
    C = golden("codec")
    x = C["quantize_x"]
    for q in (4, 16):
        np.testing.assert_array_equal(O.e8_decode(O.e8_encode(x, q, 2), q, 2), C[f"quantize_q{q}"])


def test_generator_inverse_is_exact():
    Ginv = np.linalg.inv(G)
    assert np.array_equal(Ginv * 2, np.rint(Ginv * 2))
    z = np.random.default_rng(0).integers(0, 16, size=(64, 8))
    y = z @ G.T
    np.testing.assert_array_equal(O.decode_coords(z.astype(np.int32)), y.astype(np.float32))
    for q in (4, 16):
        zq = z % q
        np.testing.assert_array_equal(O.encode_coords((zq @ G.T).astype(np.float32), q), zq)


def _e8_member(y):
    two = 2 * y
    if not np.array_equal(two, np.rint(two)):
        return False
    allint = np.all(np.rint(y) == y)
    allhalf = np.all(np.rint(y - 0.5) == y - 0.5)
    return (allint or allhalf) and (np.sum(y) % 2 == 0)


def test_projection_invariants():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2000, 8)).astype(np.float32) * 2
    y = O.projection(x)
    assert all(_e8_member(v.astype(np.float64)) for v in y)
    # idempotent on lattice points
    np.testing.assert_array_equal(O.projection(y), y)


def test_projection_brute_force_candidates():
    """The core projection returns the nearer of its two coset candidates,
    and each candidate is the D8 (resp. D8+1/2) point the g_x rule names.
    Brute force over the 17 points {f} U {f +- e_i} confirms the D8 side
    lies among them; the chosen point is never farther than either."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((500, 8)).astype(np.float32)
    y = O.projection(x)
    for xi, yi in zip(x.astype(np.float64), y.astype(np.float64)):
        f = np.floor(xi + 0.5)
        cands = [f] + [f + s * np.eye(8)[i] for i in range(8) for s in (1, -1)]
        d8 = [c for c in cands if np.sum(c) % 2 == 0]
        fh = np.floor(xi) + 0.5
        candsh = [fh] + [fh + s * np.eye(8)[i] for i in range(8) for s in (1, -1)]
        d8h = [c for c in candsh if np.sum(c) % 2 == 0]
        best = min(np.sum((xi - c) ** 2) for c in d8 + d8h)
        dy = np.sum((xi - yi) ** 2)
        assert any(np.array_equal(yi, c) for c in d8 + d8h)
        assert dy >= best - 1e-6


def test_zero_input_gives_zero_codes():
    codes = O.e8_encode(np.zeros((4, 8), np.float32), 4, 2)
    assert not codes.any()
    assert not O.e8_decode(codes, 4, 2).any()


def test_layer_matches_reference(golden):
    L = golden("layer")
    for name in ["c1", "c1nd", "rnd", "clip", "q16"]:
        g = lambda k: L[f"{name}_{k}"]
        Wq, qraw, _ = O.layer_quant(g("W"), g("beta"), int(g("q")), 2, float(g("clip")))
        np.testing.assert_array_equal(Wq, g("Wq"))
        gWq = g("g").T.astype(np.float64) @ g("x").astype(np.float64)
        dW, dbeta, _ = O.layer_backward(gWq, g("W"), qraw, g("beta"), float(g("clip")))
        np.testing.assert_allclose(dW, g("dW"), rtol=1e-4, atol=1e-4 * np.abs(g("dW")).max())
        bmin, bmax = g("beta_min").astype(np.float64), g("beta_max").astype(np.float64)
        s = 1 / (1 + np.exp(-g("theta").astype(np.float64)))
        dth = dbeta * (bmax - bmin) * s * (1 - s)
        np.testing.assert_allclose(dth, g("dtheta"), rtol=1e-4, atol=1e-4 * np.abs(g("dtheta")).max())


def test_c1_defaults_closed_form(golden):
    """Delta0 = 2*0.95*0.5/(q^M-1) and beta(theta=0) = 0.021441 at q4 M2."""
    L = golden("layer")
    assert abs(O.delta0(4, 2) - float(L["c1_Delta0"])) < 1e-15
    bmin, bmax = O.beta_bounds(4, 2, O.delta0(4, 2), 0.1, np.ones(10), np.ones(10))
    beta = O.beta_from_theta(np.zeros(10), bmin, bmax)
    np.testing.assert_allclose(beta, L["c1_beta"], rtol=1e-6)
    assert abs(beta[0] - 0.021441) < 1e-6
    assert not L["c1_Wq"].any()  # every block rounds to the zero point


@pytest.mark.parametrize("q", [3, 4])
def test_legacy_vlut_matches_reference(golden, q):
    V = golden("vlut_legacy")
    for i in range(2):
        v = O.build_one_sided_vlut(V[f"q{q}_a{i}"], q, legacy=True)
        ref = V[f"q{q}_vlut{i}"]
        np.testing.assert_allclose(v, ref, rtol=0, atol=1e-6 * np.abs(ref).max() * 8)


def test_vlut_matmul_equals_decode_then_dot():
    """tests/legacy/test_one_sided_vlut_pytest.py:294-333: the lookup sum
    equals <a, decode(codes)>."""
    rng = np.random.default_rng(3)
    rows, K, q, M = 6, 32, 4, 2
    w = rng.standard_normal((rows * K // 8, 8)).astype(np.float32)
    codes = O.e8_encode(w, q, M)
    dec = O.e8_decode(codes, q, M).reshape(rows, K)
    words = O.pack_words(codes, q).reshape(rows, K // 8, M)
    a = rng.standard_normal((3, K)).astype(np.float32)
    out = O.vlut_matmul(words, np.ones(rows, np.float32), a, q, M)
    np.testing.assert_allclose(out, a.astype(np.float64) @ dec.T.astype(np.float64), rtol=1e-5, atol=1e-5)


def test_pack_roundtrip():
    for q in (2, 3, 4, 16):
        b = np.random.default_rng(q).integers(0, q, size=(50, 3, 8)).astype(np.int32)
        np.testing.assert_array_equal(O.unpack_words(O.pack_words(b, q), q), b)
    # idx(b) = sum_j b_j q^(7-j) (coset/legacy/quant/vlut.py:231-236)
    b = np.array([[[1, 2, 3, 0, 0, 0, 0, 1]]], np.int32)
    assert O.pack_words(b, 4)[0, 0] == 1 * 4 ** 7 + 2 * 4 ** 6 + 3 * 4 ** 5 + 1


LEGACY_CASES = ["q4M2_p", "q3M2_p", "q8M2_a2", "q4M3_np", "q2M4_p", "q4M2_dither"]


def _legacy_case(golden, name):
    z = golden("legacy_functional")
    cfg = z[f"{name}_cfg"]
    q, M, beta, alpha, mi, prot = int(cfg[0]), int(cfg[1]), float(cfg[2]), float(cfg[3]), int(cfg[4]), int(cfg[5])
    d = z[f"{name}_dither"] if f"{name}_dither" in z else None
    return z, q, M, beta, alpha, mi, prot, d


@pytest.mark.parametrize("name", LEGACY_CASES)
def test_oracle_legacy_functional(golden, name):
    """coset/legacy/quant/functional.py encode (overload loop) / decode:
    codes, T, final overload flag and decode bit-exact against the
    reference's own outputs (tests/golden/legacy_functional.npz)."""
    z, q, M, beta, alpha, mi, prot, d = _legacy_case(golden, name)
    codes, T, ov = O.legacy_encode(z[f"{name}_x"], q, M, beta, alpha, mi, prot, d)
    np.testing.assert_array_equal(codes, z[f"{name}_codes"])
    np.testing.assert_array_equal(T, z[f"{name}_T"])
    np.testing.assert_array_equal(ov, z[f"{name}_overload"])
    np.testing.assert_array_equal(O.legacy_decode(codes, T, q, M, beta, alpha, d), z[f"{name}_decoded"])


def test_oracle_legacy_closed_forms():
    """Cases the definition fixes: tiny inputs never overload (T = 0, codes
    of Q(x/beta)); without protection T stays 0; a huge block exhausts the
    loop (T = max_iter, still overloading); the decode scales by 2^(alpha T)."""
    x = np.full((1, 8), 1e-6, np.float32)
    c, T, ov = O.legacy_encode(x, 4, 2, 0.3, 1.0, 10, True)
    assert T[0] == 0 and ov[0] == 0 and not c.any()
    big = np.full((1, 8), 1e6, np.float32)
    c, T, ov = O.legacy_encode(big, 4, 2, 0.3, 1.0, 3, True)
    assert T[0] == 3 and ov[0] == 1
    c0, T0, ov0 = O.legacy_encode(big, 4, 2, 0.3, 1.0, 3, False)
    assert T0[0] == 0 and ov0[0] == 1
    rng = np.random.default_rng(4)
    codes = rng.integers(0, 4, (16, 2, 8)).astype(np.int32)
    d0 = O.legacy_decode(codes, np.zeros(16, np.int32), 4, 2, 0.5, 1.0)
    d3 = O.legacy_decode(codes, np.full(16, 3, np.int32), 4, 2, 0.5, 1.0)
    np.testing.assert_array_equal(d3, d0 * np.float32(8.0))
