"""The oracle's statistics update, LSQ quantizer, D4 functions and the CPU
one-sided vLUT routine against the reference's own outputs
(tests/golden/layer_stats.npz, lsq.npz, d4.npz, vlut_legacy.npz), plus
checks that make a plausible slip fail (a biased variance, the clamp
counted in dalpha, a dropped level)."""
import numpy as np
import pytest

from oracle import oracle as O


def test_stats_update_matches_reference(golden):
    S = golden("layer_stats")
    for name in ("row", "c1"):
        se, xe = O.gather_stats(S[f"{name}_W"], S[f"{name}_sigma_ema_255"], S[f"{name}_xmax_ema_255"])
        np.testing.assert_array_equal(se, S[f"{name}_sigma_ema"])
        np.testing.assert_array_equal(xe, S[f"{name}_xmax_ema"])
    W = S["block_W"].reshape(-1, 8)
    se, xe = O.gather_stats(W, np.ones(32, np.float32), np.ones(32, np.float32))
    np.testing.assert_array_equal(se, S["block_sigma_ema_1"])
    np.testing.assert_array_equal(xe, S["block_xmax_ema_1"])
    se, xe = O.gather_stats(W, se, xe)
    np.testing.assert_array_equal(se, S["block_sigma_ema_2"])
    np.testing.assert_array_equal(xe, S["block_xmax_ema_2"])
    # a biased (population) variance would move the result
    Wr = S["row_W"].astype(np.float64)
    biased = (Wr.std(axis=1) + 1e-8).astype(np.float32)
    s_b = (S["row_sigma_ema_255"] * np.float32(0.99)).astype(np.float32) + (np.float32(0.01) * biased)
    assert not np.array_equal(s_b.astype(np.float32), S["row_sigma_ema"])


def test_layer_step_256_uses_updated_stats(golden):
    """The reference's step-256 beta comes from the updated statistics
    (the update runs before the bounds): the oracle's bounds from the golden
    EMA buffers reproduce it."""
    S = golden("layer_stats")
    for name in ("row", "c1"):
        bmin, bmax = O.beta_bounds(int(S[f"{name}_q"]), int(S[f"{name}_M"]), float(S[f"{name}_Delta0"]), 0.1,
                                   S[f"{name}_sigma_ema"], S[f"{name}_xmax_ema"])
        np.testing.assert_allclose(bmin, S[f"{name}_beta_min"], rtol=1e-6)
        np.testing.assert_allclose(bmax, S[f"{name}_beta_max"], rtol=1e-6)
        b_old, _ = O.beta_bounds(int(S[f"{name}_q"]), int(S[f"{name}_M"]), float(S[f"{name}_Delta0"]), 0.1,
                                 S[f"{name}_sigma_ema_255"], S[f"{name}_xmax_ema_255"])
        assert not np.allclose(b_old, S[f"{name}_beta_min"], rtol=1e-6)
        Wq, _, _ = O.layer_quant(S[f"{name}_W"], S[f"{name}_beta"], int(S[f"{name}_q"]), 2, float(S[f"{name}_clip"]))
        np.testing.assert_array_equal(Wq, S[f"{name}_Wq"])


LSQ = ["b8_a1", "b8_a03", "b4_a2", "b8_neg", "b2_a1"]


@pytest.mark.parametrize("name", LSQ)
def test_lsq_matches_reference(golden, name):
    L = golden("lsq")
    x, g = L[f"{name}_x"], L[f"{name}_g"]
    alpha, qmax = float(L[f"{name}_alpha"][0]), 2 ** (int(L[f"{name}_bits"]) - 1) - 1
    y = O.lsq_forward(x, alpha, qmax)
    assert np.array_equal(y.view(np.int32), L[f"{name}_y"].view(np.int32))
    dx, da, mag = O.lsq_backward(x, g, alpha, qmax)
    assert np.array_equal(dx.view(np.int32), L[f"{name}_dx"].view(np.int32))
    assert abs(da - float(L[f"{name}_dalpha"][0])) <= 1e-6 * mag
    # counting the clamp's bound in dalpha (it is detached) breaks the match
    if alpha > 0:
        a = np.float32(alpha + 1e-8)
        clip_term = float((g.astype(np.float64) * np.sign(x) * (np.abs(x) > a)).sum())
        if abs(clip_term) > 1e-6 * mag:
            assert abs(da + clip_term - float(L[f"{name}_dalpha"][0])) > 1e-6 * mag


def test_d4_matches_reference(golden):
    D = golden("d4")
    x = D["x"]
    assert np.array_equal(O.d4_projection(x).view(np.int32), D["projection"].view(np.int32))
    assert np.array_equal(O.d4_g_x(x), D["g_x"])
    for name in ("d4def", "d4nd", "d4clip"):
        W = D[f"{name}_W"]
        Wq = O.d4_layer_quant(W, D[f"{name}_beta"], W.shape[1] // 4, float(D[f"{name}_clip"]))
        np.testing.assert_array_equal(Wq, D[f"{name}_Wq"])
    # the clip is active in one case, the projection non-trivial in another
    assert np.abs(D["d4clip_Wq"]).max() == np.float32(D["d4clip_clip"])
    assert (D["d4nd_Wq"] != 0).mean() > 0.5


def test_onesided_rows_match_lookup_and_golden(golden):
    """The CPU-baseline routine: its tables equal the reference's one-sided
    vLUT where the rules agree (legacy golden at q = 4 uses the textbook Q:
    compare on the core rule's own table instead), and its row sums equal
    the decode-then-dot oracle."""
    rng = np.random.default_rng(3)
    R = O.residual_table(4, legacy=True, strided=False)
    V = golden("vlut_legacy")
    a = V["q4_a0"]
    table = (R.astype(np.float64) @ a.astype(np.float64))
    np.testing.assert_allclose(table, V["q4_vlut0"], rtol=0, atol=1e-5 * np.abs(a).sum() * 12)
    Rc = O.residual_table(4, legacy=False, strided=True)
    words = rng.integers(0, 4 ** 8, size=(64, 16, 2)).astype(np.uint32)
    act = rng.standard_normal((2, 128)).astype(np.float32)
    ref = O.vlut_matmul(words, np.ones(64, np.float32), act, 4, 2)
    for t in range(2):
        acc = O.vlut_onesided_rows(words, Rc, act[t], 4)
        np.testing.assert_allclose(acc, ref[t], rtol=1e-5, atol=1e-4)
        part = O.vlut_onesided_rows(words, Rc, act[t], 4, 0, 8) + O.vlut_onesided_rows(words, Rc, act[t], 4, 8, 16)
        np.testing.assert_allclose(part, acc, rtol=1e-12, atol=1e-9)
    # a dropped level (M = 1 view of the same words) does not match
    one = O.vlut_onesided_rows(np.ascontiguousarray(words[:, :, :1]), Rc, act[0], 4)
    assert not np.allclose(one, ref[0], rtol=1e-5, atol=1e-4)
