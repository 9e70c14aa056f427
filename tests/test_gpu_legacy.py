"""The paper's hierarchical quantizer with the overload loop
(coset/legacy/quant/functional.py:15-181) on the GPU, through the C ABI:
codes, T, overload flags and decoded values bit-exact against the
reference's own outputs (tests/golden/legacy_functional.npz) and the oracle."""
import warnings

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

CASES = ["q4M2_p", "q3M2_p", "q8M2_a2", "q4M3_np", "q2M4_p", "q4M2_dither"]


def _cfg(golden, name):
    import coset_amd
    z = golden("legacy_functional")
    c = z[f"{name}_cfg"]
    cfg = coset_amd.QuantizationConfig(lattice_type="E8", q=int(c[0]), M=int(c[1]), beta=float(c[2]),
                                       alpha=float(c[3]), max_scaling_iterations=int(c[4]),
                                       disable_overload_protection=not bool(c[5]),
                                       with_dither=f"{name}_dither" in z)
    d = torch.from_numpy(z[f"{name}_dither"]) if f"{name}_dither" in z else None
    return z, cfg, d


@pytest.mark.parametrize("name", CASES)
def test_blocks_match_reference(golden, name):
    from coset_amd import legacy
    z, cfg, d = _cfg(golden, name)
    x = torch.from_numpy(z[f"{name}_x"]).cuda()
    codes, T, ov, dec = legacy.encode_blocks(x, cfg, d, decoded=True)
    np.testing.assert_array_equal(codes.cpu().numpy(), z[f"{name}_codes"].astype(np.float32))
    np.testing.assert_array_equal(T.cpu().numpy(), z[f"{name}_T"])
    np.testing.assert_array_equal(ov.cpu().numpy(), z[f"{name}_overload"].astype(bool))
    np.testing.assert_array_equal(dec.cpu().numpy(), z[f"{name}_decoded"])
    # decode as its own call, from float codes and from packed words
    np.testing.assert_array_equal(legacy.decode_blocks(codes, cfg, T, d).cpu().numpy(), z[f"{name}_decoded"])
    words, T2, ov2 = legacy.encode_blocks(x, cfg, d, packed=True)
    np.testing.assert_array_equal(words.cpu().numpy().astype(np.uint32),
                                  O.pack_words(z[f"{name}_codes"], cfg.q))
    np.testing.assert_array_equal(legacy.decode_blocks(words, cfg, T2, d).cpu().numpy(), z[f"{name}_decoded"])


def test_reference_signatures(golden):
    """encode / decode / quantize on one 8-vector: shapes, host in -> host
    out, T as an int, the unresolved-overload warning, ValueErrors."""
    import coset_amd
    from coset_amd import legacy
    z, cfg, _ = _cfg(golden, "q2M4_p")
    lat = coset_amd.LegacyE8Lattice()
    ov = z["q2M4_p_overload"].astype(bool)
    i_ok, i_ov = int(np.argmin(ov)), int(np.argmax(ov))
    x = torch.from_numpy(z["q2M4_p_x"][i_ok])
    b, T = legacy.encode(x, lat, cfg)
    assert b.shape == (cfg.M, 8) and b.device.type == "cpu" and isinstance(T, int)
    np.testing.assert_array_equal(b.numpy(), z["q2M4_p_codes"][i_ok].astype(np.float32))
    assert T == z["q2M4_p_T"][i_ok]
    np.testing.assert_array_equal(legacy.decode(b, lat, cfg, T).numpy(), z["q2M4_p_decoded"][i_ok])
    np.testing.assert_array_equal(legacy.quantize(x, lat, cfg).numpy(), z["q2M4_p_decoded"][i_ok])
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        legacy.encode(torch.from_numpy(z["q2M4_p_x"][i_ov]), lat, cfg)
    assert any("Overload not resolved" in str(m.message) for m in w)
    with pytest.raises(ValueError):
        legacy.encode(torch.zeros(7), lat, cfg)
    with pytest.raises(ValueError):
        legacy.decode(torch.zeros(cfg.M + 1, 8), lat, cfg)


@pytest.mark.parametrize("q,M,beta,alpha", [(4, 2, 0.3, 1.0), (16, 3, 0.05, 1.0), (3, 2, 0.35, 2.0),
                                            (2, 4, 0.25, 1.0)])
def test_large_batch_vs_oracle(q, M, beta, alpha):
    """Batches with overloads at every T (scales up to 40), fp32 and bf16
    inputs, protection on and off, against the oracle."""
    import coset_amd
    from coset_amd import legacy
    rng = np.random.default_rng(q * 10 + M)
    x = np.concatenate([(s * rng.standard_normal((2500, 8))).astype(np.float32) for s in (0.1, 1, 4, 40)])
    for protect in (True, False):
        cfg = coset_amd.QuantizationConfig(lattice_type="E8", q=q, M=M, beta=beta, alpha=alpha,
                                           max_scaling_iterations=12, disable_overload_protection=not protect)
        for dt in (torch.float32, torch.bfloat16):
            xt = torch.from_numpy(x).to(dt)
            xin = xt.float().numpy()
            codes, T, ov, dec = legacy.encode_blocks(xt.cuda(), cfg, decoded=True)
            rc, rT, rov = O.legacy_encode(xin, q, M, beta, alpha, 12, protect)
            np.testing.assert_array_equal(codes.cpu().numpy(), rc.astype(np.float32))
            np.testing.assert_array_equal(T.cpu().numpy(), rT)
            np.testing.assert_array_equal(ov.cpu().numpy(), rov.astype(bool))
            np.testing.assert_array_equal(dec.cpu().numpy(), O.legacy_decode(rc, rT, q, M, beta, alpha))
