"""The C-ABI library loads and exports every entry point include/coset_amd.h
declares (no compute: runs without a GPU)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "coset_amd.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(coset_\w+)\s*\(", src, re.M)))


def test_header_declares_entry_points():
    names = declared()
    for must in ("coset_e8_hnlq_encode", "coset_e8_hnlq_decode", "coset_e8_hnlq_roundtrip",
                 "coset_e8_qat_fwd", "coset_e8_qat_bwd", "coset_vlut_matmul", "coset_vlut_build_one_sided"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from coset_amd import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    lib.coset_abi_version.restype = ctypes.c_int
    assert lib.coset_abi_version() == _lib.ABI_VERSION
    lib.coset_word_bytes.argtypes = [ctypes.c_int]
    assert lib.coset_word_bytes(4) == 2 and lib.coset_word_bytes(16) == 4


def test_python_signatures_cover_the_header():
    from coset_amd import _lib
    bound = set(_lib.SIGNATURES) | set(_lib.SIZE_QUERIES) | {"coset_abi_version", "coset_last_error",
                                                             "coset_word_bytes"}
    assert set(declared()) <= bound


def test_host_side_validation_without_gpu():
    """Argument checks run before any HIP call."""
    from coset_amd import _lib
    lib = _lib.load()
    rc = lib.coset_e8_hnlq_roundtrip(None, 0, 4, 0, 1.0, None, 0, 0.0, None, 0, 17, 2, 0, None, None, None, 0,
                                     None)
    assert rc == _lib.EINVAL and b"q=17" in lib.coset_last_error()
    rc = lib.coset_vlut_matmul(None, 0, None, 0, None, 0, 1, 1, 8, 3, 2, 0, 0, None, 0, None, None)
    assert rc == _lib.EUNSUPPORTED


def test_api_names_match_reference():
    import coset_amd
    for name in ("e8_encode", "e8_decode", "e8_quantize", "E8Lattice", "LatticeConfig", "HNLQLinear",
                 "HNLQLinearQAT", "create_e8_hnlq_linear", "ste_quantize", "get_generators", "LSQActivation",
                 "vLUTManager", "_encoding_to_index", "vlut_mac_operation", "QuantizationConfig"):
        assert hasattr(coset_amd, name), name


def test_layer_constructs_on_cpu_host():
    """Construction and bounds are host logic (no kernel): beta(theta=0) at
    the C1 defaults is 0.021441 (coset/core/layers.py:381-422)."""
    import coset_amd
    layer = coset_amd.create_e8_hnlq_linear(768, 10, device="cpu")
    assert abs(layer.Delta0 - 2 * 0.95 * 0.5 / 15) < 1e-15
    assert float(layer.gamma_inv) == 12.0
    beta = layer._beta().detach()
    assert abs(float(beta[0]) - 0.021441) < 1e-6
    cfg = coset_amd.LatticeConfig(lattice_type="E8", q=0, M=2)   # accepted, like the reference
    assert cfg.q == 0
