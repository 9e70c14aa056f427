"""coset_amd: MI355X-native E8 hierarchical nested-lattice quantization.

Drop-in for the E8 HNLQ hot path of mlsquare/coset: the reference's public
names (coset/core/__init__.py:10-22, coset/core/e8/__init__.py:7-33) backed by
hand-written gfx950 HIP kernels behind a C ABI (include/coset_amd.h).
"""
from .lattice import D4Lattice, E8Lattice, LatticeConfig, Lattice, LegacyE8Lattice, d4_quantize
from .codecs import (
    DecodingMethod,
    E8Decoder,
    e8_decode,
    e8_encode,
    e8_quantize,
    hnlq_decode,
    hnlq_encode,
    hnlq_roundtrip,
    word_dtype,
)

from .layers import (
    CapturedQATStep,
    E8ThetaWeightQuant,
    E8WeightQuant,
    HNLQConfig,
    HNLQLinear,
    HNLQLinearQAT,
    LSQActivation,
    StraightThroughQuantize,
    create_d4_hnlq_linear,
    create_e8_hnlq_linear,
    D4ThetaWeightQuant,
    get_generators,
    ste_quantize,
)

from .vlut import (
    QuantizationConfig,
    _encoding_to_index,
    build_one_sided_vluts,
    build_vlut,
    vLUTManager,
    vlut_accumulate_operation,
    vlut_dot,
    vlut_mac_operation,
    vlut_matmul,
    vlut_prepare,
    PreparedWords,
)

from . import legacy  # coset.legacy.quant.functional: encode / decode / quantize with the overload loop
from .packed import PackedLinear, load_packed, packed_state, save_packed

__version__ = "0.1.0"

__all__ = [
    "CapturedQATStep",
    "D4Lattice", "E8Lattice", "LatticeConfig", "Lattice", "LegacyE8Lattice", "d4_quantize",
    "e8_encode", "e8_decode", "e8_quantize", "E8Decoder", "DecodingMethod",
    "hnlq_encode", "hnlq_decode", "hnlq_roundtrip", "word_dtype",
    "HNLQLinear", "HNLQLinearQAT", "HNLQConfig", "LSQActivation", "StraightThroughQuantize",
    "E8WeightQuant", "E8ThetaWeightQuant", "D4ThetaWeightQuant", "create_d4_hnlq_linear", "create_e8_hnlq_linear", "get_generators", "ste_quantize",
    "vLUTManager", "QuantizationConfig", "build_vlut", "_encoding_to_index", "vlut_mac_operation",
    "vlut_accumulate_operation", "build_one_sided_vluts", "vlut_dot", "vlut_matmul", "vlut_prepare", "PreparedWords",
    "legacy", "PackedLinear", "load_packed", "packed_state", "save_packed",
]
