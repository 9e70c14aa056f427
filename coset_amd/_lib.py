"""ctypes binding of libcoset_amd.so (C ABI in include/coset_amd.h).

The library is loaded after torch, so it binds to the HIP runtime torch
already mapped (both carry soname libamdhip64.so.7): device pointers and
streams from torch are valid in it.  There is no fallback: if the library is
missing or no GPU is visible, every call raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libcoset_amd.so")
ABI_VERSION = 3

# mirrors of the enums in include/coset_amd.h
OK, EINVAL, EUNSUPPORTED, EHIP = 0, -1, -2, -3
F32, BF16, F16 = 0, 1, 2
SCALE_NONE, SCALE_CODEC, SCALE_LAYER = 0, 1, 2
OP_CUSTOM_ROUND, OP_G_X, OP_PROJECT, OP_ENCODE_COORDS, OP_DECODE_COORDS = range(5)

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float

# name -> argtypes; every entry point returns int
SIGNATURES = {
    "coset_e8_hnlq_encode": [_vp, _int, _i64, _int, _flt, _vp, _i64, _vp, _i64, _int, _int,
                             _vp, _vp, _vp],
    "coset_e8_hnlq_decode": [_vp, _vp, _i64, _int, _flt, _vp, _i64, _flt, _int, _int, _int,
                             _vp, _int, _vp],
    "coset_e8_hnlq_roundtrip": [_vp, _int, _i64, _int, _flt, _vp, _i64, _flt, _vp, _i64,
                                _int, _int, _int, _vp, _vp, _vp, _int, _vp],
    "coset_e8_lattice_op": [_int, _int, _vp, _i64, _int, _vp, _vp],
    "coset_e8_qat_fwd": [_vp, _i64, _i64, _vp, _i64, _flt, _int, _int, _vp, _int, _vp, _vp],
    "coset_e8_qat_bwd": [_vp, _int, _vp, _vp, _vp, _i64, _i64, _i64, _flt, _int, _int, _vp, _vp,
                         _vp],
    "coset_e8_qat_fwd_theta": [_vp, _i64, _i64, _i64, _vp, _vp, _vp, ctypes.c_double, ctypes.c_double,
                               ctypes.c_double, _int, _flt, _int, _int, _vp, _int, _vp, _vp, _vp, _vp, _vp,
                               _vp, _vp],
    "coset_e8_qat_head_fwd": [_vp, _i64, _i64, _vp, _vp, _vp, ctypes.c_double, ctypes.c_double, ctypes.c_double,
                              _int, _flt, _int, _vp, _i64, _vp, _vp, _vp, _vp],
    "coset_e8_qat_bwd_theta": [_vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _flt, _int, _int, _vp, _vp, _vp,
                               _vp],
    "coset_vlut_build_one_sided": [_vp, _i64, _int, _int, _vp, _vp],
    "coset_vlut_lookup_dot": [_vp, _i64, _int, _int, _vp, _vp, _vp],
    "coset_vlut_prepare": [_vp, _i64, _i64, _int, _int, _int, _int, _vp, _vp],
    "coset_vlut_matmul": [_vp, _int, _vp, _int, _vp, _int, _i64, _i64, _i64, _int, _int, _int, _int, _vp, _i64,
                          _vp, _vp],
    "coset_e8_legacy_encode": [_vp, _int, _i64, _flt, ctypes.c_double, _int, _int, _vp, _i64, _int, _int, _vp,
                               _vp, _vp, _vp, _vp, _vp],
    "coset_e8_legacy_decode": [_vp, _vp, _vp, _i64, _flt, ctypes.c_double, _vp, _i64, _int, _int, _vp, _vp],
    "coset_vlut_linear": [_vp, _int, _vp, _int, _vp, _int, _i64, _i64, _i64, _int, _int, _int, _int, _vp, _vp, _int,
                          _vp, _i64, _vp, _vp],
    "coset_d4_lattice_op": [_int, _vp, _i64, _int, _vp, _vp],
    "coset_d4_qat_fwd": [_vp, _i64, _i64, _vp, _i64, _flt, _vp, _int, _vp],
    "coset_d4_qat_fwd_theta": [_vp, _i64, _i64, _i64, _vp, _vp, _vp, ctypes.c_double, ctypes.c_double,
                               ctypes.c_double, _int, _int, _flt, _vp, _int, _vp, _vp, _vp, _vp],
    "coset_d4_qat_bwd": [_vp, _int, _vp, _vp, _vp, _i64, _i64, _i64, _flt, _vp, _vp, _vp, _vp],
    "coset_lsq_fwd": [_vp, _int, _i64, _vp, _int, _vp, _vp],
    "coset_lsq_bwd": [_vp, _vp, _int, _i64, _vp, _int, _vp, _vp, _vp, _i64, _vp],
    "coset_qat_stats_update": [_vp, _i64, _i64, ctypes.c_double, _vp, _vp, _vp],
    "coset_colsum": [_vp, _int, _i64, _i64, _vp, _vp, _i64, _vp],
    "coset_gemm_tn_supported": [_i64, _i64, _i64],
    "coset_gemm_tn": [_vp, _i64, _vp, _i64, _vp, _i64, _int, _i64, _i64, _i64, _vp, _vp, _i64, _vp],
    "coset_vlut_matmul_noalloc": [_vp, _int, _vp, _int, _vp, _int, _i64, _i64, _i64, _int, _int, _int, _int, _vp,
                                  _vp],
    "coset_probe_empty": [_int, _int, _int, _vp, _vp],
    "coset_probe_read": [_vp, _i64, _int, _int, _vp, _vp],
    "coset_probe_c2_stream": [_vp, _i64, _vp, _vp, _int, _vp],
    "coset_probe_valu": [_int, _int, _int, _vp, _vp],
    "coset_init": [_int],
    "coset_set_option": [_int, _int],
}

# name -> argtypes of the int64 size queries
SIZE_QUERIES = {
    "coset_vlut_workspace_floats": [_i64, _i64, _i64, _int, _int, _int, _int],
    "coset_vlut_prepared_words": [_i64, _i64, _int, _int],
    "coset_lsq_workspace_floats": [_i64],
    "coset_colsum_workspace_floats": [_i64, _i64],
    "coset_gemm_tn_workspace_floats": [_i64, _i64, _i64],
    "coset_vlut_noalloc_scratch_floats": [],
}

OPT_CODEC_PATH = 1
OPT_VLUT_DECODE = 2
OPT_VLUT_SPLITS = 3
OPT_FAST_PROJECTION = 4
OPT_CODEC_PLAIN = 5
OPT_CODEC_DYNAMIC = 6
OPT_VLUT_DEEP = 7
OPT_GEMM_TN_TILE = 8
CODEC_AUTO, CODEC_GENERIC, CODEC_LUT = 0, 1, 2

_lib = None


class CosetError(RuntimeError):
    pass


def load():
    """Load the library (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise CosetError(f"{LIB_PATH} is missing: run `python -m coset_amd.build` first")
    lib = ctypes.CDLL(LIB_PATH)
    lib.coset_abi_version.restype = _int
    lib.coset_last_error.restype = ctypes.c_char_p
    lib.coset_word_bytes.argtypes = [_int]
    lib.coset_word_bytes.restype = _int
    for name, args in SIZE_QUERIES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _i64
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _int
    v = lib.coset_abi_version()
    if v != ABI_VERSION:
        raise CosetError(f"libcoset_amd ABI {v}, expected {ABI_VERSION}: rebuild")
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    check(name, getattr(load(), name)(*args))


def word_bytes(q: int) -> int:
    return 2 if q <= 4 else 4


def ptr(t):
    """Device pointer of a tensor (or None)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """torch's current HIP stream on t's device (the raw handle)."""
    return torch._C._cuda_getCurrentRawStream(t.device.index)


def fn(name: str):
    """The bound entry point (for hot paths that call it directly and check
    the return code with check())."""
    return getattr(load(), name)


def check(name: str, rc: int) -> None:
    if rc != OK:
        msg = load().coset_last_error().decode(errors="replace")
        if rc == EINVAL:
            raise ValueError(f"{name}: {msg}")
        raise CosetError(f"{name} failed ({rc}): {msg}")


_inited = set()


def require_gpu() -> torch.device:
    """The current GPU, with the library's per-device tables built."""
    if not torch.cuda.is_available():
        raise CosetError("coset_amd needs a ROCm GPU (gfx950); none is visible")
    load()
    dev = torch.cuda.current_device()
    if dev not in _inited:
        call("coset_init", dev)
        _inited.add(dev)
    return torch.device("cuda", dev)


def set_codec_path(path: int) -> None:
    """0 automatic, 1 generic kernel, 2 LDS-table kernel (q = 2, 4)."""
    call("coset_set_option", OPT_CODEC_PATH, int(path))


def set_fast_projection(enabled: bool) -> None:
    """Encoders try the fast projection first (default) or always run the
    reference operation sequence; results are identical either way."""
    call("coset_set_option", OPT_FAST_PROJECTION, int(bool(enabled)))


def set_codec_plain(enabled: bool) -> None:
    """The fixed-format codec kernels where a call qualifies (default) -- the
    table kernel's variant for fp32 in/out, beta = 2^k, no dither, and the
    layer round-trip kernel for stored or theta-derived per-row betas at
    q = 4, 8, 16 -- or
    always the general ones (bit-identical results)."""
    call("coset_set_option", OPT_CODEC_PLAIN, int(bool(enabled)))


def set_codec_dynamic(enabled: bool) -> None:
    """Fixed-format table kernel: tiles handed out by a per-stream counter
    (default) or a static grid stride."""
    call("coset_set_option", OPT_CODEC_DYNAMIC, int(bool(enabled)))


def set_vlut_decode(byte_tables: bool) -> None:
    """MFMA vLUT decode through byte tables (default) or integer digits."""
    call("coset_set_option", OPT_VLUT_DECODE, int(bool(byte_tables)))


def set_vlut_deep(enabled: bool) -> None:
    """vLUT matmuls above 32 tokens: the deep kernel (default) or the wide one."""
    call("coset_set_option", OPT_VLUT_DEEP, int(bool(enabled)))


def set_gemm_tn_tile(tile: int) -> None:
    """coset_gemm_tn's output tiles: 0 the plan's choice (64 x 64 where they
    fit, else 96 x 96), 64 or 96 only that size."""
    call("coset_set_option", OPT_GEMM_TN_TILE, int(tile))


def set_vlut_splits(splits: int) -> None:
    """0 automatic, n > 0 forces the vLUT matmul's K splits."""
    call("coset_set_option", OPT_VLUT_SPLITS, int(splits))


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float16:
        return F16
    raise ValueError(f"unsupported dtype {dt} (float32 or bfloat16)")
