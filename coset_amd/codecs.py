"""E8 HNLQ codecs: the reference signatures plus the packed-code native API.

Reference: coset/core/e8/codecs.py (e8_encode 17-89, E8Decoder 99-180,
e8_decode 185-218, e8_quantize 221-286).  All arithmetic runs in the fused
HIP kernels of libcoset_amd.so; tensors on the host are moved to the GPU for
the call and the result returned on the input's device, like the reference's
"output device follows the input".
"""
from __future__ import annotations

from enum import Enum
from typing import Optional, Tuple

import torch

from . import _lib
from .lattice import E8Lattice, LatticeConfig, on_gpu


def _check_qm(q: int, M: int) -> None:
    if not (2 <= int(q) <= 16):
        raise ValueError(f"q={q} is outside the supported range [2, 16]")
    if not (1 <= int(M) <= 8):
        raise ValueError(f"M={M} is outside the supported range [1, 8]")


def _x_blocks(x: torch.Tensor) -> torch.Tensor:
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    return on_gpu(x).contiguous()


# --------------------------------------------------------------------------
# native packed API
# --------------------------------------------------------------------------

def word_dtype(q: int) -> torch.dtype:
    """Packed level words are uint16 for q <= 4 and uint32 up to q = 16."""
    return torch.uint16 if q <= 4 else torch.uint32


def _scale_args(beta, beta_row, blocks_per_row, n):
    if beta_row is not None:
        br = on_gpu(beta_row).float().contiguous()
        if br.numel() == 0:
            raise ValueError("beta_row is empty")
        if blocks_per_row is None:
            blocks_per_row = n // br.numel()
        if br.numel() * int(blocks_per_row) != n:
            raise ValueError(f"beta_row holds {br.numel()} values for {blocks_per_row} blocks each, "
                             f"but the input has {n} blocks")
        return _lib.SCALE_LAYER, 1.0, br, int(blocks_per_row)
    if beta is None:
        return _lib.SCALE_NONE, 1.0, None, 0
    return _lib.SCALE_CODEC, float(beta), None, 0


def _dither(dither, n):
    """(dither tensor, stride): one [8] vector broadcast (stride 0) or one
    row per block [n, 8] (stride 8); any other length is an error, as the
    reference's broadcast x / beta + dither would raise."""
    if dither is None:
        return None, 0
    d = on_gpu(dither).float().contiguous()
    if d.numel() == 8:
        return d, 0
    if d.numel() == 8 * n:
        return d, 8
    raise ValueError(f"dither must hold 8 or {8 * n} values, got {d.numel()}")


def hnlq_encode(x: torch.Tensor, q: int = 4, M: int = 2, beta: Optional[float] = 1.0, *,
                beta_row: Optional[torch.Tensor] = None, blocks_per_row: Optional[int] = None,
                dither: Optional[torch.Tensor] = None, return_codes: bool = False):
    """Packed level words [N, M] (and optionally float codes [N, M, 8]).

    x: [N, 8] (or [..., 8]) fp32 or bf16 on the GPU.  beta: codec scaling
    x / beta; beta_row: layer scaling x * beta_row[block // blocks_per_row].
    """
    _check_qm(q, M)
    xg = _x_blocks(x)
    n = xg.numel() // 8
    mode, b, brow, bpr = _scale_args(beta, beta_row, blocks_per_row, n)
    packed = torch.empty((n, M), dtype=word_dtype(q), device=xg.device)
    codes = torch.empty((n, M, 8), dtype=torch.float32, device=xg.device) if return_codes else None
    d, ds = _dither(dither, n)
    _lib.call("coset_e8_hnlq_encode", _lib.ptr(xg), _lib.dtype_code(xg.dtype), n, mode, b,
              _lib.ptr(brow), bpr, _lib.ptr(d), ds, int(q), int(M), _lib.ptr(packed),
              _lib.ptr(codes), _lib.stream_of(xg))
    return (packed, codes) if return_codes else packed


def hnlq_decode(packed: torch.Tensor, q: int = 4, M: int = 2, beta: Optional[float] = 1.0, *,
                beta_row: Optional[torch.Tensor] = None, blocks_per_row: Optional[int] = None,
                clip: float = float("inf"), out_dtype: torch.dtype = torch.float32,
                strided: Optional[bool] = None) -> torch.Tensor:
    """Decode packed words [N, M] to [N, 8] (fp32 or bf16)."""
    _check_qm(q, M)
    pk = on_gpu(packed).contiguous()
    if pk.dtype != word_dtype(q):
        raise ValueError(f"packed words for q={q} must be {word_dtype(q)}")
    n = pk.numel() // M
    mode, b, brow, bpr = _scale_args(beta, beta_row, blocks_per_row, n)
    out = torch.empty((n, 8), dtype=out_dtype, device=pk.device)
    st = (n > 1) if strided is None else bool(strided)
    _lib.call("coset_e8_hnlq_decode", _lib.ptr(pk), None, n, mode, b, _lib.ptr(brow), bpr,
              float(clip), int(q), int(M), int(st), _lib.ptr(out), _lib.dtype_code(out_dtype),
              _lib.stream_of(pk))
    return out


def hnlq_roundtrip(x: torch.Tensor, q: int = 4, M: int = 2, beta: Optional[float] = 1.0, *,
                   beta_row: Optional[torch.Tensor] = None, blocks_per_row: Optional[int] = None,
                   clip: float = float("inf"), out_dtype: torch.dtype = torch.float32,
                   want_packed: bool = True, want_decoded: bool = True,
                   packed_out: Optional[torch.Tensor] = None,
                   decoded_out: Optional[torch.Tensor] = None,
                   strided: Optional[bool] = None):
    """Fused encode -> decode in one HBM pass.  Returns (packed, decoded)."""
    _check_qm(q, M)
    xg = _x_blocks(x)
    n = xg.numel() // 8
    mode, b, brow, bpr = _scale_args(beta, beta_row, blocks_per_row, n)
    packed = packed_out
    if packed is None and want_packed:
        packed = torch.empty((n, M), dtype=word_dtype(q), device=xg.device)
    out = decoded_out
    if out is None and want_decoded:
        out = torch.empty((n, 8), dtype=out_dtype, device=xg.device)
    st = (n > 1) if strided is None else bool(strided)
    _lib.call("coset_e8_hnlq_roundtrip", _lib.ptr(xg), _lib.dtype_code(xg.dtype), n, mode, b,
              _lib.ptr(brow), bpr, float(clip), None, 0, int(q), int(M), int(st),
              _lib.ptr(packed), None, _lib.ptr(out),
              _lib.dtype_code(out.dtype) if out is not None else _lib.F32, _lib.stream_of(xg))
    return packed, out


# --------------------------------------------------------------------------
# reference signatures
# --------------------------------------------------------------------------

def e8_encode(x: torch.Tensor, config: LatticeConfig, lattice=None, dither: Optional[torch.Tensor] = None,
              device=None) -> Tuple[torch.Tensor, int]:
    """coset/core/e8/codecs.py:17-89: float codes [N, M, 8] (or [M, 8]) and T=0."""
    squeeze = x.dim() == 1
    if squeeze:
        x = x.unsqueeze(0)
    if x.shape[-1] != 8:
        raise ValueError(f"Input dimension {x.shape[-1]} doesn't match E8 dimension 8")
    home = torch.device(device) if device is not None else x.device
    q, M = int(config.q), int(config.M)
    _check_qm(q, M)
    if not float(config.beta) > 0:
        raise ValueError("beta must be positive")
    d = dither if (config.with_dither and dither is not None) else None
    _, codes = hnlq_encode(x.reshape(-1, 8), q, M, float(config.beta), dither=d, return_codes=True)
    codes = codes.to(home)
    return (codes.squeeze(0) if squeeze else codes), 0


class DecodingMethod(Enum):
    FULL = "full"


class E8Decoder:
    """coset/core/e8/codecs.py:99-180."""

    def __init__(self, device=None):
        self.device = torch.device(device) if device is not None else torch.device("cpu")
        self.lattice = None

    def decode(self, b: torch.Tensor, config: LatticeConfig, method: DecodingMethod = DecodingMethod.FULL):
        if method == DecodingMethod.FULL:
            return self._full_decode(b, config)
        raise ValueError(f"Unknown decoding method: {method}. Only 'full' is currently supported.")

    def _full_decode(self, b: torch.Tensor, config: LatticeConfig) -> torch.Tensor:
        squeeze = b.dim() == 2
        if squeeze:
            b = b.unsqueeze(0)
        n, M, d = b.shape
        if d != 8:
            raise ValueError(f"Code dimension {d} doesn't match E8 dimension 8")
        q = int(config.q)
        _check_qm(q, M)
        bg = on_gpu(b).float().contiguous()
        out = torch.empty((n, 8), dtype=torch.float32, device=bg.device)
        # one block decodes with the reference's contiguous-row distance rule,
        # a batch with its strided-row rule (only visible for q not 2^k)
        _lib.call("coset_e8_hnlq_decode", None, _lib.ptr(bg), n, _lib.SCALE_CODEC,
                  float(config.beta), None, 0, 0.0, q, M, int(n > 1), _lib.ptr(out), _lib.F32,
                  _lib.stream_of(bg))
        out = out.to(b.device)
        return out.squeeze(0) if squeeze else out


def e8_decode(b: torch.Tensor, config: LatticeConfig, method: str = "full", device=None) -> torch.Tensor:
    """coset/core/e8/codecs.py:185-218."""
    method_map = {"full": DecodingMethod.FULL}
    if method not in method_map:
        raise ValueError(f"Unknown decoding method: {method}. Available: {list(method_map.keys())}")
    return E8Decoder(device=device).decode(b, config, method_map[method])


def e8_quantize(x: torch.Tensor, q: int, lattice: Optional[E8Lattice] = None) -> torch.Tensor:
    """coset/core/e8/codecs.py:221-286: decode(encode(x)) with M=2, beta=1,
    fused into one kernel pass."""
    if x.dim() == 1 and x.shape[0] != 8:
        raise ValueError(f"Input dimension {x.shape[0]} doesn't match E8 dimension 8")
    if x.shape[-1] != 8:
        raise ValueError(f"Input dimension {x.shape[-1]} doesn't match E8 dimension 8")
    home = x.device
    _, out = hnlq_roundtrip(x.reshape(-1, 8).float(), int(q), 2, None, want_packed=False)
    return out.reshape(x.shape).to(home)
