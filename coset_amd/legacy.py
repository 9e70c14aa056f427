"""The paper's hierarchical quantizer with overload handling, on the GPU.

Mirrors coset/legacy/quant/functional.py: ``encode`` (15-80, Algorithm 1,
with the 2^alpha rescaling loop while the level chain overloads),
``_encode_internal`` (83-116, the chain and its overload flag), ``decode``
(119-181, Algorithm 2) and ``quantize`` (184-209), for the E8 lattice with
the legacy (textbook) Q.  Those functions take one 8-vector; the
``*_blocks`` forms here run the same algorithm on [N, 8] blocks in one HIP
kernel (coset_e8_legacy_encode / coset_e8_legacy_decode) and also return
the per-block overload flag, which the core codecs do not have (their T is
always 0, coset/core/e8/codecs.py:89).
"""
from __future__ import annotations

import warnings
from typing import Optional, Tuple

import torch

from . import _lib
from .codecs import word_dtype
from .lattice import on_gpu


def _check_e8(lattice) -> None:
    if getattr(lattice, "d", 8) != 8 or getattr(lattice, "name", "E8") != "E8":
        raise ValueError("coset_amd implements the hierarchical quantizer for the E8 lattice only")


def _dither_arg(config, dither, n):
    if not (getattr(config, "with_dither", False) and dither is not None):
        return None, 0
    d = on_gpu(dither).float().contiguous()
    if d.numel() == 8:
        return d, 0
    if d.numel() == 8 * n:
        return d.reshape(n, 8), 8
    raise ValueError(f"dither must hold 8 or {8 * n} values")


def _params(config):
    q, M = int(config.q), int(config.M)
    if not (2 <= q <= 16) or not (1 <= M <= 8):
        raise ValueError(f"q={q}, M={M} outside the supported range (q in [2, 16], M in [1, 8])")
    return q, M, float(config.beta), float(config.alpha)


def encode_blocks(x: torch.Tensor, config, dither: Optional[torch.Tensor] = None, *, packed: bool = False,
                  decoded: bool = False):
    """Algorithm 1 on every 8-wide block of x [N, 8] (fp32 or bf16).

    Returns (codes, T, overload[, x_hat]): codes are float [N, M, 8] like the
    reference (or uint16/uint32 level words [N, M] with ``packed``), T int32
    [N] rescale counts, overload bool [N] (the final chain's Q(x_M) != 0) and,
    with ``decoded``, Algorithm 2 of the same codes [N, 8] fp32."""
    q, M, beta, alpha = _params(config)
    xg = on_gpu(x)
    if xg.dtype not in (torch.float32, torch.bfloat16):
        xg = xg.float()
    xg = xg.contiguous()
    if xg.shape[-1] != 8:
        raise ValueError(f"Input dimension {xg.shape[-1]} doesn't match lattice dimension 8")
    n = xg.numel() // 8
    dev = xg.device
    d, stride = _dither_arg(config, dither, n)
    words = torch.empty((n, M), dtype=word_dtype(q), device=dev) if packed else None
    codes = None if packed else torch.empty((n, M, 8), dtype=torch.float32, device=dev)
    T = torch.empty(n, dtype=torch.int32, device=dev)
    ov = torch.empty(n, dtype=torch.uint8, device=dev)
    out = torch.empty((n, 8), dtype=torch.float32, device=dev) if decoded else None
    max_iter = int(getattr(config, "max_scaling_iterations", 10))
    protect = not bool(getattr(config, "disable_overload_protection", True))
    _lib.call("coset_e8_legacy_encode", _lib.ptr(xg), _lib.dtype_code(xg.dtype), n, beta, alpha, max_iter,
              int(protect), _lib.ptr(d), stride, q, M, _lib.ptr(words), _lib.ptr(codes), _lib.ptr(T), _lib.ptr(ov),
              _lib.ptr(out), _lib.stream_of(xg))
    res = (words if packed else codes, T, ov.bool())
    return res + (out,) if decoded else res


def decode_blocks(codes: torch.Tensor, config, T: Optional[torch.Tensor] = None,
                  dither: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Algorithm 2 on codes [N, M, 8] (float) or level words [N, M] with
    per-block T [N] (None: 0) -> [N, 8] fp32."""
    q, M, beta, alpha = _params(config)
    c = on_gpu(codes).contiguous()
    floaty = c.is_floating_point()
    if floaty:
        c = c.float().reshape(-1, M, 8)
    elif c.dim() != 2 or c.shape[1] != M:
        raise ValueError(f"level words must be [N, {M}]")
    n = c.shape[0]
    t = None if T is None else on_gpu(T).to(torch.int32).contiguous().reshape(-1)
    if t is not None and t.numel() != n:
        raise ValueError(f"T holds {t.numel()} values for {n} blocks")
    d, stride = _dither_arg(config, dither, n)
    out = torch.empty((n, 8), dtype=torch.float32, device=c.device)
    _lib.call("coset_e8_legacy_decode", None if floaty else _lib.ptr(c), _lib.ptr(c) if floaty else None,
              _lib.ptr(t), n, beta, alpha, _lib.ptr(d), stride, q, M, _lib.ptr(out), _lib.stream_of(c))
    return out


# --------------------------------------------------------------------------
# reference signatures (one 8-vector per call)
# --------------------------------------------------------------------------

def encode(x: torch.Tensor, lattice, config, dither: Optional[torch.Tensor] = None,
           device: Optional[torch.device] = None) -> Tuple[torch.Tensor, int]:
    """functional.py:15-80: (encoding vectors [M, d], T)."""
    _check_e8(lattice)
    home = x.device if device is None else torch.device(device)
    v = x.flatten()
    if v.shape[0] != lattice.d:
        raise ValueError(f"Input dimension {v.shape[0]} doesn't match lattice dimension {lattice.d}")
    codes, T, ov = encode_blocks(v.reshape(1, 8).float(), config, dither)
    t = int(T[0])
    if bool(ov[0]) and not getattr(config, "disable_overload_protection", True):
        warnings.warn(f"Overload not resolved after {config.max_scaling_iterations} iterations. "
                      "Consider increasing max_scaling_iterations or adjusting parameters.")
    return codes[0].to(home), t


def decode(b: torch.Tensor, lattice, config, T: int = 0, dither: Optional[torch.Tensor] = None,
           device: Optional[torch.device] = None) -> torch.Tensor:
    """functional.py:119-181: the reconstructed 8-vector."""
    _check_e8(lattice)
    home = b.device if device is None else torch.device(device)
    if b.shape[0] != config.M:
        raise ValueError(f"Number of encoding levels {b.shape[0]} doesn't match M={config.M}")
    if b.shape[1] != lattice.d:
        raise ValueError(f"Encoding dimension {b.shape[1]} doesn't match lattice dimension {lattice.d}")
    t = torch.tensor([int(T)], dtype=torch.int32)
    return decode_blocks(b.float().reshape(1, config.M, 8), config, t, dither)[0].to(home)


def quantize(x: torch.Tensor, lattice, config, dither: Optional[torch.Tensor] = None,
             device: Optional[torch.device] = None) -> torch.Tensor:
    """functional.py:184-209: decode(encode(x))."""
    b, T = encode(x, lattice, config, dither, device=device)
    return decode(b, lattice, config, T, dither, device=device)


def quantize_blocks(x: torch.Tensor, config, dither: Optional[torch.Tensor] = None):
    """Encode and decode [N, 8] blocks in one pass: (x_hat [N, 8], T, overload)."""
    _, T, ov, out = encode_blocks(x, config, dither, packed=True, decoded=True)
    return out, T, ov
