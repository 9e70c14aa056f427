"""Lattice objects with the reference interface, computing on the GPU.

Mirrors coset/core/base.py (LatticeConfig 15-62, Lattice 64-292) and
coset/core/e8/lattice.py (E8Lattice 14-169); the legacy E8 lattice whose
textbook ``Q`` defines the vLUT residual mirrors coset/legacy/lattices/e8.py.
Every numeric method runs a HIP kernel of libcoset_amd.so.
"""
from __future__ import annotations

from typing import Any, Dict, Optional

import numpy as np
import torch

from . import _lib

try:  # the reference config is a pydantic model; keep that when available
    from pydantic import BaseModel as _Base
except ImportError:  # pragma: no cover
    _Base = None


if _Base is not None:
    class LatticeConfig(_Base):
        """coset/core/base.py:15-62.  Like the reference (whose validation in
        ``__post_init__`` never runs under pydantic v2) construction accepts
        any values; the codecs check q and M when they run."""
        lattice_type: str
        q: int
        M: int
        beta: float = 1.0
        alpha: float = 1.0
        decoding: str = "full"
        check_overload: bool = True
        disable_overload_protection: bool = True
        disable_scaling: bool = True
        with_tie_dither: bool = True
        with_dither: bool = False
        max_scaling_iterations: int = 10

        @classmethod
        def from_dict(cls, config_dict: Dict[str, Any]) -> "LatticeConfig":
            return cls(**config_dict)

        def to_dict(self) -> Dict[str, Any]:
            return self.model_dump()
else:  # pragma: no cover
    from dataclasses import asdict, dataclass

    @dataclass
    class LatticeConfig:
        lattice_type: str
        q: int
        M: int
        beta: float = 1.0
        alpha: float = 1.0
        decoding: str = "full"
        check_overload: bool = True
        disable_overload_protection: bool = True
        disable_scaling: bool = True
        with_tie_dither: bool = True
        with_dither: bool = False
        max_scaling_iterations: int = 10

        @classmethod
        def from_dict(cls, d):
            return cls(**d)

        def to_dict(self):
            return asdict(self)


# E8 generator: columns are the basis vectors (coset/core/e8/lattice.py:32-41)
_E8_ROWS = [
    [2, 0, 0, 0, 0, 0, 0, 0],
    [-1, 1, 0, 0, 0, 0, 0, 0],
    [0, -1, 1, 0, 0, 0, 0, 0],
    [0, 0, -1, 1, 0, 0, 0, 0],
    [0, 0, 0, -1, 1, 0, 0, 0],
    [0, 0, 0, 0, -1, 1, 0, 0],
    [0, 0, 0, 0, 0, -1, 1, 0],
    [0.5] * 8,
]


def default_device(device=None) -> torch.device:
    if device is not None:
        return torch.device(device)
    return torch.device("cuda") if torch.cuda.is_available() else torch.device("cpu")


def on_gpu(t: torch.Tensor) -> torch.Tensor:
    """The tensor on the current GPU (a copy when it lives on the host)."""
    dev = _lib.require_gpu()
    if t.device.type != "cuda":
        t = t.to(dev)
    return t


def _blocks(x: torch.Tensor) -> torch.Tensor:
    """Contiguous fp32 view [N, 8] of a [..., 8] input."""
    if x.shape[-1] != 8:
        raise ValueError(f"Input dimension {x.shape[-1]} doesn't match E8 dimension 8")
    return on_gpu(x).to(torch.float32).contiguous().reshape(-1, 8)


class Lattice:
    """coset/core/base.py:64-292 with the arithmetic on the GPU."""

    def __init__(self, G: torch.Tensor, name: str, device=None, config: Optional[LatticeConfig] = None):
        if G.shape[0] != G.shape[1]:
            raise ValueError("Generator matrix G must be square")
        if device is not None:
            G = G.to(device)
        self.G = G
        # the E8 inverse has entries in (1/2)Z: float64 inversion rounds to it exactly
        self.G_inv = torch.linalg.inv(G.detach().cpu().double()).to(G.dtype).to(G.device)
        self.name = name
        self.d = G.shape[0]
        self.device = G.device
        self.config = config
        self.r_pack = self._compute_packing_radius()
        self.r_cov = self._compute_covering_radius()

    def get_generators(self):
        return self.G.clone().detach(), self.G_inv.clone().detach()

    def projection(self, x: torch.Tensor) -> torch.Tensor:  # pragma: no cover - abstract
        raise NotImplementedError

    def _lattice_op(self, op: int, x: torch.Tensor, q: int = 0, legacy: bool = False) -> torch.Tensor:
        squeeze = x.dim() == 1
        xb = _blocks(x)
        out = torch.empty_like(xb)
        _lib.call("coset_e8_lattice_op", op, int(legacy), _lib.ptr(xb), xb.shape[0], int(q),
                  _lib.ptr(out), _lib.stream_of(xb))
        out = out.to(x.device)
        return out.reshape(8) if squeeze else out.reshape(x.shape)

    def encode_coords(self, x: torch.Tensor, q: int) -> torch.Tensor:
        """round(G^-1 x) mod q (coset/core/base.py:134-154)."""
        return self._lattice_op(_lib.OP_ENCODE_COORDS, x, q)

    def decode_coords(self, b: torch.Tensor, q: int) -> torch.Tensor:
        """G b (coset/core/base.py:156-176)."""
        return self._lattice_op(_lib.OP_DECODE_COORDS, b.float(), q)

    def custom_round(self, x: torch.Tensor, tiny: Optional[float] = None) -> torch.Tensor:
        """floor((x - sign(x)*eps) + 0.5) (coset/core/base.py:179-202), fp32."""
        if tiny is not None and float(tiny) != float(torch.finfo(torch.float32).eps):
            raise NotImplementedError("custom_round runs with the fp32 machine epsilon only")
        if x.dtype != torch.float32:
            raise NotImplementedError("custom_round runs on float32 tensors")
        flat = on_gpu(x).contiguous().reshape(-1)
        n = flat.numel()
        nb = (n + 7) // 8
        buf = torch.zeros(nb * 8, dtype=torch.float32, device=flat.device)
        buf[:n] = flat
        out = torch.empty_like(buf)
        _lib.call("coset_e8_lattice_op", _lib.OP_CUSTOM_ROUND, 0, _lib.ptr(buf), nb, 0,
                  _lib.ptr(out), _lib.stream_of(buf))
        return out[:n].reshape(x.shape).to(x.device)

    def generate_tie_dither(self, beta: float = 1.0, Rin: float = 0.5, magnitude: str = "auto") -> torch.Tensor:
        """coset/core/base.py:204-229 (host-side constant)."""
        primes = [2, 3, 5, 7, 11, 13, 17, 19][: self.d]
        irr = torch.tensor([np.sqrt(p) for p in primes], dtype=torch.float32)
        u = (irr - torch.floor(irr)) - 0.5
        u = u / torch.norm(u)
        delta = (2.0 ** -40) * beta * Rin if magnitude == "auto" else float(magnitude)
        return delta * u

    def _compute_packing_radius(self) -> float:
        gram = (self.G.T @ self.G).double().cpu()
        ev = torch.linalg.eigvals(gram).real
        return 0.5 * float(torch.sqrt(ev[ev > 1e-10].min()))

    def _compute_covering_radius(self) -> float:
        return self.r_pack * float(np.sqrt(self.d))

    def compute_delta0(self, q: int, M: int, rho: float = 0.95) -> float:
        """Delta0 = 2 rho r_pack / (q^M - 1) (coset/core/base.py:270-284)."""
        return (2.0 * rho * self.r_pack) / (q ** M - 1)

    def __repr__(self) -> str:
        return f"{self.name}Lattice(d={self.d})"

    __str__ = __repr__


class E8Lattice(Lattice):
    """coset/core/e8/lattice.py:14-169; ``projection`` is the core closest
    point with the reference's g_x rule (a negative worst coordinate always
    steps down)."""

    def __init__(self, device=None, config: Optional[LatticeConfig] = None):
        device = default_device(device)
        G = torch.tensor(_E8_ROWS, dtype=torch.float32, device=device).T
        super().__init__(G, "E8", device=device, config=config)

    def _compute_packing_radius(self) -> float:
        return 0.5

    def _compute_covering_radius(self) -> float:
        return float(np.sqrt(2) / 2)

    def g_x(self, x: torch.Tensor) -> torch.Tensor:
        return self._lattice_op(_lib.OP_G_X, x)

    def projection(self, x: torch.Tensor) -> torch.Tensor:
        return self._lattice_op(_lib.OP_PROJECT, x)


class LegacyE8Lattice(Lattice):
    """coset/legacy/lattices/e8.py:13-103: textbook g_x (flip toward x); its
    ``Q`` is the residual rule of the legacy one-sided vLUT."""

    legacy = True

    def __init__(self, device=None):
        device = default_device(device)
        G = torch.tensor(_E8_ROWS, dtype=torch.float32, device=device).T
        super().__init__(G, "E8", device=device)

    def _compute_packing_radius(self) -> float:
        return 0.5

    def g_x(self, x: torch.Tensor) -> torch.Tensor:
        return self._lattice_op(_lib.OP_G_X, x, legacy=True)

    def Q(self, x: torch.Tensor) -> torch.Tensor:
        return self._lattice_op(_lib.OP_PROJECT, x, legacy=True)

    projection = Q


_D4_ROWS = [[-1, -1, 0, 0], [1, -1, 0, 0], [0, 1, -1, 0], [0, 0, 1, -1]]


class D4Lattice(Lattice):
    """coset/core/d4/lattice.py:14-146: integer points with an even
    coordinate sum.  ``projection`` rounds with custom_round and, for an odd
    sum, moves the first coordinate farthest from an integer by +1 when it is
    >= 0 and above its rounding, by -1 otherwise (the reference's g_x).  The
    operators run in coset_d4_lattice_op over [N, 4] blocks."""

    def __init__(self, device=None, config: Optional[LatticeConfig] = None):
        device = default_device(device)
        G = torch.tensor(_D4_ROWS, dtype=torch.float32, device=device).T
        super().__init__(G, "D4", device=device, config=config)

    def _compute_packing_radius(self) -> float:
        return 1.0 / np.sqrt(2)

    def _compute_covering_radius(self) -> float:
        return 1.0

    def _d4_op(self, op: int, x: torch.Tensor, q: int = 0) -> torch.Tensor:
        if x.shape[-1] != 4:
            raise ValueError(f"Input dimension {x.shape[-1]} doesn't match D4 dimension 4")
        squeeze = x.dim() == 1
        xb = on_gpu(x).to(torch.float32).contiguous().reshape(-1, 4)
        out = torch.empty_like(xb)
        _lib.call("coset_d4_lattice_op", op, _lib.ptr(xb), xb.shape[0], int(q), _lib.ptr(out), _lib.stream_of(xb))
        out = out.to(x.device)
        return out.reshape(4) if squeeze else out.reshape(x.shape)

    def g_x(self, x: torch.Tensor) -> torch.Tensor:
        return self._d4_op(_lib.OP_G_X, x)

    def projection(self, x: torch.Tensor) -> torch.Tensor:
        return self._d4_op(_lib.OP_PROJECT, x)

    def encode_coords(self, x: torch.Tensor, q: int) -> torch.Tensor:
        """round(G^-1 x) mod q (coset/core/base.py:134-154)."""
        return self._d4_op(_lib.OP_ENCODE_COORDS, x, q)

    def decode_coords(self, b: torch.Tensor, q: int) -> torch.Tensor:
        """G b (coset/core/base.py:156-176)."""
        return self._d4_op(_lib.OP_DECODE_COORDS, b.float(), q)


_D4_BY_DEVICE: Dict[str, "D4Lattice"] = {}


def d4_quantize(x: torch.Tensor, q: int) -> torch.Tensor:
    """The D4 layer's quantizer: the closest D4 point, q unused
    (coset/core/d4/layers.py:46-47)."""
    key = str(x.device)
    lat = _D4_BY_DEVICE.get(key)
    if lat is None:
        lat = _D4_BY_DEVICE[key] = D4Lattice(device=x.device)
    return lat.projection(x)
