"""Value lookup tables (vLUTs) with the reference interface, on the GPU.

Mirrors coset/legacy/quant/vlut.py (vLUTManager 16-198, build_vlut 201-214,
_encoding_to_index 217-238, vlut_mac_operation 241-279,
vlut_accumulate_operation 282-307) and the legacy QuantizationConfig
(coset/legacy/quant/params.py:12-121) the manager is constructed with.
One-sided tables, lookups and the matmul run in HIP kernels
(coset_vlut_* in include/coset_amd.h).

Differences from the reference, by design:
  * the one-sided cache is keyed by the query's values; the reference keys it
    by ``f"{query.sum():.6f}"`` (vlut.py:91), so two queries with equal sums
    share one table there;
  * ``vlut_matmul`` (a matmul over packed codes) has no reference counterpart
    (QLinear._lut_matmul, coset/legacy/nn/qlinear.py:272-281, is F.linear).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from . import _lib
from .lattice import LegacyE8Lattice, on_gpu


@dataclass
class QuantizationConfig:
    """coset/legacy/quant/params.py:12-121 (E8 rows of its beta table)."""
    lattice_type: str = "D4"
    q: int = 4
    M: int = 2
    beta: float = 1.0
    alpha: float = 1.0
    max_scaling_iterations: int = 10
    with_tie_dither: bool = True
    with_dither: bool = False
    disable_scaling: bool = True
    disable_overload_protection: bool = True

    _E8_BETAS = {(2, 2): 0.4, (3, 2): 0.35, (4, 2): 0.3, (5, 2): 0.25, (8, 2): 0.2}

    def __post_init__(self):
        if self.lattice_type not in ["D4", "E8", "Z2"]:
            raise ValueError(f"Unsupported lattice type: {self.lattice_type}")
        if self.q <= 0:
            raise ValueError("q must be positive")
        if self.M <= 0:
            raise ValueError("M must be positive")
        if self.beta <= 0:
            raise ValueError("beta must be positive")
        if self.alpha <= 0:
            raise ValueError("alpha must be positive")
        if self.beta == 1.0:
            # the reference replaces the default beta by its table value, or
            # by 1/sqrt(q) off the table (params.py:45-94, 119-121)
            if self.lattice_type == "E8" and (self.q, self.M) in self._E8_BETAS:
                self.beta = self._E8_BETAS[(self.q, self.M)]
            elif self.lattice_type == "E8":
                self.beta = 1.0 / (self.q ** 0.5)


def _is_legacy(lattice) -> bool:
    return isinstance(lattice, LegacyE8Lattice) or (hasattr(lattice, "Q") and not hasattr(lattice, "projection"))


class vLUTManager:
    """coset/legacy/quant/vlut.py:16-198.  ``lattice`` selects the residual
    rule: a LegacyE8Lattice (textbook Q, as in the reference) or the core
    E8Lattice (the rule of e8_decode)."""

    def __init__(self, lattice, config):
        self.lattice = lattice
        self.config = config
        self.q = config.q
        self.d = lattice.d
        self.M = config.M
        self.legacy = _is_legacy(lattice)
        self._two_sided_vlut: Optional[torch.Tensor] = None
        self._one_sided_vluts: Dict[tuple, torch.Tensor] = {}

    def build_two_sided_vlut(self, device=None) -> torch.Tensor:
        """vLUT[i, j] = <p_i, p_j> over all q^d lattice points (vlut.py:35-70)."""
        device = torch.device("cpu") if device is None else torch.device(device)
        if self._two_sided_vlut is not None and self._two_sided_vlut.device == device:
            return self._two_sided_vlut
        n = self.q ** self.d
        if n > 8192:
            raise ValueError(f"two-sided vLUT of {n} x {n} entries is too large (q^d <= 8192)")
        pts = on_gpu(self._decode_encodings_to_lattice_points(self._generate_all_encodings()))
        self._two_sided_vlut = (pts.double() @ pts.double().T).float().to(device)
        return self._two_sided_vlut

    def build_one_sided_vlut(self, query_vector: torch.Tensor, device=None) -> torch.Tensor:
        """vLUT[i] = <query, r(b_i)> over the q^d codes (vlut.py:72-117)."""
        device = torch.device("cpu") if device is None else torch.device(device)
        if query_vector.numel() != self.d or self.d != 8:
            raise ValueError("one-sided E8 vLUT needs a query of 8 values")
        qv = query_vector.detach().reshape(8).float()
        key = (tuple(qv.cpu().tolist()), str(device))
        hit = self._one_sided_vluts.get(key)
        if hit is not None:
            return hit
        vlut = build_one_sided_vluts(qv.reshape(1, 8), self.q, legacy=self.legacy)[0].to(device)
        self._one_sided_vluts[key] = vlut
        return vlut

    def _generate_all_encodings(self) -> torch.Tensor:
        """All q^d digit vectors, last digit fastest (vlut.py:119-135)."""
        return torch.cartesian_prod(*[torch.arange(self.q) for _ in range(self.d)])

    def _decode_encodings_to_lattice_points(self, encodings: torch.Tensor) -> torch.Tensor:
        """encodings @ G^T (vlut.py:137-156)."""
        G = self.lattice.G.to(encodings.device).float()
        return encodings.float() @ G.T

    def get_vlut_size(self) -> int:
        return self.q ** self.d

    def build_sum_lut(self, device=None) -> torch.Tensor:
        """sum_LUT[i, j] = p_i + p_j (vlut.py:162-193)."""
        device = torch.device("cpu") if device is None else torch.device(device)
        n = self.q ** self.d
        if n > 2048:
            raise ValueError(f"sum LUT of {n} x {n} x {self.d} entries is too large (q^d <= 2048)")
        pts = on_gpu(self._decode_encodings_to_lattice_points(self._generate_all_encodings()))
        return (pts[:, None, :] + pts[None, :, :]).to(device)

    def clear_cache(self):
        self._two_sided_vlut = None
        self._one_sided_vluts.clear()


def build_vlut(lattice, config, device=None) -> torch.Tensor:
    """vlut.py:201-214."""
    return vLUTManager(lattice, config).build_two_sided_vlut(device)


def _encoding_to_index(encoding: torch.Tensor, q: int) -> torch.Tensor:
    """idx = sum_j encoding[:, j] q^(d-1-j) (vlut.py:217-238)."""
    _, d = encoding.shape
    powers = torch.pow(q, torch.arange(d - 1, -1, -1, dtype=torch.long, device=encoding.device))
    return torch.sum(encoding * powers, dim=1).long()


def vlut_mac_operation(encodings_x: List[torch.Tensor], encodings_y: List[torch.Tensor],
                       vlut: torch.Tensor) -> torch.Tensor:
    """sum_i vLUT[idx(b_i(x)), idx(b_i(y))] (vlut.py:241-279)."""
    M = len(encodings_x)
    d = encodings_x[0].shape[1]
    q = int(round(vlut.shape[0] ** (1.0 / d)))
    ix = torch.stack([_encoding_to_index(encodings_x[i], q) for i in range(M)])
    iy = torch.stack([_encoding_to_index(encodings_y[i], q) for i in range(M)])
    return torch.sum(vlut[ix, iy], dim=0)


def vlut_accumulate_operation(encodings: List[torch.Tensor]) -> List[torch.Tensor]:
    """vlut.py:282-307 (sums each level's encodings across the list)."""
    M = len(encodings[0])
    return [torch.sum(torch.stack([enc[i] for enc in encodings], dim=0), dim=0) for i in range(M)]


# --------------------------------------------------------------------------
# native entry points
# --------------------------------------------------------------------------

def build_one_sided_vluts(queries: torch.Tensor, q: int, legacy: bool = True) -> torch.Tensor:
    """[n, 8] queries -> [n, q^8] one-sided tables on the GPU."""
    if not (2 <= q <= 8):
        raise ValueError("one-sided E8 vLUTs need q in [2, 8]")
    qs = on_gpu(queries).float().contiguous().reshape(-1, 8)
    out = torch.empty((qs.shape[0], q ** 8), dtype=torch.float32, device=qs.device)
    _lib.call("coset_vlut_build_one_sided", _lib.ptr(qs), qs.shape[0], int(q), int(legacy), _lib.ptr(out),
              _lib.stream_of(qs))
    return out


def vlut_dot(words: torch.Tensor, vlut: torch.Tensor, q: int) -> torch.Tensor:
    """sum_m q^m vlut[words[:, m]] for packed level words [N, M]."""
    w = on_gpu(words).contiguous()
    v = on_gpu(vlut).float().contiguous()
    n, M = w.shape
    out = torch.empty(n, dtype=torch.float32, device=w.device)
    _lib.call("coset_vlut_lookup_dot", _lib.ptr(w), n, int(q), int(M), _lib.ptr(v), _lib.ptr(out),
              _lib.stream_of(w))
    return out


_METHODS = {"auto": 0, "lds": 1, "mfma": 2}
_LAYOUTS = {"rowmajor": 1, "tiled": 2, "decoded": 3, "pairs": 4, "decoded6": 5}


@dataclass
class PreparedWords:
    """Level words converted once for vlut_matmul (coset_vlut_prepare):
    uint32 cid << 16 | idx values, row-major or tiled in matrix-core fragment
    order (16 rows x 4 k-blocks per 64-entry tile), ("decoded") the
    pairs' 2 x_hat as biased bytes in the tiled order, ("decoded6") the same
    decode in 6 bytes per pair (one parity bit and eight 6-bit fields,
    chunks of 8 k-quads per lane), or ("pairs") each level word's four
    coordinate-pair ids, [rows / 64][kb][M][64 rows], which the LDS-table
    method reads without a map lookup."""
    data: torch.Tensor
    rows: int
    kb: int
    M: int
    q: int
    legacy: bool
    layout: str

    @property
    def word_format(self) -> int:
        return _LAYOUTS[self.layout]


def vlut_prepare(words: torch.Tensor, q: int = 4, legacy: bool = False, layout: str = "tiled") -> PreparedWords:
    """uint16 level words [rows, K/8, M] -> PreparedWords, the weight format
    vlut_matmul reads without the coarse-id gather ("rowmajor", "tiled") or
    without any table lookup ("decoded": 8 bytes per pair, q = 4 with M <= 2
    or q = 2 with M <= 4; "decoded6": 6 bytes per pair where the decode's
    range fits, e.g. q = 4 with M <= 2; both on the matrix cores), or as the coordinate-pair
    ids the LDS-table method looks up ("pairs": any activation dtype,
    method "lds" or "auto").  Done once per weight; ``legacy`` fixes the
    residual rule the matmul will use."""
    w = on_gpu(words).contiguous()
    if w.dtype != torch.uint16 or w.dim() != 3:
        raise ValueError("vlut_prepare takes uint16 level words [rows, K/8, M] (q <= 4)")
    if layout not in _LAYOUTS:
        raise ValueError(f"layout must be one of {sorted(_LAYOUTS)}")
    rows, kb, M = w.shape
    fmt = _LAYOUTS[layout]
    n = _lib.load().coset_vlut_prepared_words(rows, kb, M, fmt)
    out = torch.empty(max(int(n), 1), dtype=torch.uint32, device=w.device)
    _lib.call("coset_vlut_prepare", _lib.ptr(w), rows, kb, int(M), int(q), int(legacy), fmt, _lib.ptr(out),
              _lib.stream_of(w))
    return PreparedWords(out, rows, kb, M, int(q), bool(legacy), layout)


def vlut_matmul(words, act: torch.Tensor, q: int = 4, *, scale: Optional[torch.Tensor] = None,
                scale_mode: str = "mul", legacy: bool = False, method: str = "auto",
                workspace: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                act_quant: Optional[Tuple[torch.Tensor, int]] = None) -> torch.Tensor:
    """out[B, rows] = s_o * sum_k sum_m q^m vLUT_{act[:, 8k:8k+8]}[words[o, k, m]].

    words: packed level words [rows, K/8, M] (uint16, q in {2, 4}), or a
    PreparedWords from vlut_prepare (its q and legacy rule are used); act:
    [B, K] float32 / bfloat16 / float16.  scale (per output row) multiplies
    (``scale_mode="mul"``, codec convention) or divides (``"div"``, layer
    convention).  With the core rule (legacy=False) the result equals
    act @ (e8_decode(codes) * s)^T.

    method: "lds" (per-token inner-product tables in LDS), "mfma" (decoded
    weights on the matrix cores; fp32 activations run as three exact bf16
    planes) or "auto" (mfma wherever 2 x_hat is exact in the operand type).

    Epilogue, fused into the output write (coset_vlut_linear): ``bias``
    [rows] is added, then ``act_quant = (alpha, qmax)`` applies the LSQ
    activation quantizer with that parameter (inference: no gradient).
    """
    if isinstance(words, PreparedWords):
        rows, kb, M = words.rows, words.kb, words.M
        q, legacy, fmt = words.q, words.legacy, words.word_format
        w = words.data
    else:
        w = on_gpu(words).contiguous()
        if w.dim() != 3 or w.dtype != torch.uint16:
            raise ValueError("words must be uint16 [rows, K/8, M] or PreparedWords")
        rows, kb, M = w.shape
        fmt = 0
    a = on_gpu(act).contiguous()
    if a.dim() != 2 or a.shape[1] != 8 * kb:
        raise ValueError(f"act must be [B, {8 * kb}]")
    B, K = a.shape
    m = _METHODS[method]
    if fmt == _LAYOUTS["pairs"]:
        if method == "mfma":
            raise ValueError('the "pairs" layout is read by the lds method only')
        m = _METHODS["lds"]
    dt = _lib.dtype_code(a.dtype)
    need = _lib.load().coset_vlut_workspace_floats(B, rows, K, int(q), int(M), dt, m)
    if need > 0 and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(int(need), dtype=torch.float32, device=a.device)
    s = None
    if scale is not None:
        s = on_gpu(scale).float().contiguous()
        if s.numel() != rows:
            raise ValueError(f"scale must hold one value per output row ({rows}), got {s.numel()}")
    if scale_mode not in ("mul", "div"):
        raise ValueError(f"scale_mode must be 'mul' or 'div', got {scale_mode!r}")
    out = torch.empty((B, rows), dtype=torch.float32, device=a.device)
    ws_n = workspace.numel() if workspace is not None else 0
    if bias is None and act_quant is None:
        _lib.call("coset_vlut_matmul", _lib.ptr(w), fmt, _lib.ptr(s), 0 if scale_mode == "mul" else 1, _lib.ptr(a),
                  dt, B, rows, K, int(q), int(M), int(legacy), m, _lib.ptr(workspace), ws_n, _lib.ptr(out),
                  _lib.stream_of(a))
        return out
    b = None if bias is None else on_gpu(bias).float().contiguous()
    if b is not None and b.numel() != rows:
        raise ValueError(f"bias must hold {rows} values")
    alpha, qmax = (None, 0) if act_quant is None else act_quant
    al = None if alpha is None else on_gpu(alpha).detach().float().reshape(1).contiguous()
    _lib.call("coset_vlut_linear", _lib.ptr(w), fmt, _lib.ptr(s), 0 if scale_mode == "mul" else 1, _lib.ptr(a), dt,
              B, rows, K, int(q), int(M), int(legacy), m, _lib.ptr(b), _lib.ptr(al), int(qmax),
              _lib.ptr(workspace), ws_n, _lib.ptr(out), _lib.stream_of(a))
    return out
