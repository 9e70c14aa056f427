"""numpy front end of the C parity oracle (oracle/e8_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by the ``cpu_baseline`` leg of bench.py, always as the checker.  The
product (coset_amd/) never imports it.

Each wrapper restates one reference function (cited in e8_oracle.c); the
closed forms here (``beta_bounds``, ``layer_backward``) restate
coset/core/layers.py:381-426 and the autograd chain of layers.py:428-478.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libe8oracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float


def build() -> str:
    """Compile the oracle with its Makefile (gcc, no contraction)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_custom_round.argtypes = [_flt]
        L.or_custom_round.restype = _flt
        L.or_g_x.argtypes = [_f32p, _int, _f32p]
        L.or_projection.argtypes = [_f32p, _i64, _int, _f32p]
        L.or_encode_coords.argtypes = [_f32p, _i64, _int, _i32p]
        L.or_decode_coords.argtypes = [_i32p, _i64, _f32p]
        L.or_pack_index.argtypes = [_i32p, _int]
        L.or_pack_index.restype = ctypes.c_uint32
        L.or_e8_encode.argtypes = [_f32p, _i64, _flt, _int, _int, _i32p]
        L.or_e8_decode.argtypes = [_i32p, _i64, _flt, _int, _int, _f32p]
        L.or_residual.argtypes = [_i32p, _int, _int, _int, _f32p]
        L.or_layer_quant.argtypes = [_f32p, _i64, _i64, _f32p, _int, _int, _flt,
                                     _f32p, ctypes.c_void_p, ctypes.c_void_p]
        L.or_build_one_sided_vlut.argtypes = [_f32p, _int, _int, _f32p]
        L.or_vlut_matmul.argtypes = [_u32p, _f32p, _int, _f32p, _i64, _i64, _i64,
                                     _int, _int, _int, _f32p]
        L.or_residual_table.argtypes = [_int, _int, _int, _f32p]
        L.or_vlut_onesided_accumulate.argtypes = [_u32p, _i64, _i64, _int, _int, _f32p, _f32p, _i64, _i64,
                                                  _f32p, np.ctypeslib.ndpointer(dtype=np.float64,
                                                                                flags="C_CONTIGUOUS")]
        _u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
        L.or_legacy_encode.argtypes = [_f32p, _i64, _flt, _flt, _int, _int, ctypes.c_void_p, _i64, _int, _int,
                                       _i32p, _i32p, _u8p]
        L.or_legacy_decode.argtypes = [_i32p, _i32p, _i64, _flt, _f32p, ctypes.c_void_p, _i64, _int, _int,
                                       _f32p]
        L.or_d4_g_x.argtypes = [_f32p, _f32p]
        L.or_d4_projection.argtypes = [_f32p, _i64, _f32p]
        L.or_d4_encode_coords.argtypes = [_f32p, _i64, _int, _i32p]
        L.or_d4_decode_coords.argtypes = [_i32p, _i64, _f32p]
        L.or_d4_layer_quant.argtypes = [_f32p, _i64, _i64, _f32p, _i64, _flt, _f32p]
        _lib = L
    return _lib


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def custom_round(x):
    x = _f32(x)
    f = np.vectorize(lambda v: lib().or_custom_round(float(v)), otypes=[np.float32])
    return f(x).astype(np.float32)


def g_x(x, legacy=False):
    x = _f32(x).reshape(-1, 8)
    out = np.empty_like(x)
    for i in range(x.shape[0]):
        row = np.empty(8, np.float32)
        lib().or_g_x(np.ascontiguousarray(x[i]), int(legacy), row)
        out[i] = row
    return out


def projection(x, legacy=False):
    x = _f32(x).reshape(-1, 8)
    y = np.empty_like(x)
    lib().or_projection(x, x.shape[0], int(legacy), y)
    return y


def encode_coords(y, q):
    y = _f32(y).reshape(-1, 8)
    b = np.empty(y.shape, np.int32)
    lib().or_encode_coords(y, y.shape[0], int(q), b)
    return b


def decode_coords(b):
    b = np.ascontiguousarray(b, np.int32).reshape(-1, 8)
    y = np.empty(b.shape, np.float32)
    lib().or_decode_coords(b, b.shape[0], y)
    return y


def e8_encode(x, q, M, beta=1.0):
    """Codes [N, M, 8] int32 of coset/core/e8/codecs.py:17-89 (no dither)."""
    x = _f32(x).reshape(-1, 8)
    codes = np.empty((x.shape[0], M, 8), np.int32)
    lib().or_e8_encode(x, x.shape[0], float(np.float32(beta)), int(q), int(M), codes)
    return codes


def e8_decode(codes, q, M, beta=1.0):
    codes = np.ascontiguousarray(codes, np.int32).reshape(-1, M, 8)
    out = np.empty((codes.shape[0], 8), np.float32)
    lib().or_e8_decode(codes, codes.shape[0], float(np.float32(beta)), int(q), int(M), out)
    return out


def residual(b, q, legacy=False, strided=False):
    b = np.ascontiguousarray(b, np.int32).reshape(-1, 8)
    out = np.empty(b.shape, np.float32)
    for i in range(b.shape[0]):
        r = np.empty(8, np.float32)
        lib().or_residual(np.ascontiguousarray(b[i]), int(q), int(legacy), int(strided), r)
        out[i] = r
    return out


def pack_words(codes, q):
    """[N, M, 8] digits -> [N, M] level words idx(b) = sum_j b_j q^(7-j)."""
    codes = np.asarray(codes, np.int64)
    w = np.zeros(codes.shape[:-1], np.int64)
    for j in range(8):
        w = w * q + codes[..., j]
    return w.astype(np.uint32)


def unpack_words(words, q):
    w = np.asarray(words, np.int64)
    out = np.empty(w.shape + (8,), np.int32)
    for j in range(7, -1, -1):
        out[..., j] = w % q
        w = w // q
    return out


def layer_quant(W, beta_row, q, M, clip):
    """W_q, unscaled Q and codes of coset/core/layers.py:428-463."""
    W = _f32(W)
    rows, cols = W.shape
    beta_row = _f32(beta_row).reshape(-1)
    Wq = np.empty_like(W)
    qraw = np.empty_like(W)
    codes = np.empty((rows * cols // 8, M, 8), np.int32)
    lib().or_layer_quant(W, rows, cols, beta_row, int(q), int(M), float(clip), Wq,
                         qraw.ctypes.data, codes.ctypes.data)
    return Wq, qraw, codes


def build_one_sided_vlut(a, q, legacy=True):
    a = _f32(a).reshape(8)
    out = np.empty(q ** 8, np.float32)
    lib().or_build_one_sided_vlut(a, int(q), int(legacy), out)
    return out


def vlut_matmul(words, scale, act, q, M, scale_mode=0, legacy=False):
    """out[B, rows] of the one-sided lookup over packed words [rows, K/8, M]."""
    words = np.ascontiguousarray(words, np.uint32)
    rows, kb, m = words.shape
    assert m == M
    act = _f32(act)
    B, K = act.shape
    assert K == 8 * kb
    out = np.empty((B, rows), np.float32)
    lib().or_vlut_matmul(words, _f32(scale).reshape(-1), int(scale_mode), act, B, rows, K,
                         int(q), int(M), int(legacy), out)
    return out


def residual_table(q, legacy=False, strided=True):
    """r(b) for all q^8 level words, [q^8, 8] fp32 (or_residual per word)."""
    R = np.empty((q ** 8, 8), np.float32)
    lib().or_residual_table(int(q), int(legacy), int(strided), R)
    return R


def vlut_onesided_rows(words, R, a_row, q, kb0=0, kb1=None):
    """sum over k-blocks [kb0, kb1) of the one-sided vLUT lookups for one
    activation row a_row [K] (vlut.py:72-117 + the lookup sum of
    test_one_sided_vlut_pytest.py:22-43): float64 [rows] partial sums."""
    words = np.ascontiguousarray(words, np.uint32)
    rows, kb, M = words.shape
    kb1 = kb if kb1 is None else kb1
    acc = np.zeros(rows, np.float64)
    table = np.empty(q ** 8, np.float32)
    lib().or_vlut_onesided_accumulate(words, rows, kb, M, int(q), R, _f32(a_row).reshape(-1), int(kb0), int(kb1),
                                      table, acc)
    return acc


# --------------------------------------------------------------------------
# beta pipeline and backward closed forms (float64 restatements; the layer
# tolerances are 1e-3 relative so the float64 form is the stricter checker)
# --------------------------------------------------------------------------

def delta0(q, M, rho=0.95, r_pack=0.5):
    """coset/core/base.py:270-284."""
    return (2.0 * rho * r_pack) / (q ** M - 1)


def beta_bounds(q, M, Delta0, eta, sigma_ema, xmax_ema, gamma_inv=12.0):
    """coset/core/layers.py:381-396 in float64."""
    qM = float(q ** M)
    sigma = np.asarray(sigma_ema, np.float64)
    xmax = np.asarray(xmax_ema, np.float64)
    bmin = (Delta0 / qM) / (eta * gamma_inv * sigma)
    bmax = np.minimum((Delta0 * (qM - 1)) / (2 * gamma_inv * xmax),
                      (Delta0 * (qM - 1)) / (2 * eta * gamma_inv * sigma))
    bmin = np.minimum(bmin, bmax * 0.9)
    return bmin, bmax


def beta_from_theta(theta, bmin, bmax):
    """coset/core/layers.py:419-422."""
    s = 1.0 / (1.0 + np.exp(-np.asarray(theta, np.float64)))
    return bmin + s * (bmax - bmin)


def layer_backward(gWq, W, qraw, beta_row, clip):
    """dL/dW and dL/dbeta of W_q = clamp(STE(W*beta)/beta, -clip, clip).

    Autograd chain of coset/core/layers.py:431-463: clamp passes the gradient
    where -clip <= Q/beta <= clip; div gives g/beta to Q and -g*Q/beta^2 to
    beta; the STE (layers.py:87-95) is the identity; mul gives (.)*beta to W
    and sum((.)*W) to beta.
    """
    g = np.asarray(gWq, np.float64)
    W = np.asarray(W, np.float64)
    Q = np.asarray(qraw, np.float64)
    beta = np.asarray(beta_row, np.float64).reshape(-1, 1)
    Wq_unclamped = np.asarray(qraw, np.float32) / np.asarray(beta_row, np.float32).reshape(-1, 1)
    mask = (Wq_unclamped >= -clip) & (Wq_unclamped <= clip)
    gm = g * mask
    gQ = gm / beta
    dW = gQ * beta
    dbeta = (gQ * W).sum(axis=1) - (gm * Q / (beta * beta)).sum(axis=1)
    return dW, dbeta, mask


def gather_stats(W_tiles, sigma_ema, xmax_ema, momentum=0.99):
    """coset/core/layers.py:366-379 on [tiles, n] weights: the unbiased std
    (variance in float64, its root rounded once to fp32, as torch's CPU
    reduction), abs-max, + 1e-8, and the fp32 EMA with m and 1 - m rounded
    to fp32.  Returns the new (sigma_ema, xmax_ema)."""
    W = np.asarray(W_tiles, np.float32)
    Wd = W.astype(np.float64)
    n = W.shape[1]
    mean = Wd.mean(axis=1, keepdims=True)
    sd = np.sqrt(((Wd - mean) ** 2).sum(axis=1) / (n - 1)).astype(np.float32)
    eps = np.float32(1e-8)
    s1 = (sd + eps).astype(np.float32)
    x1 = (np.abs(W).max(axis=1) + eps).astype(np.float32)
    m, om = np.float32(momentum), np.float32(1.0 - momentum)
    se = (np.asarray(sigma_ema, np.float32) * m).astype(np.float32) + (om * s1).astype(np.float32)
    xe = (np.asarray(xmax_ema, np.float32) * m).astype(np.float32) + (om * x1).astype(np.float32)
    return se.astype(np.float32), xe.astype(np.float32)


def _lsq_parts(x, alpha, qmax):
    """fp32 intermediates of LSQActivation.forward (coset/core/layers.py:
    129-137) in the reference's operation order, with the straight-through
    terms of ste_clip / ste_round (layers.py:20-26) kept: (x - x) and
    (y - y) are +0 for finite values and turn a -0 result into +0."""
    x = np.asarray(x, np.float32)
    a = np.float32(np.float32(max(np.float32(alpha), np.float32(0))) + np.float32(1e-8))
    with np.errstate(invalid="ignore"):
        xc = ((x - x).astype(np.float32) + np.clip(x, -a, a).astype(np.float32)).astype(np.float32)
        s = np.float32(a / np.float32(qmax))
        y = (xc / s).astype(np.float32)
        yq = ((y - y).astype(np.float32) + np.round(y).astype(np.float32)).astype(np.float32)
    return a, s, xc, y, yq


def lsq_forward(x, alpha, qmax):
    """LSQActivation.forward: round(clamp(x, -a, a) / s) * s, a = relu(alpha)
    + 1e-8, s = a / qmax (round half to even), fp32."""
    _, s, _, _, yq = _lsq_parts(x, alpha, qmax)
    return (yq * s).astype(np.float32)


def lsq_backward(x, g, alpha, qmax):
    """Autograd of lsq_forward: the STE terms pass g straight through the
    clamp and the rounding, so dx = (g s) / s (fp32), and the clamp bound is
    detached (no gradient to alpha through it); alpha's gradient comes from
    s alone: dalpha = [alpha > 0] (sum g yq - sum (g s)((xc / s) / s)) / qmax,
    the products in fp32 as autograd forms them, the sums in float64.
    Returns (dx, dalpha, the sum of the terms' magnitudes / qmax)."""
    g = np.asarray(g, np.float32)
    a, s, xc, y, yq = _lsq_parts(x, alpha, qmax)
    gs = (g * s).astype(np.float32)
    dx = (gs / s).astype(np.float32)
    t1 = (g * yq).astype(np.float32).astype(np.float64)
    t2 = (gs * ((xc / s).astype(np.float32) / s).astype(np.float32)).astype(np.float32).astype(np.float64)
    mag = (np.abs(t1).sum() + np.abs(t2).sum()) / qmax
    if not np.float32(alpha) > 0:
        return dx, 0.0, mag
    return dx, float((t1.sum() - t2.sum()) / qmax), mag


# --------------------------------------------------------------------------
# legacy hierarchical encode / decode (coset/legacy/quant/functional.py)
# --------------------------------------------------------------------------

def legacy_scale_table(alpha, n=64):
    """(float)2^(alpha t), t = 0..n-1: the decode's 2 ** (alpha * T) in fp32."""
    return np.array([np.float32(2.0 ** (alpha * t)) for t in range(n)], np.float32)


def legacy_encode(x, q, M, beta, alpha=1.0, max_iter=10, protect=True, dither=None):
    """functional.py:15-116 per 8-vector: codes [N, M, 8], T [N], overload [N]."""
    x = _f32(x).reshape(-1, 8)
    n = x.shape[0]
    codes = np.empty((n, M, 8), np.int32)
    T = np.empty(n, np.int32)
    ov = np.empty(n, np.uint8)
    d = None if dither is None else _f32(dither)
    stride = 0 if d is None or d.size == 8 else 8
    lib().or_legacy_encode(x, n, float(np.float32(beta)), float(np.float32(2.0 ** alpha)), int(max_iter),
                           int(bool(protect)), None if d is None else d.ctypes.data, stride, int(q), int(M),
                           codes, T, ov)
    return codes, T, ov


def legacy_decode(codes, T, q, M, beta, alpha=1.0, dither=None):
    """functional.py:119-181 per 8-vector: [N, 8]."""
    codes = np.ascontiguousarray(codes, np.int32).reshape(-1, M, 8)
    n = codes.shape[0]
    T = np.ascontiguousarray(T, np.int32).reshape(-1)
    out = np.empty((n, 8), np.float32)
    d = None if dither is None else _f32(dither)
    stride = 0 if d is None or d.size == 8 else 8
    lib().or_legacy_decode(codes, T, n, float(np.float32(beta)), legacy_scale_table(alpha),
                           None if d is None else d.ctypes.data, stride, int(q), int(M), out)
    return out


# ---------------------------------------------------------------- D4

def d4_g_x(x):
    """coset/core/d4/lattice.py:62-111 on [N, 4] rows."""
    x = _f32(x).reshape(-1, 4)
    out = np.empty_like(x)
    for i in range(x.shape[0]):
        row = np.empty(4, np.float32)
        lib().or_d4_g_x(np.ascontiguousarray(x[i]), row)
        out[i] = row
    return out


def d4_projection(x):
    """coset/core/d4/lattice.py:113-146 on [N, 4] rows."""
    x = _f32(x).reshape(-1, 4)
    y = np.empty_like(x)
    lib().or_d4_projection(x, x.shape[0], y)
    return y


def d4_encode_coords(y, q):
    y = _f32(y).reshape(-1, 4)
    b = np.empty(y.shape, np.int32)
    lib().or_d4_encode_coords(y, y.shape[0], int(q), b)
    return b


def d4_decode_coords(b):
    b = np.ascontiguousarray(b, dtype=np.int32).reshape(-1, 4)
    y = np.empty(b.shape, np.float32)
    lib().or_d4_decode_coords(b, b.shape[0], y)
    return y


def d4_layer_quant(W, beta, blocks_per_tile, clip):
    """coset/core/layers.py:428-463 with the D4 quantizer (d4/layers.py:46-47)."""
    W = _f32(W)
    rows, cols = W.shape
    Wq = np.empty_like(W)
    lib().or_d4_layer_quant(W, rows, cols, _f32(beta).reshape(-1), int(blocks_per_tile), float(clip), Wq)
    return Wq
