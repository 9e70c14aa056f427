"""QAT layer with the reference interface on the MI355X kernels.

Mirrors coset/core/layers.py (StraightThroughQuantize 62-95, ste_quantize
98-110, LSQActivation 117-137, HNLQConfig 141-163, HNLQLinearQAT 166-658,
HNLQLinear 662) and the factory coset/core/e8/layers.py:15-66.

When the injected ``quantize_fn`` is this package's ``e8_quantize`` (what the
factory injects), the weight path theta -> beta bounds -> scale -> STE
quantize -> unscale -> clamp (and the step counter) runs as one HIP kernel
forward (coset_e8_qat_fwd_theta) and one backward (coset_e8_qat_bwd_theta)
that re-decodes the saved packed codes and returns dW and dtheta; the dense
products go to hipBLASLt through F.linear.  Any other injected quantizer
runs the reference composition around it.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .codecs import e8_quantize, word_dtype
from .lattice import D4Lattice, E8Lattice, d4_quantize, default_device, on_gpu


def ste_round(x):
    """Straight-through rounding (coset/core/layers.py:20-22)."""
    return (x - x.detach()) + torch.round(x).detach()


def ste_clip(x, min_val, max_val):
    """Straight-through clipping (coset/core/layers.py:24-26)."""
    return (x - x.detach()) + torch.clamp(x, min_val, max_val).detach()


def get_generators(lattice) -> Tuple[torch.Tensor, torch.Tensor]:
    """coset/core/layers.py:29-52."""
    return lattice.get_generators()


class StraightThroughQuantize(torch.autograd.Function):
    """Forward quantizes with the injected function, backward is the identity
    (coset/core/layers.py:62-95)."""

    @staticmethod
    def forward(ctx, x, quantize_fn, q):
        ctx.quantize_fn = quantize_fn
        ctx.q = q
        return quantize_fn(x, q=q)

    @staticmethod
    def backward(ctx, grad_output):
        return grad_output, None, None


def ste_quantize(x, quantize_fn, q):
    """coset/core/layers.py:98-110."""
    return StraightThroughQuantize.apply(x, quantize_fn, q)


class _LSQFunction(torch.autograd.Function):
    """LSQActivation's forward and its autograd as two fused kernels
    (coset_lsq_fwd / coset_lsq_bwd): the value and the gradients of
    coset/core/layers.py:129-137, computed in fp32 on the GPU."""

    @staticmethod
    def forward(ctx, x, alpha, qmax):
        xg = x.contiguous()
        a = alpha.detach().to(torch.float32).reshape(1).contiguous()
        out = torch.empty_like(xg)
        _lib.call("coset_lsq_fwd", _lib.ptr(xg), _lib.dtype_code(xg.dtype), xg.numel(), _lib.ptr(a), int(qmax),
                  _lib.ptr(out), _lib.stream_of(xg))
        ctx.save_for_backward(xg, a)
        ctx.qmax = int(qmax)
        ctx.alpha_meta = (alpha.shape, alpha.dtype)
        return out

    @staticmethod
    def backward(ctx, grad):
        xg, a = ctx.saved_tensors
        g = grad.to(xg.dtype).contiguous()
        dx = torch.empty_like(xg)
        d_alpha = torch.empty(1, dtype=torch.float32, device=xg.device)
        ws = torch.empty(max(1, _lib.load().coset_lsq_workspace_floats(xg.numel())), dtype=torch.float32,
                         device=xg.device)
        _lib.call("coset_lsq_bwd", _lib.ptr(xg), _lib.ptr(g), _lib.dtype_code(xg.dtype), xg.numel(), _lib.ptr(a),
                  ctx.qmax, _lib.ptr(dx), _lib.ptr(d_alpha), _lib.ptr(ws), ws.numel(), _lib.stream_of(xg))
        shape, dtype = ctx.alpha_meta
        return dx, d_alpha.reshape(shape).to(dtype), None


class LSQActivation(nn.Module):
    """Learnable per-tensor symmetric activation quantizer
    (coset/core/layers.py:117-137): out = round(clamp(x, -a, a) / s) * s with
    a = relu(alpha) + 1e-8, s = a / qmax, straight-through gradients to x and
    alpha.  One fused kernel each way (fp32 arithmetic in the reference's
    order, the result written in x's dtype); host tensors are processed on the
    GPU and returned on the host."""

    def __init__(self, bit_width: int = 8, init_alpha: float = 1.0):
        super().__init__()
        self.bit_width = bit_width
        self.qmax = 2 ** (bit_width - 1) - 1
        self.alpha = nn.Parameter(torch.tensor(init_alpha))

    def forward(self, x):
        home = x.device
        xg = on_gpu(x)
        if xg.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            xg = xg.float()
        alpha = self.alpha if self.alpha.device == xg.device else self.alpha.to(xg.device)
        out = _LSQFunction.apply(xg, alpha, self.qmax)
        return out if out.device == home else out.to(home)


@dataclass
class HNLQConfig:
    """coset/core/layers.py:141-163 (kept for API parity; the layer takes
    keyword arguments)."""
    q: int = 4
    M: int = 2
    Delta0: float = 1.5
    eta: float = 0.1
    k: int = 1
    tiling: str = "row"
    block_size: int = 8
    quantize_activations: bool = False
    act_bit_width: int = 8
    act_init_alpha: float = 1.0
    init_method: str = "normal"
    init_kwargs: Dict[str, Any] = None

    def __post_init__(self):
        if self.init_kwargs is None:
            self.init_kwargs = {}
        if self.tiling not in ["row", "block"]:
            raise ValueError(f"tiling must be 'row' or 'block', got {self.tiling}")
        if self.block_size <= 0:
            raise ValueError(f"block_size must be positive, got {self.block_size}")


class E8WeightQuant(torch.autograd.Function):
    """W -> clamp(Q(W * beta_t) / beta_t, +-clip) with the straight-through
    gradient, on the HIP kernels.  beta has one entry per tile of
    ``blocks_per_tile`` 8-wide blocks (row tiling: one per output row)."""

    @staticmethod
    def forward(ctx, W, beta, q, M, clip, blocks_per_tile, out_dtype):
        Wc = W.detach().contiguous()
        if Wc.dtype != torch.float32:
            raise ValueError("HNLQ weights must be float32")
        b = beta.detach().contiguous()
        rows, cols = Wc.shape
        n = rows * (cols // 8)
        Wq = torch.empty((rows, cols), dtype=out_dtype, device=Wc.device)
        packed = torch.empty((n, M), dtype=word_dtype(q), device=Wc.device)
        _lib.call("coset_e8_qat_fwd", _lib.ptr(Wc), rows, cols, _lib.ptr(b), int(blocks_per_tile),
                  float(clip), int(q), int(M), _lib.ptr(Wq), _lib.dtype_code(out_dtype),
                  _lib.ptr(packed), _lib.stream_of(Wc))
        ctx.save_for_backward(Wc, b, packed)
        ctx.cfg = (q, M, float(clip), int(blocks_per_tile), beta.shape)
        return Wq

    @staticmethod
    def backward(ctx, g):
        Wc, b, packed = ctx.saved_tensors
        q, M, clip, bpt, beta_shape = ctx.cfg
        if g.dtype not in (torch.float32, torch.bfloat16):
            g = g.float()
        g = g.contiguous()
        rows, cols = Wc.shape
        dW = torch.empty_like(Wc)
        dbeta = torch.empty(b.numel(), dtype=torch.float32, device=Wc.device)
        _lib.call("coset_e8_qat_bwd", _lib.ptr(g), _lib.dtype_code(g.dtype), _lib.ptr(Wc),
                  _lib.ptr(packed), _lib.ptr(b), rows, cols, bpt, clip, int(q), int(M),
                  _lib.ptr(dW), _lib.ptr(dbeta), _lib.stream_of(Wc))
        return dW, dbeta.view(beta_shape), None, None, None, None, None


def qat_fwd_theta(Wc, theta, sigma, xmax, step_count, bounds, q, M, clip, blocks_per_tile, out_dtype, bias=None):
    """One coset_e8_qat_fwd_theta call: (W_q [rows, cols] in out_dtype,
    level words [rows * cols / 8, M], beta [tiles], d beta / d theta [tiles],
    and, given an fp32 bias [rows], that bias in out_dtype from the same
    launch, else None)."""
    th = theta.contiguous()
    rows, cols = Wc.shape
    dev = Wc.device
    Wq = torch.empty((rows, cols), dtype=out_dtype, device=dev)
    packed = torch.empty((rows * (cols // 8), M), dtype=word_dtype(q), device=dev)
    beta = torch.empty(th.numel(), dtype=torch.float32, device=dev)
    dbdt = torch.empty_like(beta)
    b_in = b_out = None
    if bias is not None:
        b_in = bias.detach().float().contiguous()
        if b_in.numel() != rows:
            raise ValueError(f"bias must hold {rows} values")
        b_out = torch.empty(rows, dtype=out_dtype, device=dev)
    delta0, eta, ginv, m_bounds = bounds
    _lib.check("coset_e8_qat_fwd_theta", _lib.fn("coset_e8_qat_fwd_theta")(
        Wc.data_ptr(), rows, cols, blocks_per_tile, th.data_ptr(), sigma.contiguous().data_ptr(),
        xmax.contiguous().data_ptr(), delta0, eta, ginv, m_bounds, clip, q, M, Wq.data_ptr(),
        _lib.dtype_code(out_dtype), packed.data_ptr(), beta.data_ptr(), dbdt.data_ptr(),
        _lib.ptr(step_count), _lib.ptr(b_in), _lib.ptr(b_out), _lib.stream_of(Wc)))
    return Wq, packed, beta, dbdt, b_out


class E8ThetaWeightQuant(torch.autograd.Function):
    """The fused QAT weight path: beta from theta and the EMA buffers, scale,
    quantize (M = 2), unscale, clamp and the step counter in one kernel
    (coset_e8_qat_fwd_theta); the backward returns dW and dtheta from one
    kernel (coset_e8_qat_bwd_theta).  The forward records beta and
    d beta / d theta per tile, so later in-place updates of the EMA buffers
    do not affect this step's gradient."""

    @staticmethod
    def forward(ctx, W, theta, sigma, xmax, step_count, bounds, q, M, clip, blocks_per_tile, out_dtype, bias=None):
        Wc = W.detach().contiguous()
        Wq, packed, beta, dbdt, b_cast = qat_fwd_theta(Wc, theta.detach(), sigma, xmax, step_count, bounds, q, M,
                                                       clip, blocks_per_tile, out_dtype, bias)
        ctx.save_for_backward(Wc, packed, beta, dbdt)
        ctx.cfg = (q, M, clip, blocks_per_tile, theta.shape)
        if b_cast is None:
            return Wq
        # the bias in the product's dtype rides along, not differentiable here:
        # its gradient reaches the fp32 bias through QATLinearFn.  Unused
        # gradients stay None (autograd would otherwise fill a zero tensor
        # for b_cast on every backward: one more launch per step)
        ctx.mark_non_differentiable(b_cast)
        ctx.set_materialize_grads(False)
        return Wq, b_cast

    @staticmethod
    def backward(ctx, g, g_bias=None):
        if g is None:
            return (None,) * 12
        Wc, packed, beta, dbdt = ctx.saved_tensors
        q, M, clip, bpt, theta_shape = ctx.cfg
        if g.dtype not in (torch.float32, torch.bfloat16):
            g = g.float()
        g = g.contiguous()
        rows, cols = Wc.shape
        dW = torch.empty_like(Wc)
        dbeta = torch.empty_like(beta)
        dtheta = torch.empty_like(beta)
        _lib.check("coset_e8_qat_bwd_theta", _lib.fn("coset_e8_qat_bwd_theta")(
            g.data_ptr(), _lib.dtype_code(g.dtype), Wc.data_ptr(), packed.data_ptr(), beta.data_ptr(),
            dbdt.data_ptr(), rows, cols, bpt, clip, q, M, dW.data_ptr(), dbeta.data_ptr(), dtheta.data_ptr(),
            _lib.stream_of(Wc)))
        return dW, dtheta.view(theta_shape), None, None, None, None, None, None, None, None, None, None


def d4_qat_fwd_theta(Wc, theta, sigma, xmax, step_count, bounds, q, clip, blocks_per_tile, out_dtype):
    """One coset_d4_qat_fwd_theta call: (W_q [rows, cols] in out_dtype,
    beta [tiles], d beta / d theta [tiles])."""
    th = theta.contiguous()
    rows, cols = Wc.shape
    dev = Wc.device
    Wq = torch.empty((rows, cols), dtype=out_dtype, device=dev)
    beta = torch.empty(th.numel(), dtype=torch.float32, device=dev)
    dbdt = torch.empty_like(beta)
    delta0, eta, ginv, m_bounds = bounds
    _lib.check("coset_d4_qat_fwd_theta", _lib.fn("coset_d4_qat_fwd_theta")(
        Wc.data_ptr(), rows, cols, blocks_per_tile, th.data_ptr(), sigma.contiguous().data_ptr(),
        xmax.contiguous().data_ptr(), delta0, eta, ginv, q, m_bounds, clip, Wq.data_ptr(),
        _lib.dtype_code(out_dtype), beta.data_ptr(), dbdt.data_ptr(), _lib.ptr(step_count), _lib.stream_of(Wc)))
    return Wq, beta, dbdt


class D4ThetaWeightQuant(torch.autograd.Function):
    """The D4 layer's fused weight path (coset_d4_qat_fwd_theta /
    coset_d4_qat_bwd): beta from theta, scale, D4 projection, unscale, clamp
    and the step counter in one kernel; the backward recomputes the
    projection and returns dW and dtheta."""

    @staticmethod
    def forward(ctx, W, theta, sigma, xmax, step_count, bounds, q, clip, blocks_per_tile, out_dtype):
        Wc = W.detach().contiguous()
        Wq, beta, dbdt = d4_qat_fwd_theta(Wc, theta.detach(), sigma, xmax, step_count, bounds, q, clip,
                                          blocks_per_tile, out_dtype)
        ctx.save_for_backward(Wc, beta, dbdt)
        ctx.cfg = (clip, blocks_per_tile, theta.shape)
        return Wq

    @staticmethod
    def backward(ctx, g):
        Wc, beta, dbdt = ctx.saved_tensors
        clip, bpt, theta_shape = ctx.cfg
        if g.dtype not in (torch.float32, torch.bfloat16):
            g = g.float()
        g = g.contiguous()
        rows, cols = Wc.shape
        dW = torch.empty_like(Wc)
        dbeta = torch.empty_like(beta)
        dtheta = torch.empty_like(beta)
        _lib.check("coset_d4_qat_bwd", _lib.fn("coset_d4_qat_bwd")(
            g.data_ptr(), _lib.dtype_code(g.dtype), Wc.data_ptr(), beta.data_ptr(), dbdt.data_ptr(), rows, cols,
            bpt, clip, dW.data_ptr(), dbeta.data_ptr(), dtheta.data_ptr(), _lib.stream_of(Wc)))
        return dW, dtheta.view(theta_shape), None, None, None, None, None, None, None, None


def _colsum_buffers(g2: torch.Tensor):
    """The output and workspace of colsum(g2), allocated on the current stream."""
    rows, cols = g2.shape
    out = torch.empty(cols, dtype=torch.float32, device=g2.device)
    need = int(_lib.load().coset_colsum_workspace_floats(rows, cols))
    ws = torch.empty(max(need, 1), dtype=torch.float32, device=g2.device)
    return out, ws


def _colsum_into(g2: torch.Tensor, out: torch.Tensor, ws: torch.Tensor) -> None:
    """coset_colsum of a contiguous g2 into out, on the current stream."""
    rows, cols = g2.shape
    dt = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}[g2.dtype]
    _lib.check("coset_colsum", _lib.fn("coset_colsum")(g2.data_ptr(), dt, rows, cols, out.data_ptr(), ws.data_ptr(),
                                                       ws.numel(), _lib.stream_of(g2)))


def colsum(g2: torch.Tensor) -> torch.Tensor:
    """sum over rows of a [rows, cols] fp32/bf16/fp16 tensor, accumulated in
    fp32 in a fixed order (coset_colsum): the bias gradient of a product."""
    g2 = g2.contiguous()
    out, ws = _colsum_buffers(g2)
    _colsum_into(g2, out, ws)
    return out


# 1: the weight gradient gy^T x runs on coset_gemm_tn where the shape and
# dtypes allow it (coset_gemm_tn_supported, bf16), 0: always on torch.mm
# (hipBLASLt)
_GEMM_TN = [1]
# 1: where coset_gemm_tn runs the weight gradient of a step, the bias
# gradient's column sums come from the same launch (workgroups of their own
# beside the product's tiles), so a step that forks its backward over two
# streams (CapturedQATStep) leaves only dX on the second stream; 0: from
# coset_colsum (beside dX on the second stream, or after dW on one stream)
_FUSE_BIAS_GRAD = [1]


def set_gemm_tn(enabled: bool) -> None:
    """Route the layer's weight-gradient product to coset_gemm_tn (default)
    or to torch.mm."""
    _GEMM_TN[0] = 1 if enabled else 0


def gemm_tn(a: torch.Tensor, b: torch.Tensor, out_dtype: Optional[torch.dtype] = None,
            colsum: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """a^T b for bf16 a [K, M] and b [K, N] on the GPU (coset_gemm_tn: fp32
    accumulation in a fixed order, output bf16 rounded to nearest even or
    fp32); colsum (optional fp32 [M]) also receives the column sums of a in
    the same pass.  None where the kernel does not take the shape or dtypes
    (colsum then untouched)."""
    if out_dtype is None:
        out_dtype = a.dtype
    if (a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16 or out_dtype not in (torch.bfloat16, torch.float32)
            or a.dim() != 2 or b.dim() != 2 or a.shape[0] != b.shape[0] or not a.is_cuda or b.device != a.device):
        return None
    K, M = a.shape
    N = b.shape[1]
    lib = _lib.load()
    if not lib.coset_gemm_tn_supported(M, N, K):
        return None
    if colsum is not None and (colsum.dtype != torch.float32 or colsum.numel() != M or not colsum.is_contiguous()):
        raise ValueError("colsum must be a contiguous fp32 tensor of M elements")
    a = a.contiguous()
    b = b.contiguous()
    out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    need = int(lib.coset_gemm_tn_workspace_floats(M, N, K))
    ws = torch.empty(max(need, 4), dtype=torch.float32, device=a.device)
    _lib.check("coset_gemm_tn", lib.coset_gemm_tn(a.data_ptr(), M, b.data_ptr(), N, out.data_ptr(), N,
                                                 _lib.BF16 if out_dtype == torch.bfloat16 else _lib.F32, M, N, K,
                                                 0 if colsum is None else colsum.data_ptr(), ws.data_ptr(), need,
                                                 _lib.stream_of(a)))
    return out


def _gemm_tn_takes(g2: torch.Tensor, x2: torch.Tensor) -> bool:
    """Whether _weight_grad runs g2^T x2 on coset_gemm_tn."""
    return (_GEMM_TN[0] == 1 and g2.is_cuda and g2.dtype == x2.dtype == torch.bfloat16 and g2.dim() == 2
            and x2.dim() == 2 and g2.shape[0] == x2.shape[0]
            and bool(_lib.load().coset_gemm_tn_supported(g2.shape[1], x2.shape[1], g2.shape[0])))


def _weight_grad(g2: torch.Tensor, x2: torch.Tensor, colsum: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dW_q = g2^T x2: coset_gemm_tn where it applies (with colsum: also the
    fp32 column sums of g2, the bias gradient, in the same pass), else
    torch.mm (colsum must then be None)."""
    if _gemm_tn_takes(g2, x2):
        out = gemm_tn(g2, x2, colsum=colsum)
        if out is not None:
            return out
    if colsum is not None:
        raise RuntimeError("column sums requested where coset_gemm_tn does not run")
    return g2.t() @ x2


# 1: no-grad forwards of small fp32 batches run as one fused launch
# (coset_e8_qat_head_fwd); 0: the quantizer and F.linear as two launches
_HEAD_FWD = [1]


def set_head_forward(enabled: bool) -> None:
    """Run no-grad forwards of up to 64 fp32 tokens as one launch (default)
    or as the quantizer followed by F.linear."""
    _HEAD_FWD[0] = 1 if enabled else 0


_AUX_STREAMS: Dict[int, "torch.cuda.Stream"] = {}
# > 0 while CapturedQATStep warms up and captures: the backward then forks
# its independent products onto a second stream (graph branches).  Eager
# steps stay on one stream, where the host's launch time is the limit and
# the fork and join would only add to it.
_OVERLAP_BACKWARD = [0]


def _aux_stream(device: torch.device) -> "torch.cuda.Stream":
    """A second stream per device (default priority) for the backward's
    products that do not depend on each other."""
    s = _AUX_STREAMS.get(device.index)
    if s is None:
        s = _AUX_STREAMS[device.index] = torch.cuda.Stream(device=device)
    return s


class QATLinearFn(torch.autograd.Function):
    """y = x W_q^T + b, the layer's F.linear (coset/core/layers.py:478): the
    weight gradient runs on coset_gemm_tn where it applies (bf16), with the
    bias gradient's column sums in the same pass, the other products on
    hipBLASLt (torch.mm); elsewhere the bias gradient is the fp32 column sum
    of the output gradient (coset_colsum).  Either way a bf16 layer's fp32
    bias gets an fp32 sum of its gradient, not a reduction in bf16."""

    @staticmethod
    def forward(ctx, x, Wq, bias, bias_cast=None):
        """bias_cast (optional): bias already in x's dtype (the fused
        quantizer writes it); the gradient still goes to bias."""
        ctx.save_for_backward(x, Wq)
        ctx.bias_dtype = None if bias is None else bias.dtype
        if bias is not None and bias_cast is None:
            bias_cast = bias.to(x.dtype)
        return F.linear(x, Wq, bias_cast)

    @staticmethod
    def backward(ctx, gy):
        x, Wq = ctx.saved_tensors
        g2 = gy.reshape(-1, gy.shape[-1])
        dx = dW = db = None
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        fast_db = (ctx.bias_dtype is not None and ctx.needs_input_grad[2] and g2.shape[1] % 8 == 0
                   and g2.dtype in (torch.float32, torch.bfloat16, torch.float16))
        overlap = g2.is_cuda and (_OVERLAP_BACKWARD[0] > 0 or torch.cuda.is_current_stream_capturing())
        x2 = x.reshape(-1, x.shape[-1])
        if overlap and need_dw and (need_dx or fast_db) and g2.dtype == Wq.dtype == x.dtype:
            # dX (and the bias gradient where coset_gemm_tn does not take it)
            # on a second stream while dW runs on this one: the dW product
            # alone leaves CUs idle at these shapes (one 64 x 64 or 128 x 128
            # tile per CU or fewer).  Outputs are allocated here, on the
            # current stream, before the fork; the join comes before they are
            # returned.  Under graph capture the two streams become two
            # branches of the graph.
            g2 = g2.contiguous()
            fuse = (_FUSE_BIAS_GRAD[0] == 1 and fast_db and g2.dtype == torch.bfloat16
                    and _gemm_tn_takes(g2, x2))
            main = torch.cuda.current_stream(g2.device)
            aux = _aux_stream(g2.device)
            dx2 = torch.empty((g2.shape[0], Wq.shape[1]), dtype=g2.dtype, device=g2.device) if need_dx else None
            cs = _colsum_buffers(g2) if fast_db and not fuse else None
            dbf = torch.empty(g2.shape[1], dtype=torch.float32, device=g2.device) if fuse else None
            aux.wait_stream(main)
            with torch.cuda.stream(aux):
                if need_dx:
                    torch.mm(g2, Wq, out=dx2)
                if cs is not None:
                    _colsum_into(g2, *cs)
            dW = _weight_grad(g2, x2, colsum=dbf)
            main.wait_stream(aux)
            if need_dx:
                dx = dx2.reshape(x.shape)
            if fast_db:
                db = (dbf if fuse else cs[0]).to(ctx.bias_dtype)
            elif ctx.bias_dtype is not None and ctx.needs_input_grad[2]:
                db = g2.float().sum(0).to(ctx.bias_dtype)
            return dx, dW, db, None
        # one stream: the bias gradient in the weight-gradient kernel's pass
        # where that kernel runs (bf16), the column sums of gy with gy^T x
        if (_FUSE_BIAS_GRAD[0] == 1 and fast_db and need_dw and g2.dtype == torch.bfloat16 and g2.is_contiguous()
                and _gemm_tn_takes(g2, x2)):
            dbf = torch.empty(g2.shape[1], dtype=torch.float32, device=g2.device)
            dW = _weight_grad(g2, x2, colsum=dbf)
            db = dbf.to(ctx.bias_dtype)
            if need_dx:
                dx = (g2 @ Wq).reshape(x.shape)
            return dx, dW, db, None
        if ctx.needs_input_grad[0]:
            dx = (g2 @ Wq).reshape(x.shape)
        if ctx.needs_input_grad[1]:
            dW = _weight_grad(g2, x.reshape(-1, x.shape[-1]))
        if ctx.bias_dtype is not None and ctx.needs_input_grad[2]:
            if g2.shape[1] % 8 == 0 and g2.dtype in (torch.float32, torch.bfloat16, torch.float16):
                db = colsum(g2).to(ctx.bias_dtype)
            else:
                db = g2.float().sum(0).to(ctx.bias_dtype)
        return dx, dW, db, None


class HNLQLinearQAT(nn.Module):
    """Hierarchical nested-lattice quantized linear layer with QAT cold start
    (coset/core/layers.py:166-658); same constructor, buffers, state_dict
    keys and methods."""

    def __init__(self, in_features: int, out_features: int, lattice, quantize_fn, q: int = 4, M: int = 2,
                 Delta0: Optional[float] = None, eta: float = 0.1, tiling: str = "row", block_size: int = 8,
                 quantize_activations: bool = False, act_bit_width: int = 8, act_init_alpha: float = 1.0,
                 init_method: str = "normal", init_kwargs: Optional[Dict[str, Any]] = None, bias: bool = True,
                 warmup_epochs: int = 0, enable_diagnostics: bool = False, weight_clip_value: float = 2.0,
                 theta_trainable: bool = True, theta_init_value: float = 0.0, rho: float = 0.95):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.quantize_fn = quantize_fn
        self.lattice = lattice
        self.lattice_type = lattice.name
        self.q = q
        self.M = M
        self.eta = eta
        self.tiling = tiling
        self.block_size = block_size
        self.quantize_activations = quantize_activations
        self.init_method = init_method
        self.init_kwargs = init_kwargs or {}
        self.theta_trainable = theta_trainable
        self.theta_init_value = theta_init_value
        self.rho = rho
        self.Delta0 = lattice.compute_delta0(q, M, rho) if Delta0 is None else Delta0

        device = lattice.G.device
        G, Ginv = lattice.get_generators()
        self.register_buffer("G", G)
        self.register_buffer("Ginv", Ginv)

        self.blocks_per_row = in_features // block_size
        if in_features % block_size != 0:
            raise ValueError(f"Input dimension {in_features} must be divisible by block_size {block_size}")

        self.weight = nn.Parameter(torch.empty(out_features, in_features, device=device))
        self._initialize_weights()
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, device=device))
        else:
            self.register_parameter("bias", None)

        tiles = out_features if tiling == "row" else out_features * (in_features // block_size)
        theta0 = torch.full((tiles,), theta_init_value, device=device)
        if theta_trainable:
            self.theta_beta = nn.Parameter(theta0)
        else:
            self.register_buffer("theta_beta", theta0)
        self.register_buffer("sigma_ema", torch.ones(tiles, device=device))
        self.register_buffer("xmax_ema", torch.ones(tiles, device=device))
        self.ema_momentum = 0.99
        self.stat_update_interval = 256
        self.register_buffer("step_count", torch.tensor(0, dtype=torch.long, device=device))
        self.register_buffer("gamma_inv", Ginv.abs().sum(dim=1).max())
        # host mirrors of buffers the forward reads every step (no device sync)
        self._host_step: Optional[int] = None
        self._ginv_f: float = float(self.gamma_inv)

        self.actq = LSQActivation(bit_width=act_bit_width, init_alpha=act_init_alpha) if quantize_activations else None
        self.warmup_epochs = warmup_epochs
        self.current_epoch = 0
        self.quantization_enabled = warmup_epochs == 0
        self.enable_diagnostics = enable_diagnostics
        self.weight_clip_value = weight_clip_value
        self._weight_history = [] if enable_diagnostics else None
        self._quantization_errors = [] if enable_diagnostics else None

    # ------------------------------------------------------------------
    def _initialize_weights(self):
        """coset/core/layers.py:314-330 (normal_ with no kwargs is N(0, 1))."""
        m = self.init_method
        if m == "normal":
            nn.init.normal_(self.weight, **self.init_kwargs)
        elif m == "xavier":
            nn.init.xavier_normal_(self.weight, **self.init_kwargs)
        elif m == "kaiming":
            nn.init.kaiming_normal_(self.weight, **self.init_kwargs)
        elif m == "zeros":
            nn.init.zeros_(self.weight)
        elif m == "ones":
            nn.init.ones_(self.weight)
        elif m == "load":
            pass
        else:
            raise ValueError(f"Unknown init_method: {m}")

    def load_weights(self, weight: torch.Tensor, bias: Optional[torch.Tensor] = None):
        if weight.shape != (self.out_features, self.in_features):
            raise ValueError(f"Weight shape {weight.shape} doesn't match expected {(self.out_features, self.in_features)}")
        self.weight.data = weight.clone().to(self.weight.device, self.weight.dtype)
        if bias is not None:
            if self.bias is None:
                raise ValueError("Cannot load bias: layer was initialized with bias=False")
            if bias.shape != (self.out_features,):
                raise ValueError(f"Bias shape {bias.shape} doesn't match expected {(self.out_features,)}")
            self.bias.data = bias.clone().to(self.bias.device, self.bias.dtype)

    def load_from_linear(self, linear_layer: nn.Linear):
        if linear_layer.in_features != self.in_features:
            raise ValueError(f"Input features mismatch: {linear_layer.in_features} vs {self.in_features}")
        if linear_layer.out_features != self.out_features:
            raise ValueError(f"Output features mismatch: {linear_layer.out_features} vs {self.out_features}")
        self.load_weights(linear_layer.weight.data,
                          linear_layer.bias.data if linear_layer.bias is not None else None)

    def _load_from_state_dict(self, *args, **kwargs):
        super()._load_from_state_dict(*args, **kwargs)
        self._host_step = None
        self._ginv_f = float(self.gamma_inv)

    # ------------------------------------------------------------------
    def _gather_stats(self, W_blocks):
        """EMA of the unscaled weights' std and abs-max (layers.py:366-379).
        On the GPU one kernel (coset_qat_stats_update) computes both
        statistics and updates both buffers with the reference's CPU
        arithmetic (variance in double)."""
        if W_blocks.is_cuda and W_blocks.dtype == torch.float32 and self.sigma_ema.is_cuda:
            Wc = W_blocks.detach().contiguous()
            if self.tiling == "row":
                tiles, size = self.out_features, self.blocks_per_row * self.block_size
            else:
                tiles, size = self.out_features * self.blocks_per_row, self.block_size
            if self.sigma_ema.is_contiguous() and self.xmax_ema.is_contiguous() and size >= 2:
                _lib.check("coset_qat_stats_update", _lib.fn("coset_qat_stats_update")(
                    Wc.data_ptr(), tiles, size, float(self.ema_momentum), self.sigma_ema.data_ptr(),
                    self.xmax_ema.data_ptr(), _lib.stream_of(Wc)))
                return
        with torch.no_grad():
            m = self.ema_momentum
            if self.tiling == "row":
                sigma = W_blocks.std(dim=(1, 2)) + 1e-8
                xmax = W_blocks.abs().amax(dim=(1, 2)) + 1e-8
                self.sigma_ema[: self.out_features].mul_(m).add_((1 - m) * sigma)
                self.xmax_ema[: self.out_features].mul_(m).add_((1 - m) * xmax)
            else:
                sigma = W_blocks.std(dim=2).reshape(-1) + 1e-8
                xmax = W_blocks.abs().amax(dim=2).reshape(-1) + 1e-8
                self.sigma_ema.mul_(m).add_((1 - m) * sigma)
                self.xmax_ema.mul_(m).add_((1 - m) * xmax)

    def _bounds(self):
        """Adaptive beta bounds from the EMA statistics (layers.py:381-396)."""
        qM = float(self.q ** self.M)
        ginv = self._ginv_f
        beta_min = (self.Delta0 / qM) / (self.eta * ginv * self.sigma_ema)
        beta_max_det = (self.Delta0 * (qM - 1)) / (2 * ginv * self.xmax_ema)
        beta_max_prob = (self.Delta0 * (qM - 1)) / (2 * self.eta * ginv * self.sigma_ema)
        beta_max = torch.minimum(beta_max_det, beta_max_prob)
        beta_min = torch.minimum(beta_min, beta_max * 0.9)
        return beta_min, beta_max

    def _advance_step(self, device_increment: bool = True):
        """step_count += 1 and the every-256-steps statistics update
        (layers.py:408-413), with the counter mirrored on the host.  The
        fused kernel increments the device buffer itself."""
        if self._host_step is None:
            self._host_step = int(self.step_count)
        self._host_step += 1
        if device_increment:
            with torch.no_grad():
                self.step_count += 1
        if self._host_step % self.stat_update_interval == 0 and not (
                self.weight.is_cuda and torch.cuda.is_current_stream_capturing()):
            # under graph capture the statistics update stays out of the graph:
            # CapturedQATStep runs it eagerly before the replay that needs it
            self.gather_step_stats()

    def gather_step_stats(self):
        W = self.weight.view(self.out_features, self.blocks_per_row, self.block_size)
        self._gather_stats(W.detach())

    def _beta(self):
        beta_min, beta_max = self._bounds()
        if self.tiling == "row":
            theta = self.theta_beta[: self.out_features]
            return beta_min[: self.out_features] + torch.sigmoid(theta) * (
                beta_max[: self.out_features] - beta_min[: self.out_features])
        return beta_min + torch.sigmoid(self.theta_beta) * (beta_max - beta_min)

    def _fused(self) -> bool:
        return (self.quantize_fn is e8_quantize and self.block_size == 8
                and self.lattice_type == "E8" and self.weight.is_cuda)

    def _fused_d4(self) -> bool:
        return (self.quantize_fn is d4_quantize and self.block_size == 4
                and self.lattice_type == "D4" and self.weight.is_cuda)

    def _quantize_weights_as(self, out_dtype: torch.dtype):
        return self._quantize_weights_with_bias(out_dtype, False)[0]

    def _quantize_weights_with_bias(self, out_dtype: torch.dtype, cast_bias: bool):
        """(W_q in out_dtype, the bias in out_dtype written by the same fused
        launch when cast_bias and the fused E8 path runs, else None)."""
        W = self.weight
        if not self.quantization_enabled:
            if self.enable_diagnostics:
                self._weight_history.append(W.detach().clone())
            return W, None
        b_cast = None
        fused = self._fused()
        fused_d4 = self._fused_d4()
        self._advance_step(device_increment=not (fused or fused_d4))
        if fused_d4:
            bpt = self.blocks_per_row if self.tiling == "row" else 1
            W_q = D4ThetaWeightQuant.apply(W, self.theta_beta, self.sigma_ema, self.xmax_ema, self.step_count,
                                           (float(self.Delta0), float(self.eta), self._ginv_f, int(self.M)),
                                           int(self.q), float(self.weight_clip_value), int(bpt), out_dtype)
        elif fused:
            bpt = self.blocks_per_row if self.tiling == "row" else 1
            # one theta per tile: out_features entries for row tiling, so no slice is needed
            # the injected e8_quantize always encodes with M = 2 (codecs.py:245-254)
            out = E8ThetaWeightQuant.apply(W, self.theta_beta, self.sigma_ema, self.xmax_ema, self.step_count,
                                           (float(self.Delta0), float(self.eta), self._ginv_f, int(self.M)),
                                           int(self.q), 2, float(self.weight_clip_value), int(bpt), out_dtype,
                                           self.bias if cast_bias else None)
            W_q, b_cast = out if isinstance(out, tuple) else (out, None)
        else:
            W_q = self._reference_composition(W, self._beta()).to(out_dtype)
        if self.enable_diagnostics:
            self._weight_history.append(W.detach().clone())
            self._quantization_errors.append(torch.norm(W - W_q.float()).item())
        return W_q, b_cast

    def _reference_composition(self, W, beta):
        """layers.py:428-463 around an arbitrary injected quantize_fn."""
        if self.tiling == "row":
            beta = beta.view(-1, 1)
            W_scaled = W * beta
        else:
            beta = beta.view(self.out_features, self.blocks_per_row, 1)
            W_scaled = (W.view(self.out_features, self.blocks_per_row, self.block_size) * beta).reshape(
                self.out_features, self.in_features)
        flat = W_scaled.view(self.out_features, self.blocks_per_row, self.block_size).reshape(-1, self.block_size)
        Wq = ste_quantize(flat, self.quantize_fn, self.q).reshape(self.out_features, self.in_features)
        Wq = Wq / (beta if self.tiling == "row" else beta.reshape(self.out_features, -1).repeat_interleave(
            self.block_size, dim=1))
        return torch.clamp(Wq, -self.weight_clip_value, self.weight_clip_value)

    def _quantize_weights(self):
        """coset/core/layers.py:398-470 (fp32 W_q)."""
        return self._quantize_weights_as(torch.float32)

    def _head_takes(self, x) -> bool:
        """Whether forward() runs as one fused launch (coset_e8_qat_head_fwd):
        a no-grad forward of at most 64 fp32 tokens through the fused E8
        quantizer with row tiling and q = 2, 4."""
        if not (_HEAD_FWD[0] == 1 and x.is_cuda and x.dtype == torch.float32 and self.quantization_enabled
                and self._fused() and self.tiling == "row" and self.q in (2, 4) and not self.enable_diagnostics
                and x.shape[-1] == self.in_features and self.in_features <= 8192 and x.numel() > 0
                and x.numel() // self.in_features <= 64):
            return False
        params = (self.weight, self.theta_beta) + ((self.bias,) if self.bias is not None else ())
        return not torch.is_grad_enabled() or not (x.requires_grad or any(p.requires_grad for p in params))

    def _head_forward(self, x):
        """y = x W_q^T + bias with W_q quantized in the same launch."""
        self._advance_step(device_increment=False)   # the kernel increments step_count
        x2 = x.reshape(-1, self.in_features).contiguous()
        y = torch.empty((x2.shape[0], self.out_features), dtype=torch.float32, device=x.device)
        W = self.weight.detach().contiguous()
        _lib.call("coset_e8_qat_head_fwd", W.data_ptr(), self.out_features, self.in_features,
                  self.theta_beta.detach().contiguous().data_ptr(), self.sigma_ema.data_ptr(),
                  self.xmax_ema.data_ptr(), float(self.Delta0), float(self.eta), self._ginv_f, int(self.M),
                  float(self.weight_clip_value), int(self.q), x2.data_ptr(), x2.shape[0],
                  None if self.bias is None else self.bias.detach().data_ptr(), y.data_ptr(),
                  self.step_count.data_ptr(), _lib.stream_of(x2))
        y = y.reshape(*x.shape[:-1], self.out_features)
        if self.quantize_activations and self.actq is not None:
            y = self.actq(y)
        return y

    def forward(self, x):
        """F.linear(x, W_q, bias) (layers.py:472-484); W_q is produced in the
        activation dtype (float32 or bfloat16) for the GEMM.  No-grad forwards
        of up to 64 fp32 tokens run as one launch (quantizer and product)."""
        if self._head_takes(x):
            return self._head_forward(x)
        wdt = x.dtype if x.dtype in (torch.bfloat16, torch.float16) else torch.float32
        if wdt == torch.float16:
            wdt = torch.float32
        # a bf16 product takes the bias in bf16: the fused quantizer writes it
        # in the same launch as W_q
        cast_bias = x.is_cuda and self.bias is not None and wdt == torch.bfloat16 and x.dtype == wdt
        W_q, b_cast = self._quantize_weights_with_bias(wdt, cast_bias)
        if W_q.dtype != x.dtype:
            W_q = W_q.to(x.dtype)
        if x.is_cuda:
            x = QATLinearFn.apply(x, W_q, self.bias, b_cast)
        else:
            x = F.linear(x, W_q, self.bias.to(x.dtype) if self.bias is not None else None)
        if self.quantize_activations and self.actq is not None:
            x = self.actq(x)
        return x

    # cold start control (layers.py:487-506)
    def update_epoch(self, epoch: int):
        self.current_epoch = epoch
        if epoch >= self.warmup_epochs and not self.quantization_enabled:
            self.quantization_enabled = True
            print(f"Epoch {epoch}: Enabling quantization (warmup complete)")

    def enable_quantization(self):
        self.quantization_enabled = True
        print("Quantization manually enabled")

    def disable_quantization(self):
        self.quantization_enabled = False
        print("Quantization manually disabled")

    def is_quantization_enabled(self) -> bool:
        return self.quantization_enabled

    # diagnostics (layers.py:509-618)
    def get_weight_quantiles(self, quantiles: List[float] = None) -> torch.Tensor:
        if quantiles is None:
            quantiles = [0.0, 0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9, 1.0]
        W = self.weight.detach().flatten()
        return torch.quantile(W, torch.tensor(quantiles, device=W.device))

    def get_weight_statistics(self) -> Dict[str, float]:
        W = self.weight.detach()
        return {"mean": W.mean().item(), "std": W.std().item(), "min": W.min().item(), "max": W.max().item(),
                "median": W.median().item(), "l2_norm": torch.norm(W).item(), "l1_norm": torch.norm(W, p=1).item()}

    def get_quantization_error(self) -> float:
        if not self.quantization_enabled:
            return 0.0
        return torch.norm(self.weight.detach() - self._quantize_weights().detach()).item()

    def get_scaling_factors(self) -> torch.Tensor:
        return self.theta_beta.detach()

    def get_quantization_histogram(self, bins: int = 50):
        W = self.weight.detach() if not self.quantization_enabled else self._quantize_weights().detach()
        return torch.histogram(W.flatten().cpu(), bins=bins)

    def get_sparsity_ratio(self, threshold: float = 1e-6) -> float:
        return (self.weight.detach().abs() < threshold).float().mean().item()

    def get_effective_bits(self) -> float:
        if not self.quantization_enabled:
            return 32.0
        u = torch.unique(self._quantize_weights().detach())
        return torch.log2(torch.tensor(len(u), dtype=torch.float32)).item()

    def compare_weights(self) -> Dict[str, float]:
        if not self.quantization_enabled:
            return {"error": 0.0, "relative_error": 0.0, "cosine_similarity": 1.0}
        W = self.weight.detach()
        Wq = self._quantize_weights().detach()
        err = torch.norm(W - Wq).item()
        return {"error": err, "relative_error": err / torch.norm(W).item(),
                "cosine_similarity": F.cosine_similarity(W.flatten(), Wq.flatten(), dim=0).item()}

    def get_weight_clipping_stats(self) -> Dict[str, float]:
        W = self.weight.detach()
        clipped = torch.sum((W.abs() > self.weight_clip_value).float()).item()
        return {"clipping_ratio": clipped / W.numel(), "clipped_count": clipped, "total_count": W.numel(),
                "clip_value": self.weight_clip_value, "max_weight": W.abs().max().item()}

    def get_diagnostic_summary(self) -> Dict[str, Any]:
        s = {"epoch": self.current_epoch, "quantization_enabled": self.quantization_enabled,
             "warmup_epochs": self.warmup_epochs, "weight_stats": self.get_weight_statistics(),
             "quantization_error": self.get_quantization_error(), "effective_bits": self.get_effective_bits(),
             "sparsity_ratio": self.get_sparsity_ratio(), "weight_clipping": self.get_weight_clipping_stats()}
        if self.quantization_enabled:
            s["weight_comparison"] = self.compare_weights()
        return s

    def export_quantized(self):
        """layers.py:620-650, plus the packed level words and per-tile beta
        of the same quantization (keys 'codes', 'beta')."""
        with torch.no_grad():
            W_q = self._quantize_weights()
            metadata = {"lattice_type": self.lattice_type, "q": self.q, "M": self.M, "Delta0": self.Delta0,
                        "tiling": self.tiling, "block_size": self.block_size,
                        "quantize_activations": self.quantize_activations}
            if self.quantize_activations and self.actq is not None:
                metadata.update({"act_bit_width": self.actq.bit_width, "act_alpha": self.actq.alpha.item()})
            out = {"weight": W_q, "bias": self.bias, "metadata": metadata}
            if self._fused() and self.quantization_enabled:
                # the same quantization again, without advancing the step:
                # its level words and beta reproduce W_q bit for bit
                bpt = self.blocks_per_row if self.tiling == "row" else 1
                _, packed, beta, _, _ = qat_fwd_theta(
                    self.weight.detach().contiguous(), self.theta_beta.detach(), self.sigma_ema, self.xmax_ema,
                    None, (float(self.Delta0), float(self.eta), self._ginv_f, int(self.M)), int(self.q), 2,
                    float(self.weight_clip_value), int(bpt), torch.float32)
                out["codes"] = packed.view(self.out_features, self.blocks_per_row, 2)
                out["beta"] = beta
            return out

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"lattice_type={self.lattice_type}, q={self.q}, M={self.M}, "
                f"Delta0={self.Delta0:.4f}, tiling={self.tiling}, block_size={self.block_size}, "
                f"quantize_activations={self.quantize_activations}, bias={self.bias is not None}, "
                f"theta_trainable={self.theta_trainable}, theta_init_value={self.theta_init_value}, "
                f"rho={self.rho}")


HNLQLinear = HNLQLinearQAT


class CapturedQATStep:
    """One QAT layer step (forward, and backward when ``grad_output`` is
    given) captured once into a HIP graph and replayed by ``step()``.

    No counterpart in the reference, whose layer runs eagerly on the CPU.
    An eager step issues about fifteen small launches from Python (the fused
    quantizer, hipBLASLt's products, the backward and bias-gradient kernels),
    so at BERT shapes the host, not the GPU, sets its time; a replay issues
    them as one graph launch.

    Semantics per ``step()`` are those of an eager step preceded by
    ``layer.zero_grad(set_to_none=True)``: the gradients of the layer's
    parameters and of the static input are overwritten, not accumulated, and
    live in tensors owned by the graph; every ``step()`` binds them to
    ``param.grad`` (and ``x.grad``) again, so an optimizer loop that calls
    ``opt.zero_grad()`` (which sets them to None) before ``step()`` and
    ``opt.step()`` after it sees this step's gradients.  The graph reads the
    parameters' storage: in-place updates (optimizer steps,
    ``load_state_dict``) are seen by the next replay, while replacing a
    parameter's storage (``load_weights``, ``load_from_linear``,
    ``param.data = ...``) makes ``step()`` raise; capture again then.  The device step counter advances inside the graph (the fused
    kernel increments it); the host mirror of the counter and the
    every-``stat_update_interval``-steps EMA update of the weight statistics
    run eagerly, on the same stream, before the replay that reads them
    (coset/core/layers.py:408-413 updates them before the bounds).  The
    returned output is the graph's static tensor, overwritten by the next
    step.  A change of ``quantization_enabled`` (warm-up epochs) needs a new
    capture; ``step()`` raises instead of replaying a stale graph.  The
    warm-up runs that torch needs before capture leave the layer's buffers
    and counters as they were.

    ``tune_gemms=True`` also captures the step with the dense products
    (forward and input gradient; the weight gradient is the library's own
    kernel) chosen by PyTorch-ROCm's TunableOp (``torch.cuda.tunable``: each
    product shape benchmarked over the hipBLASLt and rocBLAS solutions during
    the warm-up), times a few replays of both graphs and keeps TunableOp's
    where it is at least 1 % faster, else the default one (``gemm_selection``:
    "default" or "tunableop"; ``tune_us``: the timed replay of each).  A product that is fastest alone is not always fastest
    in the step, where the weight gradient runs beside it, hence the timing
    of whole replays.  TunableOp's enable and tuning flags are restored
    afterwards; its table of tuned shapes stays in the process.  Products of
    other solutions round differently: the step's output and input gradient
    then match an eager step to the products' rounding, not bit for bit.
    """

    def __init__(self, layer: HNLQLinearQAT, x: torch.Tensor, grad_output: Optional[torch.Tensor] = None,
                 warmup: int = 3, tune_gemms: bool = False):
        if not x.is_cuda or not layer.weight.is_cuda:
            raise ValueError("CapturedQATStep needs the layer and its input on a GPU")
        if layer.enable_diagnostics:
            raise ValueError("CapturedQATStep: diagnostics read values back to the host on every step")
        self.layer = layer
        self.x = x
        self.grad_output = grad_output
        self._mode = layer.quantization_enabled
        if layer._host_step is None:
            layer._host_step = int(layer.step_count)
        host_step = layer._host_step
        saved = {name: b.clone() for name, b in layer.named_buffers()}

        _OVERLAP_BACKWARD[0] += 1   # warm-up and capture take the same (two-stream) backward
        try:
            cands = [self._capture(warmup, saved, False)]
            if tune_gemms:
                cands.append(self._capture(warmup, saved, True))
        finally:
            _OVERLAP_BACKWARD[0] -= 1
        self.gemm_selection = "default"
        self.tune_us = None
        best = 0
        if len(cands) > 1:
            times = self._time_replays([c[0] for c in cands], saved)
            self.tune_us = {"default": round(times[0], 2), "tunableop": round(times[1], 2)}
            best = 1 if times[1] < 0.99 * times[0] else 0   # ties keep the eager step's own products
            self.gemm_selection = ("default", "tunableop")[best]
        self.graph, self.y, self._grads, self._x_grad = cands[best]
        del cands
        layer._host_step = host_step
        # the winner's gradient tensors are the parameters' (and the input's) grads
        for p, g in self._grads:
            p.grad = g
        if self._x_grad is not None:
            self.x.grad = self._x_grad
        self._storage = self._param_ptrs()

    def _restore_buffers(self, saved):
        with torch.no_grad():
            for name, b in self.layer.named_buffers():
                b.copy_(saved[name])

    def _capture(self, warmup, saved, tuned):
        """Warm-up steps on a side stream (with ``tuned``: under TunableOp,
        tuning each new product shape), the layer's buffers restored, then
        the capture.  Returns the graph, its output, the (parameter, grad)
        pairs and the input's grad it writes."""
        x = self.x
        tun = torch.cuda.tunable
        prev = (tun.is_enabled(), tun.tuning_is_enabled()) if tuned else None
        try:
            if tuned:
                tun.enable(True)
                tun.tuning_enable(True)
            side = torch.cuda.Stream(device=x.device)
            side.wait_stream(torch.cuda.current_stream(x.device))
            with torch.cuda.stream(side):
                for _ in range(max(1, int(warmup))):
                    self._zero_grads()
                    self._run()
            torch.cuda.current_stream(x.device).wait_stream(side)
            self._restore_buffers(saved)
            self._zero_grads()
            if tuned:
                tun.tuning_enable(False)   # the capture only looks the tuned solutions up
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                y = self._run()
        finally:
            if tuned:
                tun.tuning_enable(prev[1])
                tun.enable(prev[0])
        grads = [(p, p.grad) for p in self.layer.parameters() if p.grad is not None]
        return graph, y, grads, (x.grad if x.requires_grad else None)

    def _time_replays(self, graphs, saved, rounds: int = 9, reps: int = 10):
        """Median time (us) of one replay of each graph, the graphs timed in
        turn after a few untimed replays each; the layer's buffers (the device
        step counter among them) are restored afterwards."""
        stream = torch.cuda.current_stream(self.x.device)
        for g in graphs:
            for _ in range(reps):
                g.replay()
        ts = [[] for _ in graphs]
        for _ in range(rounds):
            for k, g in enumerate(graphs):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(reps):
                    g.replay()
                e1.record(stream)
                e1.synchronize()
                ts[k].append(e0.elapsed_time(e1) * 1e3 / reps)
        self._restore_buffers(saved)
        stream.synchronize()
        return [sorted(t)[len(t) // 2] for t in ts]

    def _param_ptrs(self):
        return [(name, p.data_ptr()) for name, p in self.layer.named_parameters()]

    def _zero_grads(self):
        self.layer.zero_grad(set_to_none=True)
        if self.x.requires_grad:
            self.x.grad = None

    def _run(self):
        if self.grad_output is None:
            with torch.no_grad():
                return self.layer(self.x)
        y = self.layer(self.x)
        y.backward(self.grad_output)
        return y.detach()

    def step(self, x: Optional[torch.Tensor] = None, grad_output: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Replay the step, after copying new values (if given) into the
        static input and output-gradient tensors."""
        L = self.layer
        if L.quantization_enabled != self._mode:
            raise RuntimeError("CapturedQATStep: quantization was switched since the capture; capture again")
        if grad_output is not None and self.grad_output is None:
            raise ValueError("CapturedQATStep: captured without a backward")
        if self._param_ptrs() != self._storage:
            raise RuntimeError("CapturedQATStep: a parameter's storage was replaced since the capture "
                               "(load_weights / load_from_linear / .data assignment); capture again")
        with torch.no_grad():
            if x is not None:
                self.x.copy_(x)
            if grad_output is not None:
                self.grad_output.copy_(grad_output)
        if self._mode:
            if L._host_step is None:       # after load_state_dict: mirror the loaded counter once
                L._host_step = int(L.step_count)
            L._host_step += 1
            if L._host_step % L.stat_update_interval == 0:
                L.gather_step_stats()
        self.graph.replay()
        for p, g in self._grads:
            if p.grad is not g:
                p.grad = g
        if self._x_grad is not None and self.x.grad is not self._x_grad:
            self.x.grad = self._x_grad
        return self.y


def create_d4_hnlq_linear(in_dim, out_dim, device=None, **kwargs):
    """coset/core/d4/layers.py:14-68: HNLQLinearQAT over 4-wide blocks
    quantized by the D4 projection (d4_quantize; q sets only the beta
    bounds).  device defaults to the GPU when one is visible."""
    if in_dim % 4 != 0:
        raise ValueError(f"Input dimension {in_dim} must be divisible by 4 for D4 lattice")
    device = default_device(device)
    lattice = D4Lattice(device=device)
    defaults = {"lattice": lattice, "quantize_fn": d4_quantize, "block_size": 4, "q": 4, "M": 2,
                "Delta0": None, "warmup_epochs": 0, "enable_diagnostics": False, "weight_clip_value": 2.0,
                "theta_trainable": True, "theta_init_value": 0.0, "rho": 0.95}
    defaults.update(kwargs)
    return HNLQLinearQAT(in_dim, out_dim, **defaults)


def create_e8_hnlq_linear(in_dim, out_dim, device=None, **kwargs):
    """coset/core/e8/layers.py:15-66 with this package's e8_quantize
    injected.  device defaults to the GPU when one is visible."""
    if in_dim % 8 != 0:
        raise ValueError(f"Input dimension {in_dim} must be divisible by 8 for E8 lattice")
    device = default_device(device)
    lattice = E8Lattice(device=device)
    defaults = {"lattice": lattice, "quantize_fn": e8_quantize, "block_size": 8, "q": 4, "M": 2,
                "Delta0": None, "warmup_epochs": 0, "enable_diagnostics": False, "weight_clip_value": 2.0,
                "theta_trainable": True, "theta_init_value": 0.0, "rho": 0.95}
    defaults.update(kwargs)
    return HNLQLinearQAT(in_dim, out_dim, **defaults)
