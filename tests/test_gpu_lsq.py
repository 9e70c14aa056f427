"""LSQ activation quantizer (coset/core/layers.py:117-137) through the fused
kernels coset_lsq_fwd / coset_lsq_bwd.

Pinned two ways: against torch on the CPU running the reference module's
own op sequence (ste_clip, ste_round, layers.py:20-26) in fp32 -- bit for
bit for the forward and dx, to summation order for dalpha -- and against
closed forms: outputs lie on the grid s * Z, clipped values sit at
+-qmax * s, and with nothing clipped dalpha = sum g (round(y) - y) / qmax."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def reference_lsq(x, alpha, qmax):
    """The reference forward (layers.py:129-137), as torch ops."""
    a = torch.relu(alpha) + 1e-8
    xc = (x - x.detach()) + torch.clamp(x, -a, a).detach()
    scale = a / qmax
    y = xc / scale
    yq = (y - y.detach()) + torch.round(y).detach()
    return yq * scale


def _inputs(n, seed, alpha):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, generator=g) * 1.5
    s = (alpha + 1e-8) / 127
    # exact ties of y = x / s, grid points, the clip bounds, signed zeros, tiny values
    k = torch.arange(-130, 130, dtype=torch.float32)
    special = torch.cat([(k + 0.5) * s, k * s, torch.tensor([alpha, -alpha, 0.0, -0.0, 1e-30, -1e-30, 3e38, -3e38])])
    x[: special.numel()] = special
    return x


def _bits(t):
    return t.contiguous().view(torch.int32)


@pytest.mark.parametrize("alpha,bits", [(1.3, 8), (0.7, 4), (2.0, 2)])
def test_forward_and_dx_bit_exact_fp32(alpha, bits):
    import coset_amd as ca
    torch.manual_seed(0)
    m = ca.LSQActivation(bit_width=bits, init_alpha=alpha).cuda()
    x = _inputs(70001, 1, alpha)
    xg = x.cuda().requires_grad_(True)
    out = m(xg)
    g = torch.randn(x.shape)
    out.backward(g.cuda())

    a_ref = torch.tensor(alpha, requires_grad=True)
    x_ref = x.clone().requires_grad_(True)
    out_ref = reference_lsq(x_ref, a_ref, m.qmax)
    out_ref.backward(g)
    assert torch.equal(_bits(out.detach().cpu()), _bits(out_ref.detach())), "forward differs"
    assert torch.equal(_bits(xg.grad.cpu()), _bits(x_ref.grad)), "dx differs"
    ga, gr = m.alpha.grad.item(), a_ref.grad.item()
    assert abs(ga - gr) <= 1e-4 * max(1.0, abs(gr)), (ga, gr)


def test_specials_and_closed_forms():
    import coset_amd as ca
    m = ca.LSQActivation(bit_width=8, init_alpha=1.0).cuda()
    a = 1.0 + 1e-8
    s = torch.tensor(a, dtype=torch.float32) / 127
    x = torch.tensor([float("inf"), float("-inf"), float("nan"), 5.0, -5.0, -0.0, -0.001, 0.3])
    out = m(x.cuda()).cpu()
    assert torch.isnan(out[:3]).all()            # (x - x) is NaN for +-inf
    assert out[3] == 127 * s and out[4] == -127 * s
    assert out[5].item() == 0.0 and not torch.signbit(out[5])   # (y - y) + round(y) is +0
    assert out[6].item() == 0.0 and not torch.signbit(out[6])
    q = (m(torch.randn(4096).cuda() * 3).cpu() / s)
    assert torch.equal(q, torch.round(q)) and q.abs().max() <= 127


def test_dalpha_closed_form_unclipped():
    """|x| < a: xc = x, so dL/ds = sum g (round(y) - y) exactly in reals."""
    import coset_amd as ca
    m = ca.LSQActivation(bit_width=6, init_alpha=4.0).cuda()
    gen = torch.Generator().manual_seed(5)
    x = (torch.rand(100000, generator=gen) - 0.5) * 7.0
    g = torch.randn(100000, generator=gen)
    xg = x.cuda().requires_grad_(True)
    m(xg).backward(g.cuda())
    a = torch.tensor(4.0 + 1e-8, dtype=torch.float32)
    s = (a / 31).double()
    y = x.double() / s
    want = (g.double() * (torch.round(y) - y)).sum() / 31
    assert abs(m.alpha.grad.item() - want.item()) <= 1e-4 * max(1.0, abs(want.item()))


def test_nonpositive_alpha():
    import coset_amd as ca
    m = ca.LSQActivation(bit_width=8, init_alpha=-0.5).cuda()
    x = torch.randn(1000).cuda().requires_grad_(True)
    out = m(x)
    out.sum().backward()
    assert m.alpha.grad.item() == 0.0              # relu backward
    assert out.abs().max().item() <= 1e-8 * 1.01  # a = 1e-8


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_half_dtypes_round_once(dtype):
    """16-bit activations: the fp32 result of the same chain, rounded once."""
    import coset_amd as ca
    m = ca.LSQActivation(bit_width=8, init_alpha=1.1).cuda()
    x = _inputs(50000, 3, 1.1).to(dtype)
    g = torch.randn(x.shape).to(dtype)
    xg = x.cuda().requires_grad_(True)
    out = m(xg)
    out.backward(g.cuda())
    assert out.dtype == dtype and xg.grad.dtype == dtype
    a = torch.tensor(1.1)
    x32 = x.float().requires_grad_(True)
    ref = reference_lsq(x32, a, m.qmax)
    ref.backward(g.float())
    # +-3e38 overflow fp16 to +-inf, and both sides give NaN there
    torch.testing.assert_close(out.detach().cpu(), ref.detach().to(dtype), rtol=0, atol=0, equal_nan=True)
    torch.testing.assert_close(xg.grad.cpu(), x32.grad.to(dtype), rtol=0, atol=0, equal_nan=True)


def test_empty_and_strided():
    import coset_amd as ca
    m = ca.LSQActivation(bit_width=8, init_alpha=1.0).cuda()
    e = torch.empty(0, 5).cuda().requires_grad_(True)
    out = m(e)
    out.sum().backward()
    assert out.shape == (0, 5) and m.alpha.grad.item() == 0.0
    x = torch.randn(64, 48).cuda()
    xt = x.t()                                      # non-contiguous view
    assert torch.equal(m(xt), m(xt.contiguous()))


def test_layer_with_activation_quantization():
    """HNLQLinearQAT(quantize_activations=True): actq applied to F.linear's
    output (layers.py:472-484), gradients reach alpha."""
    import coset_amd as ca
    torch.manual_seed(2)
    layer = ca.create_e8_hnlq_linear(64, 32, quantize_activations=True, act_bit_width=8, act_init_alpha=2.0)
    x = torch.randn(16, 64).cuda()
    y = layer(x)
    W_q = layer.export_quantized()["weight"]
    lin = torch.nn.functional.linear(x, W_q.to(x.dtype), layer.bias)
    assert torch.equal(y, layer.actq(lin))
    y.sum().backward()
    assert layer.actq.alpha.grad is not None and torch.isfinite(layer.actq.alpha.grad)


@pytest.mark.parametrize("name", ["b8_a1", "b8_a03", "b4_a2", "b8_neg", "b2_a1"])
def test_lsq_matches_reference_golden(golden, name):
    """LSQActivation against the reference module's own outputs
    (tests/golden/lsq.npz): forward and dx bit for bit, dalpha within 1e-6
    of the magnitude of its summands (summation order)."""
    import numpy as np
    import coset_amd as ca
    from oracle import oracle as O
    L = golden("lsq")
    x, g = L[f"{name}_x"], L[f"{name}_g"]
    alpha, bits = float(L[f"{name}_alpha"][0]), int(L[f"{name}_bits"])
    m = ca.LSQActivation(bit_width=bits, init_alpha=alpha).cuda()
    xg = torch.from_numpy(x).cuda().requires_grad_(True)
    y = m(xg)
    y.backward(torch.from_numpy(g).cuda())
    assert np.array_equal(y.detach().cpu().numpy().view(np.int32), L[f"{name}_y"].view(np.int32))
    assert np.array_equal(xg.grad.cpu().numpy().view(np.int32), L[f"{name}_dx"].view(np.int32))
    _, _, mag = O.lsq_backward(x, g, alpha, m.qmax)
    assert abs(m.alpha.grad.item() - float(L[f"{name}_dalpha"][0])) <= 1e-6 * mag
