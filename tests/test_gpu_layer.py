"""QAT layer (create_e8_hnlq_linear / HNLQLinearQAT) on the HIP kernels
against the reference's own forward/backward (tests/golden/layer.npz) and the
oracle's closed-form backward.  Tolerances: outputs and gradients within
1e-3 of the reference's max magnitude (fp32 accumulate); quantized weights
bit-exact where the layer's beta is bit-equal to the reference's."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

LAYER_CASES = [
    ("c1", 768, 10, dict(q=4, M=2, theta_init_value=0.0, weight_clip_value=2.0)),
    ("c1nd", 768, 10, dict(q=4, M=2, Delta0=1.5, weight_clip_value=2.0)),
    ("rnd", 64, 16, dict(q=4, M=2, Delta0=1.5, weight_clip_value=2.0)),
    ("clip", 64, 16, dict(q=4, M=2, Delta0=6.0, weight_clip_value=0.5)),
    ("q16", 64, 8, dict(q=16, M=3, Delta0=1.5, weight_clip_value=2.0)),
]


def close(a, b, tol=1e-3):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = max(np.abs(b).max(), 1e-30)
    assert np.abs(a - b).max() <= tol * scale, (np.abs(a - b).max(), scale)


@pytest.mark.parametrize("name,fin,fout,kw", LAYER_CASES)
def test_layer_matches_reference(golden, name, fin, fout, kw):
    import coset_amd
    L = golden("layer")
    g = lambda k: L[f"{name}_{k}"]
    layer = coset_amd.create_e8_hnlq_linear(fin, fout, **kw)
    assert layer.weight.is_cuda
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(g("W")))
        layer.bias.copy_(torch.from_numpy(g("bias")))
        layer.theta_beta.copy_(torch.from_numpy(g("theta")))
    beta = layer._beta().detach().cpu().numpy()
    np.testing.assert_allclose(beta, g("beta"), rtol=2e-7)
    x = torch.from_numpy(g("x")).cuda().requires_grad_(True)
    y = layer(x)
    (y * torch.from_numpy(g("g")).cuda()).sum().backward()
    close(y.detach().cpu().numpy(), g("y"))
    close(layer.weight.grad.cpu().numpy(), g("dW"))
    close(layer.theta_beta.grad.cpu().numpy(), g("dtheta"))
    close(layer.bias.grad.cpu().numpy(), g("dbias"))
    close(x.grad.cpu().numpy(), g("dx"))
    assert int(layer.step_count) == 1
    with torch.no_grad():
        Wq = layer._quantize_weights().cpu().numpy()
    if np.array_equal(beta, g("beta")):
        np.testing.assert_array_equal(Wq, g("Wq"))
    else:
        close(Wq, g("Wq"))


@pytest.mark.parametrize("tiling", ["row", "block"])
@pytest.mark.parametrize("q,gdt", [(4, torch.float32), (4, torch.bfloat16), (16, torch.float32), (3, torch.float32)])
def test_weight_quant_kernels_vs_oracle(tiling, q, gdt):
    """coset_e8_qat_fwd/bwd against the oracle's quantizer and closed-form
    backward, with the clamp active on part of the weights."""
    from coset_amd import E8WeightQuant
    rng = np.random.default_rng(q)
    rows, cols, clip = 24, 128, 1.2
    W = rng.standard_normal((rows, cols)).astype(np.float32)
    ntile = rows if tiling == "row" else rows * cols // 8
    bpt = cols // 8 if tiling == "row" else 1
    beta = rng.uniform(0.3, 2.0, size=ntile).astype(np.float32)
    Wt = torch.from_numpy(W).cuda().requires_grad_(True)
    bt = torch.from_numpy(beta).cuda().requires_grad_(True)
    Wq = E8WeightQuant.apply(Wt, bt, q, 2, clip, bpt, torch.float32)
    beta_el = np.repeat(beta, cols // 8 if tiling == "row" else 1).reshape(-1)
    # oracle: per-block beta through a [n_blocks, 8] view (one block per "row")
    Wb = W.reshape(-1, 8)
    bb = np.repeat(beta, bpt).astype(np.float32)
    Wq_ref, qraw, _ = O.layer_quant(Wb, bb, q, 2, clip)
    np.testing.assert_array_equal(Wq.detach().cpu().numpy().reshape(-1, 8), Wq_ref)
    G = rng.standard_normal((rows, cols)).astype(np.float32)
    gt = torch.from_numpy(G).cuda().to(gdt)
    Wq.backward(gt)
    Gf = gt.float().cpu().numpy().reshape(-1, 8)
    dW_ref, dbeta_blk, _ = O.layer_backward(Gf, Wb, qraw, bb, clip)
    close(Wt.grad.cpu().numpy().reshape(-1, 8), dW_ref, 1e-6)
    dbeta_ref = dbeta_blk.reshape(ntile, bpt).sum(axis=1)
    close(bt.grad.cpu().numpy(), dbeta_ref, 1e-5)


def test_c5_shape_bf16_forward_backward():
    """BERT-base 768->3072 layer, 4096 bf16 tokens, Delta0 = 1.5 and
    W ~ N(0,1) so the quantizer is not degenerate.  W_q bit-exact vs the
    oracle on sampled rows; y and dx against fp32 products of the same bf16
    operands within 2^-7 of the max magnitude (bf16 output rounding)."""
    import coset_amd
    torch.manual_seed(7)
    layer = coset_amd.create_e8_hnlq_linear(768, 3072, Delta0=1.5)
    x = torch.randn(4096, 768, device="cuda").to(torch.bfloat16).requires_grad_(True)
    y = layer(x)
    assert y.dtype == torch.bfloat16
    gy = torch.randn_like(y)
    y.backward(gy)
    with torch.no_grad():
        beta = layer._beta()
        layer.step_count.zero_()
        layer._host_step = None
        Wq = layer._quantize_weights()
    rows = torch.arange(0, 3072, 97)
    Wq_ref, _, _ = O.layer_quant(layer.weight[rows].detach().cpu().numpy(), beta[rows].cpu().numpy(), 4, 2, 2.0)
    np.testing.assert_array_equal(Wq[rows].cpu().numpy(), Wq_ref)
    Wq_b = Wq.to(torch.bfloat16).float()
    y_ref = x.detach().float() @ Wq_b.T + layer.bias.detach().float()
    close(y.detach().float().cpu().numpy(), y_ref.cpu().numpy(), 2 ** -7)
    dx_ref = gy.float() @ Wq_b
    close(x.grad.float().cpu().numpy(), dx_ref.cpu().numpy(), 2 ** -7)
    assert torch.isfinite(layer.weight.grad).all() and torch.isfinite(layer.theta_beta.grad).all()


def test_custom_quantize_fn_runs_reference_composition():
    """An injected quantizer other than e8_quantize goes through the
    reference's ste_quantize composition (coset/core/layers.py:444)."""
    import coset_amd
    calls = []

    def qfn(x, q):
        calls.append(x.shape)
        return torch.round(x)

    lat = coset_amd.E8Lattice()
    layer = coset_amd.HNLQLinearQAT(16, 4, lat, qfn, Delta0=1.5)
    y = layer(torch.randn(3, 16, device="cuda"))
    y.sum().backward()
    assert calls == [(8, 8)]
    assert layer.weight.grad is not None


def test_stats_update_every_256_steps():
    import coset_amd
    layer = coset_amd.create_e8_hnlq_linear(16, 4, init_method="normal")
    x = torch.randn(2, 16, device="cuda")
    with torch.no_grad():
        for _ in range(255):
            layer(x)
        assert torch.equal(layer.sigma_ema, torch.ones_like(layer.sigma_ema))
        layer(x)
    assert int(layer.step_count) == 256
    W = layer.weight.detach().view(4, 2, 8)
    sigma = 0.99 + 0.01 * (W.std(dim=(1, 2)) + 1e-8)
    torch.testing.assert_close(layer.sigma_ema, sigma)


def test_state_dict_roundtrip():
    import coset_amd
    a = coset_amd.create_e8_hnlq_linear(32, 8, Delta0=1.5)
    b = coset_amd.create_e8_hnlq_linear(32, 8, Delta0=1.5)
    a(torch.randn(2, 32, device="cuda"))
    b.load_state_dict(a.state_dict())
    assert set(a.state_dict()) == {"weight", "bias", "theta_beta", "G", "Ginv", "sigma_ema", "xmax_ema",
                                   "step_count", "gamma_inv"}
    x = torch.randn(5, 32, device="cuda")
    torch.testing.assert_close(a(x), b(x))
    assert int(b.step_count) == 2
    ex = b.export_quantized()
    assert ex["codes"].shape == (8, 4, 2) and ex["weight"].shape == (8, 32) and ex["beta"].shape == (8,)


@pytest.mark.parametrize("tiling", ["row", "block"])
def test_fused_theta_path_matches_torch_beta_path(tiling):
    """The in-kernel beta (theta, EMA buffers) equals the torch composition of
    _bounds/_beta to 1 ulp-level tolerance, and dtheta equals autograd through
    it; W_q is bit-equal wherever beta is."""
    import coset_amd
    from coset_amd import E8WeightQuant
    torch.manual_seed(3)
    layer = coset_amd.create_e8_hnlq_linear(128, 24, Delta0=1.5, tiling=tiling)
    with torch.no_grad():
        layer.theta_beta.uniform_(-3, 3)
        layer.sigma_ema.uniform_(0.5, 2.0)
        layer.xmax_ema.uniform_(1.0, 4.0)
    Wq = layer._quantize_weights()
    g = torch.randn_like(Wq)
    (Wq * g).sum().backward()
    dtheta_fused = layer.theta_beta.grad.clone()
    dW_fused = layer.weight.grad.clone()
    layer.zero_grad()
    beta = layer._beta()
    bpt = 16 if tiling == "row" else 1
    Wq2 = E8WeightQuant.apply(layer.weight, beta, 4, 2, 2.0, bpt, torch.float32)
    (Wq2 * g).sum().backward()
    close(dtheta_fused.cpu().numpy(), layer.theta_beta.grad.cpu().numpy(), 1e-5)
    close(dW_fused.cpu().numpy(), layer.weight.grad.cpu().numpy(), 1e-6)
    diff = (Wq != Wq2).float().mean().item()
    assert diff < 1e-3, diff
    assert int(layer.step_count) == 1
