"""QAT layer (create_e8_hnlq_linear / HNLQLinearQAT) on the HIP kernels
against the reference's own forward/backward (tests/golden/layer.npz) and the
oracle's closed-form backward.

Tolerances are elementwise: |a - b| <= rtol * mag, where mag is the
magnitude of the summands that make up the value (|x| @ |W|^T for a
product, the sum of |terms| for a reduction), so rtol bounds the relative
error of the accumulation itself; rtol = 1e-3 (fp32 accumulate, the north
star's bound) unless a test says otherwise.  Quantized weights and the
kernel's beta are bit-exact."""
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


def close(a, b, mag, rtol=1e-3):
    """Elementwise |a - b| <= rtol * mag (mag >= |b|: the summands' magnitude)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    mag = np.maximum(np.asarray(mag, np.float64), np.abs(b))
    err = np.abs(a - b)
    bad = err > rtol * mag
    assert not bad.any(), (int(bad.sum()), float(err[bad].max()), float(mag[bad][np.argmax(err[bad])]))


def kernel_beta(layer):
    """The beta, d beta / d theta, W_q and words of one call of the fused
    quantizer kernel with the layer's theta and statistics (no step)."""
    from coset_amd.layers import qat_fwd_theta
    bpt = layer.blocks_per_row if layer.tiling == "row" else 1
    Wq, packed, beta, dbdt, _ = qat_fwd_theta(
        layer.weight.detach().contiguous(), layer.theta_beta.detach(), layer.sigma_ema, layer.xmax_ema, None,
        (float(layer.Delta0), float(layer.eta), layer._ginv_f, int(layer.M)), int(layer.q), 2,
        float(layer.weight_clip_value), int(bpt), torch.float32)
    return beta, dbdt, Wq, packed


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
    # the beta the fused kernel derives from theta and the statistics, and the
    # W_q it writes with it: bit-exact against the reference
    kb, _, kWq, _ = kernel_beta(layer)
    np.testing.assert_array_equal(kb.cpu().numpy(), g("beta"))
    np.testing.assert_array_equal(kWq.cpu().numpy(), g("Wq"))
    beta = layer._beta().detach().cpu().numpy()
    np.testing.assert_allclose(beta, g("beta"), rtol=2e-7)
    x = torch.from_numpy(g("x")).cuda().requires_grad_(True)
    y = layer(x)
    (y * torch.from_numpy(g("g")).cuda()).sum().backward()
    X, G, Wq, W = (g(k).astype(np.float64) for k in ("x", "g", "Wq", "W"))
    bref = g("beta").astype(np.float64)
    close(y.detach().cpu().numpy(), g("y"), np.abs(X) @ np.abs(Wq).T + np.abs(g("bias")))
    gWq = np.abs(G).T @ np.abs(X)                   # magnitude of dL/dW_q's summands
    close(layer.weight.grad.cpu().numpy(), g("dW"), gWq)
    # dtheta = (beta_max - beta_min) s (1 - s) * sum_row (g m / beta) W - (g m) Q / beta^2
    Qr = Wq * bref[:, None]
    dbdt = (g("beta_max") - g("beta_min")).astype(np.float64)
    s = 1 / (1 + np.exp(-g("theta").astype(np.float64)))
    mag_dtheta = np.abs(dbdt * s * (1 - s)) * (gWq / bref[:, None] * np.abs(W) + gWq * np.abs(Qr) / bref[:, None] ** 2
                                                ).sum(axis=1)
    close(layer.theta_beta.grad.cpu().numpy(), g("dtheta"), mag_dtheta)
    close(layer.bias.grad.cpu().numpy(), g("dbias"), np.abs(G).sum(axis=0))
    close(x.grad.cpu().numpy(), g("dx"), np.abs(G) @ np.abs(Wq))
    assert int(layer.step_count) == 1
    with torch.no_grad():
        Wq_layer = layer._quantize_weights().cpu().numpy()
    np.testing.assert_array_equal(Wq_layer, g("Wq"))


@pytest.mark.parametrize("tiling", ["row", "block"])
@pytest.mark.parametrize("q,gdt", [(2, torch.float32), (4, torch.float32), (4, torch.bfloat16), (8, torch.float32),
                                   (16, torch.float32), (3, torch.float32)])
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
    close(Wt.grad.cpu().numpy().reshape(-1, 8), dW_ref, np.abs(dW_ref), 1e-6)
    dbeta_ref = dbeta_blk.reshape(ntile, bpt).sum(axis=1)
    Gb = np.abs(Gf.astype(np.float64))
    bb64 = bb.astype(np.float64)[:, None]
    mag = (Gb / bb64 * np.abs(Wb) + Gb * np.abs(qraw) / bb64 ** 2).sum(axis=1).reshape(ntile, bpt).sum(axis=1)
    close(bt.grad.cpu().numpy(), dbeta_ref, mag, 1e-5)


C5_SHAPES = [(768, 768), (768, 3072), (3072, 768)]


@pytest.mark.parametrize("fin,fout", C5_SHAPES)
@pytest.mark.parametrize("variant", ["config", "delta15"])
def test_c5_shapes_bf16_forward_backward(fin, fout, variant):
    """The BERT-base C5 layers at their real size, 4096 bf16 tokens.

    variant "config": the configuration's own weights, W ~ N(0, 0.02) at the
    default Delta0 and theta = 0, where W_q == 0: the forward must give
    y == bias exactly and dx == 0, and dW / dtheta follow the oracle's
    closed-form backward.  variant "delta15": Delta0 = 1.5, W ~ N(0, 1) (the
    quantizer is not degenerate): W_q bit-exact against the oracle on sampled
    rows with the kernel's beta.  Products and gradients against fp32
    references of the same bf16 operands, elementwise within 2^-8 of the
    summands' magnitude (bf16 rounding of the GEMM outputs)."""
    import coset_amd
    torch.manual_seed(7)
    if variant == "config":
        layer = coset_amd.create_e8_hnlq_linear(fin, fout, q=4, M=2)
        with torch.no_grad():
            layer.weight.normal_(0.0, 0.02)
    else:
        layer = coset_amd.create_e8_hnlq_linear(fin, fout, q=4, M=2, Delta0=1.5)   # N(0, 1) init
    print(f"C5 {fin}x{fout} {variant}", flush=True)
    # the kernel's beta and W_q (bf16, as the forward writes it) at step 1
    kb, kdbdt, kWq, _ = kernel_beta(layer)
    bmin, bmax = O.beta_bounds(4, 2, layer.Delta0, layer.eta, np.ones(fout), np.ones(fout))
    np.testing.assert_allclose(kb.cpu().numpy(), O.beta_from_theta(np.zeros(fout), bmin, bmax), rtol=1e-6)
    torch.testing.assert_close(kb, layer._beta().detach(), rtol=2e-7, atol=0)
    rows = np.arange(0, fout, 61)
    W_rows = layer.weight.detach()[rows].cpu().numpy()
    beta_rows = kb[rows].cpu().numpy()
    Wq_ref, qraw_ref, _ = O.layer_quant(W_rows, beta_rows, 4, 2, 2.0)
    np.testing.assert_array_equal(kWq[rows].cpu().numpy(), Wq_ref)

    x = torch.randn(4096, fin, device="cuda").to(torch.bfloat16).requires_grad_(True)
    gy = torch.randn(4096, fout, device="cuda").to(torch.bfloat16)
    y = layer(x)
    assert y.dtype == torch.bfloat16
    y.backward(gy)
    xf, gf = x.detach().float(), gy.float()
    Wq_b = torch.from_numpy(O.layer_quant(layer.weight.detach().cpu().numpy(), kb.cpu().numpy(), 4, 2, 2.0)[0]
                            ).cuda().to(torch.bfloat16).float()
    if variant == "config":
        assert not Wq_b.any()
        assert torch.equal(y, layer.bias.detach().to(torch.bfloat16).expand_as(y))
        assert not x.grad.any()
    else:
        close(y.detach().float().cpu().numpy(), (xf @ Wq_b.T + layer.bias.detach()).cpu().numpy(),
              (xf.abs() @ Wq_b.abs().T).cpu().numpy(), 2 ** -8)
        close(x.grad.float().cpu().numpy(), (gf @ Wq_b).cpu().numpy(), (gf.abs() @ Wq_b.abs()).cpu().numpy(),
              2 ** -8)
    # dW and dtheta on the sampled rows: the oracle's closed form from the fp32 dL/dW_q
    gWq = (gf.T @ xf)[rows].cpu().numpy()
    mag = (gf.abs().T @ xf.abs())[rows].cpu().numpy()
    dW_ref, dbeta_ref, _ = O.layer_backward(gWq, W_rows, qraw_ref, beta_rows, 2.0)
    close(layer.weight.grad[rows].cpu().numpy(), dW_ref, mag, 2 ** -8)
    b64 = beta_rows.astype(np.float64)[:, None]
    mag_dbeta = (mag / b64 * np.abs(W_rows) + mag * np.abs(qraw_ref) / b64 ** 2).sum(axis=1)
    dbdt = kdbdt[rows].cpu().numpy().astype(np.float64)
    close(layer.theta_beta.grad[rows].cpu().numpy(), dbeta_ref * dbdt, mag_dbeta * np.abs(dbdt), 2 ** -8)
    close(layer.bias.grad.cpu().numpy(), gf.sum(0).cpu().numpy(), gf.abs().sum(0).cpu().numpy(), 1e-5)


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
    dth = layer.theta_beta.grad.cpu().numpy()
    close(dtheta_fused.cpu().numpy(), dth, np.abs(dth), 1e-5)
    dw = layer.weight.grad.cpu().numpy()
    close(dW_fused.cpu().numpy(), dw, np.abs(dw), 1e-6)
    # W_q is bit-equal on every tile whose beta the two paths computed equal
    kb = kernel_beta(layer)[0]
    same = (kb == beta.detach())
    assert same.float().mean().item() > 0.9
    tile_of = torch.arange(Wq.numel(), device=Wq.device).reshape(Wq.shape) // (128 if tiling == "row" else 8)
    eq = same[tile_of]
    assert torch.equal(Wq[eq], Wq2[eq])
    assert int(layer.step_count) == 1


STAT_CASES = [("row", 64, 16, dict(q=4, M=2, Delta0=1.5)), ("c1", 768, 10, dict(q=4, M=2))]


@pytest.mark.parametrize("name,fin,fout,kw", STAT_CASES)
def test_step_256_statistics_update_matches_reference(golden, name, fin, fout, kw):
    """A layer run across its 256th step (coset/core/layers.py:408-413): the
    EMA buffers after the update and the beta the step derives from them are
    bit-exact against the reference (tests/golden/layer_stats.npz), and so
    is W_q at step 257; outputs and gradients within the elementwise bound."""
    import coset_amd
    S = golden("layer_stats")
    g = lambda k: S[f"{name}_{k}"]
    layer = coset_amd.create_e8_hnlq_linear(fin, fout, **kw)
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(g("W")))
        layer.bias.copy_(torch.from_numpy(g("bias")))
        layer.theta_beta.copy_(torch.from_numpy(g("theta")))
    x = torch.from_numpy(g("x")).cuda()
    with torch.no_grad():
        for _ in range(255):
            layer(x)
    assert int(layer.step_count) == 255
    np.testing.assert_array_equal(layer.sigma_ema.cpu().numpy(), g("sigma_ema_255"))
    xg = x.clone().requires_grad_(True)
    y = layer(xg)
    (y * torch.from_numpy(g("g")).cuda()).sum().backward()
    np.testing.assert_array_equal(layer.sigma_ema.cpu().numpy(), g("sigma_ema"))
    np.testing.assert_array_equal(layer.xmax_ema.cpu().numpy(), g("xmax_ema"))
    kb, _, kWq, _ = kernel_beta(layer)
    np.testing.assert_array_equal(kb.cpu().numpy(), g("beta"))
    np.testing.assert_array_equal(kWq.cpu().numpy(), g("Wq"))
    X, G, Wq = (g(k).astype(np.float64) for k in ("x", "g", "Wq"))
    close(y.detach().cpu().numpy(), g("y"), np.abs(X) @ np.abs(Wq).T + np.abs(g("bias")))
    close(layer.weight.grad.cpu().numpy(), g("dW"), np.abs(G).T @ np.abs(X))
    close(xg.grad.cpu().numpy(), g("dx"), np.abs(G) @ np.abs(Wq))
    close(layer.bias.grad.cpu().numpy(), g("dbias"), np.abs(G).sum(axis=0))
    dth = g("dtheta").astype(np.float64)
    close(layer.theta_beta.grad.cpu().numpy(), dth, np.abs(dth) + 1e-3 * np.abs(dth).max())
    with torch.no_grad():
        np.testing.assert_array_equal(layer._quantize_weights().cpu().numpy(), g("Wq"))
    assert int(layer.step_count) == 257


def test_block_tiling_statistics_match_reference(golden):
    """Block tiling (one tile per 8-wide block): two updates through the
    statistics kernel, bit-exact against the reference's _gather_stats."""
    import coset_amd
    S = golden("layer_stats")
    layer = coset_amd.create_e8_hnlq_linear(32, 8, q=4, M=2, Delta0=1.5, tiling="block")
    W = torch.from_numpy(S["block_W"]).cuda()
    for i in (1, 2):
        layer._gather_stats(W.view(8, 4, 8))
        np.testing.assert_array_equal(layer.sigma_ema.cpu().numpy(), S[f"block_sigma_ema_{i}"])
        np.testing.assert_array_equal(layer.xmax_ema.cpu().numpy(), S[f"block_xmax_ema_{i}"])


@pytest.mark.parametrize("tiling", ["row", "block"])
def test_statistics_propagate_non_finite_weights(tiling):
    """A NaN weight in one tile and an infinite one in another: the
    statistics kernel's EMA buffers equal the reference's composition
    (coset/core/layers.py:366-379: W.std() + 1e-8 and W.abs().amax() + 1e-8,
    then the EMA) computed by torch on the CPU, NaN where it is NaN -- amax
    propagates NaN, which a plain fmax would drop."""
    import coset_amd
    torch.manual_seed(5)
    fout, fin = 6, 64
    layer = coset_amd.create_e8_hnlq_linear(fin, fout, q=4, M=2, Delta0=1.5, tiling=tiling)
    W = torch.randn(fout, fin) * 0.3
    W[1, 17] = float("nan")
    W[3, 40] = float("inf")
    W[4, 2] = -float("inf")
    blocks = W.view(fout, fin // 8, 8)
    layer._gather_stats(blocks.cuda())
    m = layer.ema_momentum
    if tiling == "row":
        sigma = blocks.std(dim=(1, 2)) + 1e-8
        xmax = blocks.abs().amax(dim=(1, 2)) + 1e-8
    else:
        sigma = blocks.std(dim=2).reshape(-1) + 1e-8
        xmax = blocks.abs().amax(dim=2).reshape(-1) + 1e-8
    ones = torch.ones_like(sigma)
    want_s = ones.mul(m).add((1 - m) * sigma)
    want_x = ones.mul(m).add((1 - m) * xmax)
    assert torch.isnan(want_x).any() and torch.isinf(want_x).any()
    # finite entries: torch's CPU std may round its last bit differently from
    # the kernel's double-precision variance (bit parity is pinned on the
    # reference's own statistics in layer_stats.npz); NaN and inf exactly
    torch.testing.assert_close(layer.sigma_ema.cpu(), want_s, rtol=1e-6, atol=0, equal_nan=True)
    torch.testing.assert_close(layer.xmax_ema.cpu(), want_x, rtol=0, atol=0, equal_nan=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(4096, 768), (4096, 3072), (1, 8), (65, 24), (0, 16), (130, 40)])
def test_colsum_is_exact_fp32_sum(dtype, rows, cols):
    """The bias-gradient column sum: fp32 accumulation of the given values,
    elementwise within 2^-17 of the sum of magnitudes (at 4096 rows each value
    passes through at most 16 + 2 + 64 fp32 additions, each off by at most
    2^-24 of the running magnitude), and deterministic (two calls
    bit-equal)."""
    from coset_amd.layers import colsum
    g = torch.randn(rows, cols, device="cuda").to(dtype)
    a = colsum(g)
    b = colsum(g)
    assert torch.equal(a, b)
    ref = g.double().sum(0)
    mag = g.double().abs().sum(0)
    assert ((a.double() - ref).abs() <= 2 ** -17 * mag + 1e-30).all()
    assert a.shape == (cols,) and a.dtype == torch.float32


@pytest.mark.parametrize("rows,cols", [(768, 768), (4096, 2048), (3, 8)])
def test_fused_quantizer_writes_the_bias_cast(rows, cols):
    """The quantizer launch also writes the fp32 bias in bf16, equal to
    torch's cast (round to nearest even, NaN and infinities kept), on the
    general kernel and on the table kernel's path (4096 x 2048 = 2^20
    blocks: a side launch), with W_q unchanged by it."""
    from coset_amd.layers import qat_fwd_theta
    g = torch.Generator(device="cuda").manual_seed(rows + cols)
    W = 0.02 * torch.randn((rows, cols), device="cuda", generator=g)
    theta = torch.randn(rows, device="cuda", generator=g)
    sigma = torch.full((rows,), 0.02, device="cuda")
    xmax = torch.full((rows,), 0.08, device="cuda")
    bias = torch.randn(rows, device="cuda", generator=g) * 10
    bias[0] = float("inf")
    if rows > 2:
        bias[1] = float("nan")
        bias[2] = 1.0 + 2 ** -8          # a tie: rounds to even
    args = (W, theta, sigma, xmax, None, (1.5, 0.1, 1 / 12.0, 2), 4, 2, 2.0, cols // 8, torch.bfloat16)
    Wq, packed, beta, dbdt, bc = qat_fwd_theta(*args, bias=bias)
    Wq2, packed2, beta2, _, none = qat_fwd_theta(*args)
    assert none is None and bc.dtype == torch.bfloat16 and bc.shape == (rows,)
    ref = bias.to(torch.bfloat16)
    assert torch.equal(bc.view(torch.int16)[~ref.isnan()], ref.view(torch.int16)[~ref.isnan()])
    assert torch.equal(bc.isnan(), ref.isnan())
    assert torch.equal(Wq, Wq2) and torch.equal(packed, packed2) and torch.equal(beta, beta2)


@pytest.mark.parametrize("q,M", [(4, 2), (4, 4), (8, 2), (16, 2), (16, 3), (16, 4)])
def test_theta_quantizer_layer_kernel_matches_generic(q, M):
    """The fused quantizer with beta from theta at q = 4, 8, 16 on the layer
    round-trip kernel (betas derived once per row in the workgroup, the
    decode through tables, dec / beta from one reciprocal) against the generic kernel
    (set_codec_plain(False)), bit for bit: W_q in fp32 and bf16, the level
    words, beta, d beta / d theta, the step counter and the bias cast; rows
    of 64 (the least the per-workgroup betas take), 96 and 384 blocks, and a
    row count that ends inside a workgroup."""
    from coset_amd import _lib
    from coset_amd.layers import qat_fwd_theta
    for rows, cols in ((37, 512), (768, 768), (96, 3072)):
        g = torch.Generator(device="cuda").manual_seed(rows * 7 + cols + q + M)
        W = 0.02 * torch.randn((rows, cols), device="cuda", generator=g)
        W[0, :8] = 0.0
        theta = 3 * torch.randn(rows, device="cuda", generator=g)
        sigma = 0.02 * (0.5 + torch.rand(rows, device="cuda", generator=g))
        xmax = 4 * sigma
        bias = torch.randn(rows, device="cuda", generator=g)
        for odt in (torch.float32, torch.bfloat16):
            res = []
            for plain in (True, False):
                _lib.set_codec_plain(plain)
                try:
                    sc = torch.zeros((), dtype=torch.int64, device="cuda")
                    out = qat_fwd_theta(W, theta, sigma, xmax, sc, (1.5, 0.1, 1 / 12.0, M), q, M, 2.0, cols // 8, odt,
                                        bias=bias)
                    res.append([t.clone() for t in out] + [sc.clone()])
                finally:
                    _lib.set_codec_plain(True)
            case = f"q={q} M={M} rows={rows} cols={cols} {odt}"
            for a, b in zip(res[0], res[1]):
                if a.dtype in (torch.float32, torch.bfloat16):
                    a, b = a.view(torch.int32 if a.dtype == torch.float32 else torch.int16), \
                        b.view(torch.int32 if b.dtype == torch.float32 else torch.int16)
                assert torch.equal(a, b), case
            assert int(res[0][-1]) == 1, case


@pytest.mark.parametrize("fin,fout,q,kw,wstd", [(768, 10, 4, dict(theta_init_value=0.0), 0.02),
                                                (768, 10, 4, dict(Delta0=1.5), 1.0),
                                                (512, 96, 2, dict(Delta0=1.5), 1.0),
                                                (2048, 33, 4, dict(Delta0=1.5, weight_clip_value=0.5), 1.0)])
def test_head_forward_matches_two_launch_path(fin, fout, q, kw, wstd):
    """A no-grad forward of up to 64 fp32 tokens in one launch
    (coset_e8_qat_head_fwd: the quantizer's W_q bit for bit, then fp32
    products in a fixed order) against the quantizer followed by F.linear
    (set_head_forward(False)): outputs within the fp32 accumulation bound of
    the products' magnitude, the same step counter, and token counts 1, 7, 32,
    64 and a 3-D input.  A forward that needs gradients takes the two-launch
    path."""
    import coset_amd as ca
    from coset_amd import layers as L
    torch.manual_seed(fin + fout)
    layer = ca.create_e8_hnlq_linear(fin, fout, q=q, M=2, **kw)
    with torch.no_grad():
        layer.weight.normal_(0.0, wstd)
        layer.bias.normal_(0.0, 0.1)
        layer.theta_beta.uniform_(-2.0, 2.0)
    for shape in ((1, fin), (7, fin), (32, fin), (64, fin), (2, 16, fin)):
        x = torch.randn(shape, device="cuda")
        outs, steps = [], []
        for fused in (True, False):
            L.set_head_forward(fused)
            try:
                s0 = int(layer.step_count)
                with torch.no_grad():
                    outs.append(layer(x))
                steps.append(int(layer.step_count) - s0)
            finally:
                L.set_head_forward(True)
        with torch.no_grad():
            Wq = layer._quantize_weights()
        mag = (x.reshape(-1, fin).abs().double() @ Wq.abs().double().t()).reshape(outs[1].shape) + 1e-30
        assert steps == [1, 1], shape
        assert outs[0].shape == outs[1].shape == (*shape[:-1], fout)
        # two fp32 sums of fin products in different orders: each within
        # fin 2^-24 of the products' magnitude
        assert ((outs[0].double() - outs[1].double()).abs() <= fin * 2.0 ** -23 * mag + 1e-7).all(), shape
    # gradients needed: the two-launch path (autograd through QATLinearFn)
    x = torch.randn(8, fin, device="cuda", requires_grad=True)
    assert not layer._head_takes(x)
    y = layer(x)
    assert y.grad_fn is not None


def test_head_forward_refuses_unsupported_sizes():
    """More than 64 tokens, columns past 8192 or not a multiple of 8, q
    outside {2, 4}: COSET_EUNSUPPORTED or EINVAL before any launch."""
    from coset_amd import _lib
    lib = _lib.load()
    W = torch.zeros((4, 64), device="cuda")
    x = torch.zeros((65, 64), device="cuda")
    y = torch.zeros((65, 4), device="cuda")
    t = torch.zeros(4, device="cuda")
    args = lambda tokens, cols, q: (W.data_ptr(), 4, cols, t.data_ptr(), t.data_ptr(), t.data_ptr(), 1.5, 0.1,
                                    1 / 12.0, 2, 2.0, q, x.data_ptr(), tokens, None, y.data_ptr(), None,
                                    _lib.stream_of(x))
    assert lib.coset_e8_qat_head_fwd(*args(65, 64, 4)) != 0
    assert lib.coset_e8_qat_head_fwd(*args(8, 8200, 4)) != 0
    assert lib.coset_e8_qat_head_fwd(*args(8, 60, 4)) != 0
    assert lib.coset_e8_qat_head_fwd(*args(8, 64, 8)) != 0
