"""D4 variant on the GPU: coset_d4_lattice_op and the D4 layer's fused
weight quantizer (coset_d4_qat_fwd / _fwd_theta / _bwd) against the oracle
(tests/test_oracle_d4.py pins it) and against torch autograd of the
reference composition (coset/core/layers.py:428-463 with d4_quantize)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _x(n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n, 4)) * 3).astype(np.float32)
    x[: n // 8] = np.round(x[: n // 8] * 4) / 4                 # ties of rounding and argmax
    x[n // 8: n // 8 + 64] = rng.choice(np.array([0.5, -0.5, 1.5, -1.5, 0.0, -0.0, 1e-30, 2.0 ** 23 + 1, -(2.0 ** 23) - 3,
                                                  2.5e7, -7.5], np.float32), size=(64, 4))
    return x


def test_lattice_ops_match_oracle():
    import coset_amd as ca
    lat = ca.D4Lattice()
    x = _x(20000, 1)
    xt = torch.from_numpy(x).cuda()
    assert np.array_equal(lat.projection(xt).cpu().numpy().view(np.int32), orc.d4_projection(x).view(np.int32))
    assert np.array_equal(lat.g_x(xt).cpu().numpy(), orc.d4_g_x(x))
    y = orc.d4_projection(x[:5000] / 64)    # small lattice points
    for q in (2, 3, 4, 7):
        b = lat.encode_coords(torch.from_numpy(y).cuda(), q).cpu().numpy()
        assert np.array_equal(b, orc.d4_encode_coords(y, q).astype(np.float32))
        assert np.array_equal(lat.decode_coords(torch.from_numpy(b).cuda(), q).cpu().numpy(),
                              orc.d4_decode_coords(b.astype(np.int32)))
    one = lat.projection(torch.tensor([0.6, 0.6, 0.2, -0.1], device="cuda"))    # single-vector form
    assert one.shape == (4,)


@pytest.mark.parametrize("tiling", ["row", "block"])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_qat_forward_matches_oracle(tiling, out_dtype):
    from coset_amd import _lib
    rng = np.random.default_rng(2)
    rows, cols = 24, 64
    W = (rng.standard_normal((rows, cols)) * 0.7).astype(np.float32)
    bpt = cols // 4 if tiling == "row" else 1
    beta = (rng.random(rows * cols // 4 // bpt) * 3 + 0.5).astype(np.float32)
    Wg = torch.from_numpy(W).cuda()
    bg = torch.from_numpy(beta).cuda()
    Wq = torch.empty((rows, cols), dtype=out_dtype, device="cuda")
    _lib.call("coset_d4_qat_fwd", Wg.data_ptr(), rows, cols, bg.data_ptr(), bpt, 2.0, Wq.data_ptr(),
              _lib.dtype_code(out_dtype), _lib.stream_of(Wg))
    want = torch.from_numpy(orc.d4_layer_quant(W, beta, bpt, 2.0)).to(out_dtype)
    assert torch.equal(Wq.cpu(), want)


class _STE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, p):
        return p

    @staticmethod
    def backward(ctx, g):
        return g, None


@pytest.mark.parametrize("tiling", ["row", "block"])
def test_qat_backward_matches_autograd(tiling):
    """dW bit for bit and dbeta to summation order against torch autograd of
    the reference composition on the CPU (STE identity backward)."""
    from coset_amd import _lib
    rng = np.random.default_rng(3)
    rows, cols, clip = 16, 48, 1.0
    W = (rng.standard_normal((rows, cols)) * 0.8).astype(np.float32)
    bpt = cols // 4 if tiling == "row" else 1
    nt = rows * cols // 4 // bpt
    beta = (rng.random(nt) * 2 + 0.5).astype(np.float32)
    g = rng.standard_normal((rows, cols)).astype(np.float32)

    Wt = torch.from_numpy(W).requires_grad_(True)
    bt = torch.from_numpy(beta).requires_grad_(True)
    bfull = bt.view(-1, 1) if tiling == "row" else bt.view(rows, cols // 4, 1)
    Ws = Wt * bfull if tiling == "row" else (Wt.view(rows, cols // 4, 4) * bfull).reshape(rows, cols)
    P = torch.from_numpy(orc.d4_projection(Ws.detach().numpy()).reshape(rows, cols))
    Q = _STE.apply(Ws, P)
    den = bfull if tiling == "row" else bt.view(rows, cols // 4).repeat_interleave(4, dim=1)
    out = torch.clamp(Q / den, -clip, clip)
    out.backward(torch.from_numpy(g))

    dW = torch.empty((rows, cols), device="cuda")
    dbeta = torch.empty(nt, device="cuda")
    gg, Wg, bg = (torch.from_numpy(a).cuda() for a in (g, W, beta))
    _lib.call("coset_d4_qat_bwd", gg.data_ptr(), _lib.dtype_code(gg.dtype), Wg.data_ptr(), bg.data_ptr(), None,
              rows, cols, bpt, clip, dW.data_ptr(), dbeta.data_ptr(), None, _lib.stream_of(gg))
    assert torch.equal(dW.cpu(), Wt.grad)
    np.testing.assert_allclose(dbeta.cpu().numpy(), bt.grad.numpy(), rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("tiling", ["row", "block"])
def test_d4_layer_fused_matches_torch_composition(tiling):
    """create_d4_hnlq_linear takes the fused D4 path; its W_q and gradients
    agree with the reference composition driven by torch's beta (in-kernel
    beta equals it to ulp level, as on the E8 path)."""
    import coset_amd as ca
    torch.manual_seed(5)
    layer = ca.create_d4_hnlq_linear(64, 24, tiling=tiling)
    assert layer._fused_d4() and layer.block_size == 4 and layer.q == 4 and layer.M == 2
    assert abs(layer.Delta0 - 2 * 0.95 * (1 / np.sqrt(2)) / 15) < 1e-12
    assert float(layer.gamma_inv) == 2.0
    with torch.no_grad():
        layer.theta_beta.uniform_(-3, 3)
        layer.sigma_ema.uniform_(0.5, 2.0)
        layer.xmax_ema.uniform_(1.0, 4.0)
    Wq = layer._quantize_weights()
    g = torch.randn_like(Wq)
    (Wq * g).sum().backward()
    dtheta, dW = layer.theta_beta.grad.clone(), layer.weight.grad.clone()
    layer.zero_grad()
    Wq2 = layer._reference_composition(layer.weight, layer._beta())
    (Wq2 * g).sum().backward()
    assert (Wq != Wq2).float().mean().item() < 1e-3
    torch.testing.assert_close(dW, layer.weight.grad, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(dtheta, layer.theta_beta.grad, rtol=1e-5, atol=1e-5)
    assert int(layer.step_count) == 1


def test_d4_layer_trains():
    import coset_amd as ca
    torch.manual_seed(1)
    layer = ca.create_d4_hnlq_linear(128, 32, quantize_activations=True)
    opt = torch.optim.SGD(layer.parameters(), lr=1e-2)
    x = torch.randn(64, 128, device="cuda")
    target = torch.randn(64, 32, device="cuda")
    for _ in range(3):
        opt.zero_grad()
        loss = torch.nn.functional.mse_loss(layer(x), target)
        loss.backward()
        opt.step()
    assert torch.isfinite(loss) and int(layer.step_count) == 3
    with pytest.raises(ValueError):
        ca.create_d4_hnlq_linear(10, 4)


@pytest.mark.parametrize("name,fin,fout,kw", [("d4def", 64, 16, dict(q=4, M=2)),
                                              ("d4nd", 64, 16, dict(q=4, M=2, Delta0=1.5)),
                                              ("d4clip", 32, 8, dict(q=4, M=2, Delta0=6.0, weight_clip_value=0.5))])
def test_d4_layer_matches_reference_golden(golden, name, fin, fout, kw):
    """create_d4_hnlq_linear against the reference's own D4 layer
    (tests/golden/d4.npz): the kernel's beta and W_q bit-exact, outputs and
    gradients elementwise within 1e-3 of the summands' magnitude; the
    projection and g_x bit-exact on the golden blocks."""
    import coset_amd as ca
    from coset_amd.layers import d4_qat_fwd_theta
    D = golden("d4")
    g = lambda k: D[f"{name}_{k}"]
    lat = ca.D4Lattice()
    xt = torch.from_numpy(D["x"]).cuda()
    assert np.array_equal(lat.projection(xt).cpu().numpy().view(np.int32), D["projection"].view(np.int32))
    assert np.array_equal(lat.g_x(xt).cpu().numpy(), D["g_x"])
    layer = ca.create_d4_hnlq_linear(fin, fout, **kw)
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(g("W")))
        layer.bias.copy_(torch.from_numpy(g("bias")))
        layer.theta_beta.copy_(torch.from_numpy(g("theta")))
    Wq_k, beta_k, _ = d4_qat_fwd_theta(layer.weight.detach().contiguous(), layer.theta_beta.detach(),
                                       layer.sigma_ema, layer.xmax_ema, None,
                                       (float(layer.Delta0), float(layer.eta), layer._ginv_f, int(layer.M)),
                                       int(layer.q), float(layer.weight_clip_value), fin // 4, torch.float32)
    np.testing.assert_array_equal(beta_k.cpu().numpy(), g("beta"))
    np.testing.assert_array_equal(Wq_k.cpu().numpy(), g("Wq"))
    x = torch.from_numpy(g("x")).cuda().requires_grad_(True)
    y = layer(x)
    (y * torch.from_numpy(g("g")).cuda()).sum().backward()
    X, G, Wq = (g(k).astype(np.float64) for k in ("x", "g", "Wq"))

    def close(a, b, mag):
        assert (np.abs(np.asarray(a, np.float64) - b) <= 1e-3 * np.maximum(mag, np.abs(b))).all()
    close(y.detach().cpu().numpy(), g("y"), np.abs(X) @ np.abs(Wq).T + np.abs(g("bias")))
    close(layer.weight.grad.cpu().numpy(), g("dW"), np.abs(G).T @ np.abs(X))
    close(x.grad.cpu().numpy(), g("dx"), np.abs(G) @ np.abs(Wq))
    close(layer.bias.grad.cpu().numpy(), g("dbias"), np.abs(G).sum(axis=0))
    dth = g("dtheta").astype(np.float64)
    close(layer.theta_beta.grad.cpu().numpy(), dth, np.abs(dth) + 1e-3 * np.abs(dth).max())
