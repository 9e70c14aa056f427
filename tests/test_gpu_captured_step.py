"""CapturedQATStep: the QAT layer step replayed from a HIP graph against the
same steps run eagerly on an identical layer.  Every replay is checked, with
eager work (an SGD update of the parameters, the eager layer's own step and
host synchronisations) between replays, and with the statistics update
falling between replays."""
import pytest
import torch

import coset_amd


def _pair(fin, fout, tiling, interval):
    layers = []
    for _ in range(2):
        torch.manual_seed(11)
        L = coset_amd.create_e8_hnlq_linear(fin, fout, q=4, M=2, tiling=tiling)
        with torch.no_grad():
            L.weight.normal_(0.0, 0.05)
            L.theta_beta.uniform_(-1.0, 1.0)
        L.stat_update_interval = interval
        layers.append(L)
    return layers


def _grads(L, x):
    return [x.grad, L.weight.grad, L.theta_beta.grad, L.bias.grad]


@pytest.mark.gpu
@pytest.mark.parametrize("tiling,dtype,fin,fout,tokens", [
    ("row", torch.bfloat16, 256, 384, 512), ("block", torch.bfloat16, 256, 384, 512),
    ("row", torch.float32, 256, 384, 512), ("block", torch.float32, 256, 384, 512),
    # a BERT-base shape: the captured backward runs dX and the bias gradient on a
    # second stream beside dW, the eager one on one stream
    ("row", torch.bfloat16, 768, 3072, 4096)])
def test_captured_step_matches_eager_steps(tiling, dtype, fin, fout, tokens):
    steps = 7
    eager, cap_layer = _pair(fin, fout, tiling, interval=3)
    gen = torch.Generator(device="cuda").manual_seed(5)
    xs = [torch.randn(tokens, fin, device="cuda", generator=gen).to(dtype) for _ in range(steps)]
    gys = [torch.randn(tokens, fout, device="cuda", generator=gen).to(dtype) for _ in range(steps)]

    x_static = torch.zeros(tokens, fin, device="cuda", dtype=dtype, requires_grad=True)
    gy_static = torch.zeros(tokens, fout, device="cuda", dtype=dtype)
    cap = coset_amd.CapturedQATStep(cap_layer, x_static, gy_static)
    # the warm-up before capture leaves counters and statistics untouched
    assert int(cap_layer.step_count) == 0 and cap_layer._host_step == 0
    assert torch.equal(cap_layer.sigma_ema, eager.sigma_ema)

    for i in range(steps):
        eager.zero_grad(set_to_none=True)
        xa = xs[i].clone().requires_grad_(True)
        ya = eager(xa)
        ya.backward(gys[i])
        yb = cap.step(xs[i], gys[i])
        torch.cuda.synchronize()
        print(f"step {i}: tiling={tiling} dtype={dtype}", flush=True)
        assert torch.equal(ya, yb), f"output differs at step {i}"
        for name, ga, gb in zip(("x", "weight", "theta", "bias"), _grads(eager, xa), _grads(cap_layer, x_static)):
            assert gb is not None, name
            assert torch.equal(ga, gb), f"{name} gradient differs at step {i}"
        assert int(eager.step_count) == int(cap_layer.step_count) == i + 1
        assert cap_layer._host_step == i + 1
        assert torch.equal(eager.sigma_ema, cap_layer.sigma_ema), f"sigma EMA differs at step {i}"
        assert torch.equal(eager.xmax_ema, cap_layer.xmax_ema), f"abs-max EMA differs at step {i}"
        # the same in-place parameter update on both layers: the graph reads the live parameters
        with torch.no_grad():
            for pa, pb in ((eager.weight, cap_layer.weight), (eager.theta_beta, cap_layer.theta_beta),
                           (eager.bias, cap_layer.bias)):
                pa.add_(pa.grad, alpha=-1e-2)
                pb.add_(pb.grad, alpha=-1e-2)
    # the statistics were updated at steps 3 and 6, so they moved off their initial ones
    assert not torch.equal(cap_layer.sigma_ema, torch.ones_like(cap_layer.sigma_ema))


@pytest.mark.gpu
def test_captured_step_tuned_gemms():
    """tune_gemms: the graph kept (torch's default products or TunableOp's)
    gives the eager step's weight, theta and bias gradients bit for bit (the
    library's own kernels), and its output and input gradient within the
    rounding of a bf16 product summed in another order (bit for bit when the
    default selection is kept); TunableOp's flags are as they were."""
    tun = torch.cuda.tunable
    flags = (tun.is_enabled(), tun.tuning_is_enabled())
    fin, fout, tokens = 768, 3072, 4096
    eager, cap_layer = _pair(fin, fout, "row", interval=256)
    gen = torch.Generator(device="cuda").manual_seed(21)
    x_static = torch.zeros(tokens, fin, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    gy_static = torch.zeros(tokens, fout, device="cuda", dtype=torch.bfloat16)
    cap = coset_amd.CapturedQATStep(cap_layer, x_static, gy_static, tune_gemms=True)
    print(f"selection {cap.gemm_selection}, replays {cap.tune_us}", flush=True)
    assert (tun.is_enabled(), tun.tuning_is_enabled()) == flags
    assert cap.gemm_selection in ("default", "tunableop")
    assert set(cap.tune_us) == {"default", "tunableop"}
    assert int(cap_layer.step_count) == 0 and cap_layer._host_step == 0
    # the quantized weight (fixed: no parameter update here), with the
    # counters it advances restored
    saved = {n: b.clone() for n, b in eager.named_buffers()}
    host_step = eager._host_step
    with torch.no_grad():
        wq = eager._quantize_weights().float()
        for n, b in eager.named_buffers():
            b.copy_(saved[n])
    eager._host_step = host_step
    for i in range(3):
        x = torch.randn(tokens, fin, device="cuda", generator=gen).to(torch.bfloat16)
        gy = torch.randn(tokens, fout, device="cuda", generator=gen).to(torch.bfloat16)
        eager.zero_grad(set_to_none=True)
        xa = x.clone().requires_grad_(True)
        ya = eager(xa)
        ya.backward(gy)
        yb = cap.step(x, gy)
        torch.cuda.synchronize()
        print(f"step {i}", flush=True)
        for name, ga, gb in (("weight", eager.weight.grad, cap_layer.weight.grad),
                             ("theta", eager.theta_beta.grad, cap_layer.theta_beta.grad),
                             ("bias", eager.bias.grad, cap_layer.bias.grad)):
            assert torch.equal(ga, gb), f"{name} gradient differs at step {i}"
        if cap.gemm_selection == "default":
            assert torch.equal(ya, yb) and torch.equal(xa.grad, x_static.grad)
        else:
            # fp32 sums of exact bf16 products, rounded once to bf16: two
            # orders differ by at most one bf16 rounding plus the fp32 sums'
            mag_y = x.float().abs() @ wq.abs().t() + eager.bias.detach().float().abs()
            mag_dx = gy.float().abs() @ wq.abs()
            assert ((ya.float() - yb.float()).abs() <= 2.0 ** -7 * mag_y + 1e-30).all(), f"output at step {i}"
            assert ((xa.grad.float() - x_static.grad.float()).abs() <= 2.0 ** -7 * mag_dx + 1e-30).all(), \
                f"input gradient at step {i}"
        assert int(eager.step_count) == int(cap_layer.step_count) == i + 1


@pytest.mark.gpu
def test_captured_forward_only_matches_eager():
    eager, cap_layer = _pair(768, 10, "row", interval=256)
    x = torch.zeros(32, 768, device="cuda")
    cap = coset_amd.CapturedQATStep(cap_layer, x)
    gen = torch.Generator(device="cuda").manual_seed(9)
    for i in range(4):
        xi = torch.randn(32, 768, device="cuda", generator=gen)
        with torch.no_grad():
            ya = eager(xi)
        yb = cap.step(xi)
        torch.cuda.synchronize()
        assert torch.equal(ya, yb), f"forward differs at call {i}"
    assert int(cap_layer.step_count) == int(eager.step_count) == 4


@pytest.mark.gpu
def test_captured_step_refuses_stale_mode():
    _, L = _pair(64, 16, "row", interval=256)
    x = torch.randn(8, 64, device="cuda", requires_grad=True)
    cap = coset_amd.CapturedQATStep(L, x, torch.randn(8, 16, device="cuda"))
    cap.step()
    L.disable_quantization()
    with pytest.raises(RuntimeError):
        cap.step()


def test_captured_step_needs_gpu_tensors():
    L = coset_amd.create_e8_hnlq_linear(16, 8, device="cpu")
    with pytest.raises(ValueError):
        coset_amd.CapturedQATStep(L, torch.zeros(2, 16))


@pytest.mark.gpu
def test_captured_step_with_optimizer_zero_grad():
    """opt.zero_grad() (set_to_none) + cap.step() + opt.step() updates the
    parameters exactly as the same eager loop does."""
    eager, cap_layer = _pair(128, 64, "row", interval=256)
    gen = torch.Generator(device="cuda").manual_seed(21)
    xs = [torch.randn(64, 128, device="cuda", generator=gen) for _ in range(4)]
    gys = [torch.randn(64, 64, device="cuda", generator=gen) for _ in range(4)]
    x_static = torch.zeros(64, 128, device="cuda", requires_grad=True)
    cap = coset_amd.CapturedQATStep(cap_layer, x_static, torch.zeros(64, 64, device="cuda"))
    opt_a = torch.optim.SGD(eager.parameters(), lr=0.05)
    opt_b = torch.optim.SGD(cap_layer.parameters(), lr=0.05)
    for i in range(4):
        opt_a.zero_grad(set_to_none=True)
        eager(xs[i]).backward(gys[i])
        opt_a.step()
        opt_b.zero_grad(set_to_none=True)
        cap.step(xs[i], gys[i])
        opt_b.step()
        torch.cuda.synchronize()
        print(f"optimizer step {i}", flush=True)
        for name, pa, pb in (("weight", eager.weight, cap_layer.weight), ("theta", eager.theta_beta,
                                                                          cap_layer.theta_beta),
                             ("bias", eager.bias, cap_layer.bias)):
            assert torch.equal(pa, pb), f"{name} differs after optimizer step {i}"
    assert x_static.grad is not None


@pytest.mark.gpu
def test_captured_step_after_load_state_dict():
    """load_state_dict copies in place: the next replay reads the loaded
    values and the host counter mirror is re-read from the loaded buffer."""
    src_layer, cap_layer = _pair(64, 16, "row", interval=256)
    x = torch.randn(8, 64, device="cuda")
    cap = coset_amd.CapturedQATStep(cap_layer, x.clone())
    cap.step()
    with torch.no_grad():
        src_layer.weight.mul_(3.0)
        src_layer.step_count.fill_(41)
    cap_layer.load_state_dict(src_layer.state_dict())
    y = cap.step(x).clone()
    assert int(cap_layer.step_count) == 42 and cap_layer._host_step == 42
    with torch.no_grad():
        ya = src_layer(x)
    assert torch.equal(y, ya)


@pytest.mark.gpu
def test_captured_step_refuses_replaced_weights():
    _, L = _pair(64, 16, "row", interval=256)
    cap = coset_amd.CapturedQATStep(L, torch.randn(8, 64, device="cuda"))
    cap.step()
    L.load_weights(torch.randn(16, 64))
    with pytest.raises(RuntimeError):
        cap.step()
