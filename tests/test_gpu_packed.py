"""Packed-code export (QAT -> inference): a trained layer's level words and
per-row beta in a safetensors file, served by the vLUT matmul."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _layer(ca, fin=256, fout=64, clip=10.0):
    torch.manual_seed(3)
    layer = ca.create_e8_hnlq_linear(fin, fout, q=4, M=2, Delta0=1.5, weight_clip_value=clip)
    with torch.no_grad():
        layer.weight.normal_(0.0, 0.5)
    x = torch.randn(16, fin, device="cuda").to(torch.bfloat16)
    layer(x).float().sum().backward()   # one training step's forward/backward
    return layer


def test_save_load_serves_the_layer(tmp_path):
    import coset_amd as ca
    layer = _layer(ca)
    st = ca.save_packed(layer, str(tmp_path / "l.safetensors"))
    meta = st["metadata"]
    assert meta["q"] == 4 and meta["M"] == 2 and meta["clipped_weights"] == 0
    W_q = layer.export_quantized()["weight"]          # the same quantization (beta unchanged)
    pl = ca.load_packed(str(tmp_path / "l.safetensors"))
    assert pl.words.dtype == torch.uint16 and pl.words.shape == (64, 32, 2)
    # decode(words) / beta is the layer's W_q bit for bit (nothing clipped)
    torch.testing.assert_close(pl.dequantized_weight(), W_q.float(), rtol=0, atol=0)
    x = torch.randn(5, 3, 256, device="cuda")
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        xa = x.to(dt)
        y = pl(xa)
        ref = F.linear(xa.float(), W_q.float(), layer.bias.float())
        assert y.shape == (5, 3, 64)
        err = (y - ref).abs().max().item()
        assert err <= 1e-3 * ref.abs().max().item(), (dt, err)


def test_clipped_weights_are_counted(tmp_path):
    import coset_amd as ca
    layer = _layer(ca, clip=0.05)
    st = ca.save_packed(layer, str(tmp_path / "c.safetensors"))
    assert st["metadata"]["clipped_weights"] > 0


def test_rejects_block_tiling_and_foreign_files(tmp_path):
    import coset_amd as ca
    from safetensors.torch import save_file
    blk = ca.create_e8_hnlq_linear(32, 8, tiling="block")
    with pytest.raises(ValueError):
        ca.packed_state(blk)
    save_file({"w": torch.zeros(2)}, str(tmp_path / "other.safetensors"), metadata={"coset_amd": '{"format": "x"}'})
    with pytest.raises(ValueError):
        ca.load_packed(str(tmp_path / "other.safetensors"))


@pytest.mark.parametrize("splits", [0, 3])
def test_vlut_epilogue_bias_and_lsq(splits):
    """coset_vlut_linear's epilogue equals the LSQ kernel applied to
    matmul + bias, bit for bit, on the direct write and on the split-K
    reduce path."""
    import coset_amd as ca
    from coset_amd import _lib
    torch.manual_seed(4)
    rows, K, B = 96, 512, 5
    words = ca.hnlq_encode(torch.randn(rows * K // 8, 8, device="cuda") * 2, 4, 2, 1.0).reshape(rows, K // 8, 2)
    prep = ca.vlut_prepare(words, 4)
    a = torch.randn(B, K, device="cuda").to(torch.bfloat16)
    beta = torch.rand(rows, device="cuda") + 0.5
    bias = torch.randn(rows, device="cuda")
    m = ca.LSQActivation(bit_width=6, init_alpha=3.0).cuda()
    try:
        _lib.set_vlut_splits(splits)
        plain = ca.vlut_matmul(prep, a, scale=beta, scale_mode="div")
        fused = ca.vlut_matmul(prep, a, scale=beta, scale_mode="div", bias=bias, act_quant=(m.alpha, m.qmax))
        only_bias = ca.vlut_matmul(prep, a, scale=beta, scale_mode="div", bias=bias)
    finally:
        _lib.set_vlut_splits(0)
    assert torch.equal(only_bias, plain + bias)
    with torch.no_grad():
        assert torch.equal(fused, m(plain + bias))


def test_packed_layer_with_activation_quantizer(tmp_path):
    import coset_amd as ca
    torch.manual_seed(6)
    layer = ca.create_e8_hnlq_linear(256, 64, q=4, M=2, Delta0=1.5, quantize_activations=True, act_bit_width=8,
                                     act_init_alpha=4.0)
    with torch.no_grad():
        layer.weight.normal_(0.0, 0.5)
    x = torch.randn(8, 256, device="cuda").to(torch.bfloat16)
    ca.save_packed(layer, str(tmp_path / "a.safetensors"))
    pl = ca.load_packed(str(tmp_path / "a.safetensors"))
    assert pl.meta["act_bit_width"] == 8 and pl.act_qmax == 127
    y = pl(x)
    with torch.no_grad():
        W_q = pl.dequantized_weight()
        ref = layer.actq(torch.nn.functional.linear(x.float(), W_q, layer.bias.float()))
    s = (4.0 + 1e-8) / 127
    d = (y - ref).abs()
    # the matmul's fp32 order differs from F.linear; LSQ maps a difference
    # across a rounding boundary to one step s
    assert d.max().item() <= s * 1.001 + 1e-5
    assert (d > 1e-5).float().mean().item() < 0.02


def test_saved_words_and_served_output_match_oracle(tmp_path):
    """f1 against the oracle: the file's level words are the oracle's codes
    of the layer quantizer (coset/core/layers.py:428-463) at the saved beta,
    packed as idx(b) = sum_j b_j q^(7-j); the served output equals the
    oracle's one-sided lookup over those words (scale_mode 1: divide by
    beta) plus bias, elementwise within 1e-3 of the summands' magnitude."""
    import coset_amd as ca
    from safetensors import safe_open
    from oracle import oracle as O
    layer = _layer(ca)
    path = str(tmp_path / "o.safetensors")
    ca.save_packed(layer, path)
    with safe_open(path, framework="pt") as f:
        words = f.get_tensor("words").numpy()
        beta = f.get_tensor("beta").numpy()
        bias = f.get_tensor("bias").numpy()
    W = layer.weight.detach().cpu().numpy()
    _, _, codes = O.layer_quant(W, beta, 4, 2, float(layer.weight_clip_value))
    ref_words = O.pack_words(codes, 4).reshape(64, 32, 2)
    np.testing.assert_array_equal(words.astype(np.uint32), ref_words)
    pl = ca.load_packed(path)
    x = torch.randn(7, 256, device="cuda").to(torch.bfloat16)
    y = pl(x).cpu().numpy().astype(np.float64)
    xf = x.float().cpu().numpy()
    ref = O.vlut_matmul(ref_words, beta, xf, 4, 2, scale_mode=1) + bias
    dec = O.e8_decode(codes, 4, 2, 1.0).reshape(64, 256) / beta[:, None]
    mag = np.abs(xf).astype(np.float64) @ np.abs(dec).T.astype(np.float64) + np.abs(bias)
    assert (np.abs(y - ref) <= 1e-3 * mag).all()
