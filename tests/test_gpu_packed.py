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
    for dt in (torch.float16, torch.bfloat16):
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
