"""Persistent packed-code format for QAT -> inference hand-off.

The reference exports only the dequantized fp32 weight (export_quantized,
coset/core/layers.py:620-650).  Here a trained HNLQLinearQAT (row tiling,
the fused E8 path) is stored as what it really is: its level words
idx(b) = sum_j b_j q^(7-j) (the reference vLUT index, coset/legacy/quant/
vlut.py:217-238), [out, in/8, M] uint16, and its per-row beta, in a
safetensors file that executes nothing when loaded.  ``PackedLinear`` serves
such a file with the vLUT matmul: y = x @ (decode(words) / beta)^T + bias,
which equals the layer's F.linear(x, W_q, bias) wherever no weight was
clipped at +-weight_clip_value (the count of clipped weights is recorded).
A layer trained with quantize_activations also stores its LSQ parameter
(act_alpha, act_bit_width); the bias add and the activation quantizer then
run in the matmul's epilogue (coset_vlut_linear).
"""
from __future__ import annotations

import json
from typing import Dict, Optional

import torch
from torch import nn

from .codecs import hnlq_decode
from .lattice import on_gpu
from .vlut import vlut_matmul, vlut_prepare

FORMAT = "coset_amd.hnlq_packed.v1"


def packed_state(layer) -> Dict[str, object]:
    """The packed form of a layer's current quantization: tensors (words,
    beta, bias) and metadata.  Uses export_quantized (which, like the
    reference's, advances the layer's step counter once)."""
    if getattr(layer, "tiling", "row") != "row":
        raise ValueError("the packed format stores per-row beta (tiling='row')")
    ex = layer.export_quantized()
    if "codes" not in ex:
        raise ValueError("packed export needs the fused E8 path with quantization enabled")
    words, beta = ex["codes"], ex["beta"]
    q, M = int(layer.q), int(words.shape[-1])
    dec = hnlq_decode(words.reshape(-1, M), q, M, None).reshape(layer.out_features, layer.in_features)
    unclipped = (dec / beta.view(-1, 1))
    clipped = int((unclipped.abs() > float(layer.weight_clip_value)).sum())
    tensors = {"words": words.contiguous(), "beta": beta.contiguous()}
    if layer.bias is not None:
        tensors["bias"] = layer.bias.detach().float().contiguous()
    actq = getattr(layer, "actq", None)
    if getattr(layer, "quantize_activations", False) and actq is not None:
        tensors["act_alpha"] = actq.alpha.detach().float().reshape(1).contiguous()
    meta = {"format": FORMAT, "lattice": "E8", "rule": "core", "q": q, "M": M,
            "in_features": int(layer.in_features), "out_features": int(layer.out_features),
            "weight_clip_value": float(layer.weight_clip_value), "clipped_weights": clipped,
            "scale": "divide: W = decode(words) / beta[row]"}
    if "act_alpha" in tensors:
        meta["act_bit_width"] = int(actq.bit_width)
    return {"tensors": tensors, "metadata": meta}


def save_packed(layer_or_state, path: str) -> Dict[str, object]:
    """Write a layer (or a packed_state) to a safetensors file; returns the state."""
    from safetensors.torch import save_file
    st = layer_or_state if isinstance(layer_or_state, dict) else packed_state(layer_or_state)
    save_file({k: v.detach().cpu().contiguous() for k, v in st["tensors"].items()}, path,
              metadata={"coset_amd": json.dumps(st["metadata"])})
    return st


def load_packed(path: str, device: Optional[torch.device] = None) -> "PackedLinear":
    """Read a file written by save_packed (safetensors: tensors and a JSON
    metadata string, nothing executed) into a PackedLinear on the GPU."""
    from safetensors import safe_open
    tensors = {}
    with safe_open(path, framework="pt") as f:
        meta = json.loads(f.metadata()["coset_amd"])
        for k in f.keys():
            tensors[k] = f.get_tensor(k)
    if meta.get("format") != FORMAT:
        raise ValueError(f"{path}: not a {FORMAT} file")
    return PackedLinear(tensors, meta, device=device)


class PackedLinear(nn.Module):
    """y = x @ (decode(words) / beta)^T + bias through the vLUT matmul, with
    the words prepared once (decoded to bytes in fragment order).  x: [..., in]
    fp16 or bf16, or fp32 (run on the matrix cores as three exact bf16 planes
    where the decoded format applies, else by the LDS-table method) -> fp32.

    Only the prepared weight is resident on the GPU; the raw level words stay
    in host memory (``words``), read by ``dequantized_weight()`` alone."""

    def __init__(self, tensors: Dict[str, torch.Tensor], meta: Dict[str, object],
                 device: Optional[torch.device] = None):
        super().__init__()
        self.meta = dict(meta)
        self.q, self.M = int(meta["q"]), int(meta["M"])
        self.in_features, self.out_features = int(meta["in_features"]), int(meta["out_features"])
        words = on_gpu(tensors["words"]) if device is None else tensors["words"].to(device)
        if words.shape != (self.out_features, self.in_features // 8, self.M):
            raise ValueError(f"words shape {tuple(words.shape)} does not match the metadata")
        self.words = words.cpu()   # host copy: the GPU keeps only the prepared format
        # decoded once to 2 x_hat bytes where they fit (q = 4, M <= 2; q = 2, M <= 4), else cid | idx words
        fits = (self.q == 4 and self.M <= 2) or (self.q == 2 and self.M <= 4)
        self.prepared = vlut_prepare(words, self.q, legacy=False, layout="decoded" if fits else "tiled")
        beta = tensors["beta"]
        if beta.numel() != self.out_features:
            raise ValueError(f"beta holds {beta.numel()} values, expected one per output row "
                             f"({self.out_features})")
        self.register_buffer("beta", beta.reshape(-1).to(words.device).float())
        bias = tensors.get("bias")
        if bias is not None and bias.numel() != self.out_features:
            raise ValueError(f"bias holds {bias.numel()} values, expected {self.out_features}")
        alpha = tensors.get("act_alpha")
        if alpha is not None and ("act_bit_width" not in meta or alpha.numel() != 1):
            raise ValueError("act_alpha needs one value and act_bit_width in the metadata")
        self.register_buffer("bias", None if bias is None else bias.reshape(-1).to(words.device).float())
        self.register_buffer("act_alpha", None if alpha is None else alpha.to(words.device).float())
        self.act_qmax = 2 ** (int(meta["act_bit_width"]) - 1) - 1 if alpha is not None else 0

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """bias and the LSQ activation quantizer (when the layer had one) run
        in the matmul's epilogue."""
        lead = x.shape[:-1]
        a = x.reshape(-1, self.in_features)
        if a.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            a = a.float()   # fp32 runs on the matrix cores as three exact bf16 planes
        aq = None if self.act_alpha is None else (self.act_alpha, self.act_qmax)
        y = vlut_matmul(self.prepared, a, scale=self.beta, scale_mode="div", bias=self.bias, act_quant=aq)
        return y.reshape(*lead, self.out_features)

    def dequantized_weight(self) -> torch.Tensor:
        """decode(words) / beta, [out, in] fp32 (no clamp)."""
        words = self.words.to(self.beta.device)
        dec = hnlq_decode(words.reshape(-1, self.M), self.q, self.M, None)
        return dec.reshape(self.out_features, self.in_features) / self.beta.view(-1, 1)
