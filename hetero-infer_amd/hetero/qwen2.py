"""Qwen2 architecture constants and seeded random-init 4-bit weights under
the reference's tensor names (hetero/cpu_model.py:263-266, :286-289,
:298-299, :320-332).

Weights come from the draws of synth.py that NumPy and torch reproduce bit
for bit (`qlinear_ih_*`, `ih_normal_*`), so a model generated on the host
(fixtures, the NumPy stage) and the same model generated on the GPU (tests
and benchmarks of the device-resident stage, seconds instead of a minute for
28 layers) hold identical bits:
  packed weights  U{0..15} nibbles                    [n_out, n_in/8] uint32
  scales          fp16 |z * 0.02|                     [n_out, n_in/gs]
  biases          fp16 -7.5 * scale + z' * 0.002      [n_out, n_in/gs]
  q/k/v biases    fp32 z * 0.02
  norm weights    fp32 1 + z * 0.02
  KV context      fp16 z                              [n_kv, S, head_dim] per layer
with z an Irwin-Hall normal-like draw (synth.py) from the stream of
(seed, tensor name).  The biases are centred at -7.5 * scale, the mean of
the nibbles, so the dequantised weights have mean zero: with the -8 * scale
of the GEMV benchmarks every weight carries -0.5 * scale, a common mode the
residual stream accumulates over 28 layers until the logits hardly depend on
the input and greedy decoding repeats one token.
"""
from __future__ import annotations

from typing import Dict, List, Tuple

import numpy as np

from . import synth

BIAS_CENTER = 7.5

PROJECTIONS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
               "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def qwen2_7b_config(layers: int = 28) -> dict:
    """Qwen2.5-7B with MLX 4-bit group-64 quantisation."""
    return {"model_type": "qwen2", "hidden_size": 3584, "intermediate_size": 18944,
            "num_hidden_layers": layers, "num_attention_heads": 28, "num_key_value_heads": 4,
            "rms_norm_eps": 1e-6, "rope_theta": 1e6, "vocab_size": 152064,
            "tie_word_embeddings": False, "quantization": {"group_size": 64, "bits": 4}}


def projection_shapes(cfg: dict) -> Dict[str, Tuple[int, int, bool]]:
    """(n_out, n_in, has fp32 bias) of each projection of a layer."""
    h, inter = cfg["hidden_size"], cfg["intermediate_size"]
    kvd = h // cfg["num_attention_heads"] * cfg["num_key_value_heads"]
    return {"self_attn.q_proj": (h, h, True), "self_attn.k_proj": (kvd, h, True),
            "self_attn.v_proj": (kvd, h, True), "self_attn.o_proj": (h, h, False),
            "mlp.gate_proj": (inter, h, False), "mlp.up_proj": (inter, h, False),
            "mlp.down_proj": (h, inter, False)}


def tensor_specs(cfg: dict):
    """(name, kind, shape) of every tensor of the model: kind is 'q4'
    (weight/scales/biases of a 4-bit matrix [n_out, n_in]), 'bias' or 'norm'."""
    h, v = cfg["hidden_size"], cfg["vocab_size"]
    specs = [("model.embed_tokens", "q4", (v, h))]
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}"
        for proj, (n_out, n_in, bias) in projection_shapes(cfg).items():
            specs.append((f"{p}.{proj}", "q4", (n_out, n_in)))
            if bias:
                specs.append((f"{p}.{proj}.bias", "bias", (n_out,)))
        specs.append((f"{p}.input_layernorm.weight", "norm", (h,)))
        specs.append((f"{p}.post_attention_layernorm.weight", "norm", (h,)))
    specs.append(("model.norm.weight", "norm", (h,)))
    if not cfg.get("tie_word_embeddings", False):
        specs.append(("lm_head", "q4", (v, h)))
    return specs


def synthetic_weights(cfg: dict, seed: int = 0) -> Dict[str, np.ndarray]:
    """The model as host NumPy arrays (uint32 weights, float16 scales/biases,
    float32 biases and norms)."""
    gs = cfg["quantization"]["group_size"]
    out: Dict[str, np.ndarray] = {}
    for name, kind, shape in tensor_specs(cfg):
        if kind == "q4":
            w, s, b = synth.qlinear_ih_np(seed, shape[0], shape[1], gs, tag=name + ".", center=BIAS_CENTER)
            out[f"{name}.weight"], out[f"{name}.scales"], out[f"{name}.biases"] = w, s, b
        elif kind == "bias":
            out[name] = synth.ih_normal_np(seed, name, shape[0], 0.02)
        else:
            out[name] = np.float32(1.0) + synth.ih_normal_np(seed, name, shape[0], 0.02)
    return out


def synthetic_weights_torch(cfg: dict, seed: int, device) -> Dict[str, "object"]:
    """The same model generated on a torch device: int32 packed weights,
    float16 scales/biases, float32 biases and norms -- bit for bit the arrays
    of synthetic_weights()."""
    import torch
    gs = cfg["quantization"]["group_size"]
    out = {}
    for name, kind, shape in tensor_specs(cfg):
        if kind == "q4":
            w, s, b = synth.qlinear_ih_torch(seed, shape[0], shape[1], gs, device, tag=name + ".", center=BIAS_CENTER)
            out[f"{name}.weight"] = w
            out[f"{name}.scales"], out[f"{name}.biases"] = s.view(torch.float16), b.view(torch.float16)
        elif kind == "bias":
            out[name] = synth.ih_normal_torch(seed, name, shape[0], 0.02, device)
        else:
            out[name] = synth.ih_normal_torch(seed, name, shape[0], 0.02, device) + 1.0
    return out


def synthetic_context(cfg: dict, context: int, seed: int = 0) -> Tuple[List[np.ndarray], List[np.ndarray]]:
    """Per layer, `context` positions of keys and values already in the
    cache: fp16 [n_kv, context, head_dim]."""
    kh = cfg["num_key_value_heads"]
    d = cfg["hidden_size"] // cfg["num_attention_heads"]
    n = kh * context * d
    ks, vs = [], []
    for i in range(cfg["num_hidden_layers"]):
        ks.append(synth.ih_normal_np(seed, f"kv.{i}.k", n).astype(np.float16).reshape(kh, context, d))
        vs.append(synth.ih_normal_np(seed, f"kv.{i}.v", n).astype(np.float16).reshape(kh, context, d))
    return ks, vs


def synthetic_context_torch(cfg: dict, context: int, seed: int, device):
    """synthetic_context() generated on a torch device (float16 tensors)."""
    import torch
    kh = cfg["num_key_value_heads"]
    d = cfg["hidden_size"] // cfg["num_attention_heads"]
    n = kh * context * d
    ks, vs = [], []
    for i in range(cfg["num_hidden_layers"]):
        ks.append(synth.ih_normal_torch(seed, f"kv.{i}.k", n, 1.0, device).to(torch.float16).reshape(kh, context, d))
        vs.append(synth.ih_normal_torch(seed, f"kv.{i}.v", n, 1.0, device).to(torch.float16).reshape(kh, context, d))
    return ks, vs
