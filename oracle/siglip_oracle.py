"""numpy restatement of the SigLIP tower + PaliGemma projector (oracle; test infrastructure only).

Follows python/mlc_vla/model/pi0/siglip.py:20-120 (``embed_image``, pi0_model.py:97-99).
``prec="f16"`` keeps the reference's float16 cast points: every Linear rounds its fp32-
accumulated product to fp16 and adds the bias in fp16; LayerNorm computes in fp32 and
casts back (LayerNormF32, siglip.py:20-35); attention scales q in fp16, forms logits and
softmax in fp32, rounds the probabilities to fp16 and accumulates P.V in fp32
(siglip.py:58-70); GELU (tanh form) is evaluated in fp32 on the fp16 input and rounded.
``prec="f64"`` is the same graph in float64 with no roundings.

Pinned by tests/test_oracle_siglip.py: the patch flatten + Linear equals a stride-p conv2d
with the checkpoint's conv weight (torch, float64); layer_norm equals
torch.nn.functional.layer_norm; the attention equals torch scaled_dot_product_attention
(float64); gelu equals torch F.gelu(approximate="tanh").
"""
from __future__ import annotations

import math
from typing import Dict, List, Sequence, Tuple

import numpy as np

from .pi0_oracle import gelu_tanh


def vision_param_specs(cfg) -> List[Tuple[str, Tuple[int, ...]]]:
    """(name, shape) of the vision tower in attribute order (siglip.py:73-90)."""
    s = cfg
    pdim = s.patch_size * s.patch_size * s.num_channels
    out = [("vision.patch_embedding.weight", (s.hidden_size, pdim)), ("vision.patch_embedding.bias", (s.hidden_size,)),
           ("vision.position_embedding", (s.num_patches, s.hidden_size))]
    for i in range(s.num_hidden_layers):
        p = f"vision.layers.{i}."
        for proj in ("q_proj", "k_proj", "v_proj", "out_proj"):
            out += [(f"{p}self_attn.{proj}.weight", (s.hidden_size, s.hidden_size)),
                    (f"{p}self_attn.{proj}.bias", (s.hidden_size,))]
        out += [(p + "mlp.fc1.weight", (s.intermediate_size, s.hidden_size)), (p + "mlp.fc1.bias", (s.intermediate_size,)),
                (p + "mlp.fc2.weight", (s.hidden_size, s.intermediate_size)), (p + "mlp.fc2.bias", (s.hidden_size,))]
        for ln in ("layer_norm1", "layer_norm2"):
            out += [(f"{p}{ln}.weight", (s.hidden_size,)), (f"{p}{ln}.bias", (s.hidden_size,))]
    out += [("vision.post_layernorm.weight", (s.hidden_size,)), ("vision.post_layernorm.bias", (s.hidden_size,)),
            ("vision.multi_modal_projector.weight", (s.projection_dim, s.hidden_size)),
            ("vision.multi_modal_projector.bias", (s.projection_dim,))]
    return out


def _r(x, prec):
    return x.astype(np.float16).astype(np.float32) if prec == "f16" else x


def patchify(image: np.ndarray, p: int) -> np.ndarray:
    """[S, S, C] channels-last -> [num_patches, p*p*C] in (i, j, c) order (siglip.py:97-107)."""
    s, _, c = image.shape
    side = s // p
    x = image.reshape(side, p, side, p, c).transpose(0, 2, 1, 3, 4)
    return x.reshape(side * side, p * p * c)


def linear(x, w, b, prec):
    dt = np.float64 if prec == "f64" else np.float32
    y = _r(x.astype(dt) @ w.astype(dt).T, prec)
    return _r(y + b.astype(dt), prec)


def layer_norm(x, w, b, eps, prec):
    dt = np.float64 if prec == "f64" else np.float32
    x = x.astype(dt)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return _r((x - mu) / np.sqrt(var + dt(eps)) * w.astype(dt) + b.astype(dt), prec)


def attention(q, k, v, heads, prec):
    """[T, H*hd] each -> [T, H*hd] (siglip.py:58-70)."""
    t, width = q.shape
    hd = width // heads
    dt = np.float64 if prec == "f64" else np.float32
    scale = np.float16(hd ** -0.5) if prec == "f16" else hd ** -0.5
    out = np.empty((t, width), dt)
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        qs = (q[:, sl].astype(np.float16) * scale).astype(dt) if prec == "f16" else q[:, sl].astype(dt) * scale
        logits = qs @ k[:, sl].astype(dt).T
        z = np.exp(logits - logits.max(-1, keepdims=True))
        probs = _r(z / z.sum(-1, keepdims=True), prec)
        out[:, sl] = _r(probs @ v[:, sl].astype(dt), prec)
    return out


def embed_image(params: Dict[str, np.ndarray], cfg, image: np.ndarray, prec: str = "f16") -> np.ndarray:
    """One channels-last image [S, S, C] -> [num_patches, projection_dim] (pi0_model.py:97-99)."""
    P = params
    x = linear(patchify(image, cfg.patch_size), P["vision.patch_embedding.weight"], P["vision.patch_embedding.bias"],
               prec)
    x = _r(x + P["vision.position_embedding"].astype(x.dtype), prec)
    for i in range(cfg.num_hidden_layers):
        p = f"vision.layers.{i}."
        h = layer_norm(x, P[p + "layer_norm1.weight"], P[p + "layer_norm1.bias"], cfg.layer_norm_eps, prec)
        q, k, v = (linear(h, P[f"{p}self_attn.{n}.weight"], P[f"{p}self_attn.{n}.bias"], prec)
                   for n in ("q_proj", "k_proj", "v_proj"))
        a = linear(attention(q, k, v, cfg.num_attention_heads, prec), P[p + "self_attn.out_proj.weight"],
                   P[p + "self_attn.out_proj.bias"], prec)
        x = _r(x + a, prec)
        h = layer_norm(x, P[p + "layer_norm2.weight"], P[p + "layer_norm2.bias"], cfg.layer_norm_eps, prec)
        u = linear(h, P[p + "mlp.fc1.weight"], P[p + "mlp.fc1.bias"], prec)
        u = _r(gelu_tanh(u.astype(np.float64 if prec == "f64" else np.float32)), prec)
        x = _r(x + linear(u, P[p + "mlp.fc2.weight"], P[p + "mlp.fc2.bias"], prec), prec)
    h = layer_norm(x, P["vision.post_layernorm.weight"], P["vision.post_layernorm.bias"], cfg.layer_norm_eps, prec)
    return linear(h, P["vision.multi_modal_projector.weight"], P["vision.multi_modal_projector.bias"], prec)


def make_vision_params(cfg, seed: int = 0) -> Dict[str, np.ndarray]:
    """fp16 parameters: Linear weights N(0, 1/fan_in), biases 0.02 N(0,1), LayerNorm
    weights 1 + 0.1 N(0,1), position embedding 0.02 N(0,1)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in vision_param_specs(cfg):
        if len(shape) == 2 and name.endswith(".weight"):
            a = rng.standard_normal(shape) / math.sqrt(shape[1])
        elif "layer_norm" in name and name.endswith(".weight") or "post_layernorm.weight" in name:
            a = 1.0 + 0.1 * rng.standard_normal(shape)
        else:
            a = 0.02 * rng.standard_normal(shape)
        out[name] = a.astype(np.float16)
    return out
