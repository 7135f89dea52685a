"""Parameter and signature contract of the pi0.5 M1 functions.

The reference describes the model as a TVM ``nn.Module`` and gets its
``named_params`` from ``export_tvm`` (python/mlc_vla/compile.py:24-38).  Here the
same list is produced directly: names follow the module attribute paths of
Pi0Model / DualExpertGemma (pi0_model.py:81-88, gemma_dual.py:138-148,281-291,
357-371), Linear weights are [out, in], parameters are listed in attribute
definition order (each Linear: weight, then bias).  ``get_default_spec`` gives the
exported signatures (pi0_model.py:197-255).
"""

from __future__ import annotations

import dataclasses
from typing import Dict, List, Optional, Sequence, Tuple

from .pi0_config import Pi0Config

KV_FUNCS = ("prefill", "denoise_step_kv", "denoise_loop_kv")
BACKBONE_FUNCS = ("denoise_step",) + KV_FUNCS
BUILT_FUNCS = ("embed_image", "embed_language") + BACKBONE_FUNCS
PALIGEMMA_VOCAB_SIZE = 257_152  # pi0_model.py:79
_ALL_STAGES = ("vision", "embed", "backbone")


@dataclasses.dataclass(frozen=True)
class Param:
    """Shape/dtype of one parameter (mirrors the ``.shape`` / ``.dtype`` of a TVM nn.Parameter)."""

    shape: Tuple[int, ...]
    dtype: str


@dataclasses.dataclass(frozen=True)
class TensorSpec:
    shape: Tuple[int, ...]
    dtype: str


def include_for(functions) -> set:
    """Sub-modules needed by the exported functions (pi0_model.py:47-59)."""
    if functions is None:
        return set(_ALL_STAGES)
    need = set()
    for f in functions:
        if f == "embed_image":
            need.add("vision")
        elif f == "embed_language":
            need.add("embed")
        elif f in ("denoise_step", "prefill", "denoise_step_kv", "denoise_loop_kv"):
            need.add("backbone")
    return need or set(_ALL_STAGES)


def _linear(out: List[Tuple[str, Tuple[int, ...]]], name: str, n_out: int, n_in: int, bias: bool):
    out.append((f"{name}.weight", (n_out, n_in)))
    if bias:
        out.append((f"{name}.bias", (n_out,)))


def backbone_param_shapes(config: Pi0Config) -> List[Tuple[str, Tuple[int, ...]]]:
    """(name, shape) of backbone + action head + time MLP, in named_params order."""
    vlm, ae = config.vlm, config.action_expert
    n, kv, hd = vlm.num_heads, vlm.num_kv_heads, vlm.head_dim
    experts = [vlm, ae]
    out: List[Tuple[str, Tuple[int, ...]]] = []
    for L in range(vlm.depth):
        p = f"backbone.layers.{L}."
        for e, ex in enumerate(experts):
            a = f"{p}self_attn.experts.{e}."
            _linear(out, a + "q_proj", n * hd, ex.width, False)
            _linear(out, a + "k_proj", kv * hd, ex.width, False)
            _linear(out, a + "v_proj", kv * hd, ex.width, False)
            _linear(out, a + "o_proj", ex.width, n * hd, False)
        for e, ex in enumerate(experts):
            _linear(out, f"{p}mlp.{e}.gate_up_proj", 2 * ex.mlp_dim, ex.width, False)
            _linear(out, f"{p}mlp.{e}.down_proj", ex.width, ex.mlp_dim, False)
        for ln in ("input_layernorm", "post_attention_layernorm"):
            out.append((f"{p}{ln}.0.weight", (vlm.width,)))
            _linear(out, f"{p}{ln}.1.modulation", 3 * ae.width, ae.width, True)
    out.append(("backbone.final_norm.0.weight", (vlm.width,)))
    _linear(out, "backbone.final_norm.1.modulation", 3 * ae.width, ae.width, True)
    _linear(out, "action_in_proj", ae.width, config.action_dim, True)
    _linear(out, "action_out_proj", config.action_dim, ae.width, True)
    _linear(out, "time_mlp_in", ae.width, ae.width, True)
    _linear(out, "time_mlp_out", ae.width, ae.width, True)
    return out


def vision_param_shapes(config: Pi0Config) -> List[Tuple[str, Tuple[int, ...]]]:
    """(name, shape) of the SigLIP tower + projector in attribute order (siglip.py:73-90)."""
    s = config.siglip
    out: List[Tuple[str, Tuple[int, ...]]] = []
    _linear(out, "vision.patch_embedding", s.hidden_size, s.patch_size * s.patch_size * s.num_channels, True)
    out.append(("vision.position_embedding", (s.num_patches, s.hidden_size)))
    for i in range(s.num_hidden_layers):
        p = f"vision.layers.{i}."
        for proj in ("q_proj", "k_proj", "v_proj", "out_proj"):
            _linear(out, f"{p}self_attn.{proj}", s.hidden_size, s.hidden_size, True)
        _linear(out, p + "mlp.fc1", s.intermediate_size, s.hidden_size, True)
        _linear(out, p + "mlp.fc2", s.hidden_size, s.intermediate_size, True)
        for ln in ("layer_norm1", "layer_norm2"):
            out += [(f"{p}{ln}.weight", (s.hidden_size,)), (f"{p}{ln}.bias", (s.hidden_size,))]
    out += [("vision.post_layernorm.weight", (s.hidden_size,)), ("vision.post_layernorm.bias", (s.hidden_size,))]
    _linear(out, "vision.multi_modal_projector", s.projection_dim, s.hidden_size, True)
    return out


def named_params(config: Pi0Config, functions: Optional[Sequence[str]] = None) -> List[Tuple[str, Param]]:
    """``[(name, Param(shape, dtype))]`` as the reference's export_tvm returns them, in attribute
    order: the vision tower, then ``embed_tokens``, then the backbone (pi0_model.py:75-88).
    With ``functions`` None the backbone alone is listed (the M1 functions)."""
    need = include_for(functions)
    out: List[Tuple[str, Param]] = []
    if "vision" in need and functions is not None:
        out += [(name, Param(shape, config.dtype)) for name, shape in vision_param_shapes(config)]
    if "embed" in need and functions is not None:
        out.append(("embed_tokens.weight", Param((PALIGEMMA_VOCAB_SIZE, config.vlm.width), config.dtype)))
    if "backbone" in need:
        out += [(name, Param(shape, config.dtype)) for name, shape in backbone_param_shapes(config)]
    return out


def quantized_named_params(config: Pi0Config, group_size: int = 32, elems_per_word: int = 8,
                           functions: Optional[Sequence[str]] = None) -> List[Tuple[str, Param]]:
    """Parameters after GroupQuantize.quantize_model (quant.py:151-174, :269-288).

    Every Linear ``X.weight`` [N, K] becomes ``X.q_weight`` [N, ceil(K/g)*g/8]
    uint32 and ``X.q_scale`` [N, ceil(K/g)] in the model dtype, keeping ``X.bias``;
    norm weights are unchanged.
    """
    out: List[Tuple[str, Param]] = []
    for name, p in named_params(config, functions):
        if name.endswith(".weight") and len(p.shape) == 2:
            base = name[: -len(".weight")]
            n, k = p.shape
            ng = -(-k // group_size)
            out.append((base + ".q_weight", Param((n, ng * group_size // elems_per_word), "uint32")))
            out.append((base + ".q_scale", Param((n, ng), config.dtype)))
        else:
            out.append((name, p))
    return out


def get_default_spec(config: Pi0Config, functions: Optional[Sequence[str]] = None) -> Dict[str, Dict[str, TensorSpec]]:
    """Input signature of each exported function (pi0_model.py:197-255)."""
    vlm, ae = config.vlm, config.action_expert
    dt = config.dtype
    kv_shape = (vlm.depth, 1, vlm.num_kv_heads, config.prefix_len, vlm.head_dim)
    pm = (1, 1, 1, config.prefix_len)
    rope = (1, config.suffix_len, 1, vlm.head_dim // 2)
    act = (1, config.action_horizon, config.action_dim)
    sg = config.siglip
    spec = {
        "embed_image": {
            "image": TensorSpec((1, sg.image_size, sg.image_size, sg.num_channels), dt),
        },
        "embed_language": {
            "input_ids": TensorSpec((1, config.max_token_len), "int32"),
        },
        "denoise_step": {
            "prefix_embs": TensorSpec((1, config.prefix_len, vlm.width), dt),
            "x_t": TensorSpec(act, dt),
            "time_emb": TensorSpec((1, ae.width), dt),
        },
        "prefill": {
            "prefix_embs": TensorSpec((1, config.prefix_len, vlm.width), dt),
            "prefix_mask": TensorSpec(pm, "float32"),
        },
        "denoise_step_kv": {
            "keys": TensorSpec(kv_shape, "float32"),
            "values": TensorSpec(kv_shape, dt),
            "x_t": TensorSpec(act, dt),
            "time_emb": TensorSpec((1, ae.width), dt),
            "suffix_cos": TensorSpec(rope, "float32"),
            "suffix_sin": TensorSpec(rope, "float32"),
            "prefix_mask": TensorSpec(pm, "float32"),
        },
        "denoise_loop_kv": {
            "keys": TensorSpec(kv_shape, "float32"),
            "values": TensorSpec(kv_shape, dt),
            "x0": TensorSpec(act, "float32"),
            "time_embs": TensorSpec((config.num_denoise_steps, ae.width), dt),
            "suffix_cos": TensorSpec(rope, "float32"),
            "suffix_sin": TensorSpec(rope, "float32"),
            "prefix_mask": TensorSpec(pm, "float32"),
        },
    }
    if functions is not None:
        spec = {k: spec[k] for k in functions}
    return spec
