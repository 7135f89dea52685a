"""openpi checkpoint -> mlc-vla parameter names (pi0_loader.py:1-203).

The source is the state_dict of openpi's PyTorch pi0 / pi0.5 model (``PI0Pytorch``),
usually stored as safetensors. The key names form a format, so they match the
checkpoint's; the transforms are those the reference applies:

- q/k/v/o projections and down_proj are copied. gate_proj and up_proj are stacked into
  ``gate_up_proj`` as [gate; up] along the output rows (pi0_loader.py:56-58, 130-134).
- Plain RMSNorm scales are copied as stored: the forward applies ``1 + w``.
- adaRMS norms (the action expert of pi0.5) take their ``dense`` Linear as ``modulation``
  (pi0_loader.py:137-150).
- ``embed_tokens`` is tied to ``lm_head`` (pi0_loader.py:75-76, 117).
- The SigLIP patch conv [hidden, c, p, p] becomes a Linear [hidden, p*p*c] in (p, p, c)
  order (pi0_loader.py:61-65).
"""

from __future__ import annotations

from typing import Callable, Dict, Iterator, Optional, Sequence, Tuple

import numpy as np

from .pi0_config import Pi0Config

_PWE = "paligemma_with_expert."
_PALI = _PWE + "paligemma.model."
_EXPERT_ROOT = (_PALI + "language_model.", _PWE + "gemma_expert.model.")  # expert 0, expert 1
_VISION = _PALI + "vision_tower.vision_model."
_PROJECTOR = _PALI + "multi_modal_projector.linear."
_LM_HEAD = _PWE + "paligemma.lm_head.weight"


class SourceSpec:
    """How one target parameter is built: the source keys and a function of their arrays."""

    def __init__(self, keys, fn: Optional[Callable[..., np.ndarray]] = None):
        self.keys = [keys] if isinstance(keys, str) else list(keys)
        self.fn = fn

    def build(self, src: Dict[str, np.ndarray]) -> np.ndarray:
        arrays = [src[k] for k in self.keys]
        return self.fn(*arrays) if self.fn is not None else arrays[0]


def _stack_rows(*parts: np.ndarray) -> np.ndarray:
    return np.concatenate(parts, axis=0)


def _patch_conv_as_linear(w: np.ndarray) -> np.ndarray:
    hidden, c, p, q = w.shape
    return np.ascontiguousarray(w.transpose(0, 2, 3, 1)).reshape(hidden, p * q * c)


def _vision_entries(config: Pi0Config) -> Iterator[Tuple[str, SourceSpec]]:
    yield "vision.patch_embedding.weight", SourceSpec(_VISION + "embeddings.patch_embedding.weight",
                                                      _patch_conv_as_linear)
    yield "vision.patch_embedding.bias", SourceSpec(_VISION + "embeddings.patch_embedding.bias")
    yield "vision.position_embedding", SourceSpec(_VISION + "embeddings.position_embedding.weight")
    for i in range(config.siglip.num_hidden_layers):
        src, dst = f"{_VISION}encoder.layers.{i}.", f"vision.layers.{i}."
        leaves = [f"self_attn.{p}" for p in ("q_proj", "k_proj", "v_proj", "out_proj")]
        leaves += ["mlp.fc1", "mlp.fc2", "layer_norm1", "layer_norm2"]
        for leaf in leaves:
            for kind in ("weight", "bias"):
                yield f"{dst}{leaf}.{kind}", SourceSpec(f"{src}{leaf}.{kind}")
    for kind in ("weight", "bias"):
        yield f"vision.post_layernorm.{kind}", SourceSpec(f"{_VISION}post_layernorm.{kind}")
        yield f"vision.multi_modal_projector.{kind}", SourceSpec(f"{_PROJECTOR}{kind}")


def _norm_entries(dst: str, src: str, ada: bool) -> Iterator[Tuple[str, SourceSpec]]:
    if ada:
        yield f"{dst}.modulation.weight", SourceSpec(f"{src}.dense.weight")
        yield f"{dst}.modulation.bias", SourceSpec(f"{src}.dense.bias")
    else:
        yield f"{dst}.weight", SourceSpec(f"{src}.weight")


def _backbone_entries(config: Pi0Config) -> Iterator[Tuple[str, SourceSpec]]:
    ada = (False, config.pi05)  # adaRMS only on the action expert, and only for pi0.5
    for L in range(config.vlm.depth):
        dst = f"backbone.layers.{L}."
        for e in (0, 1):
            src = f"{_EXPERT_ROOT[e]}layers.{L}."
            for proj in ("q_proj", "k_proj", "v_proj", "o_proj"):
                yield f"{dst}self_attn.experts.{e}.{proj}.weight", SourceSpec(f"{src}self_attn.{proj}.weight")
            yield f"{dst}mlp.{e}.gate_up_proj.weight", SourceSpec(
                (f"{src}mlp.gate_proj.weight", f"{src}mlp.up_proj.weight"), _stack_rows)
            yield f"{dst}mlp.{e}.down_proj.weight", SourceSpec(f"{src}mlp.down_proj.weight")
            for ln in ("input_layernorm", "post_attention_layernorm"):
                yield from _norm_entries(f"{dst}{ln}.{e}", f"{src}{ln}", ada[e])
    for e in (0, 1):
        yield from _norm_entries(f"backbone.final_norm.{e}", f"{_EXPERT_ROOT[e]}norm", ada[e])
    for head in ("action_in_proj", "action_out_proj", "time_mlp_in", "time_mlp_out"):
        for kind in ("weight", "bias"):
            yield f"{head}.{kind}", SourceSpec(f"{head}.{kind}")


def build_name_map(config: Pi0Config) -> Dict[str, SourceSpec]:
    """Target parameter name -> SourceSpec for the vision tower, embed_tokens, both experts
    of the backbone, the action head and the time MLP (pi0_loader.py:83-156)."""
    out: Dict[str, SourceSpec] = dict(_vision_entries(config))
    out["embed_tokens.weight"] = SourceSpec(_LM_HEAD)
    out.update(_backbone_entries(config))
    return out


def load_safetensors(path: str, dtype: str = "float32") -> Dict[str, np.ndarray]:
    """Read a PI0Pytorch safetensors file into numpy arrays of ``dtype`` (bf16 / fp16 go
    through float32) (pi0_loader.py:159-171).  Only the tensor data is read."""
    import torch
    from safetensors.torch import load_file

    out: Dict[str, np.ndarray] = {}
    for k, v in load_file(path).items():
        if v.dtype in (torch.bfloat16, torch.float16):
            v = v.to(torch.float32)
        out[k] = v.numpy().astype(np.dtype(dtype), copy=False)
    return out


def load_params(config: Pi0Config, src: Dict[str, np.ndarray], named_params: Optional[Sequence] = None,
                dtype: Optional[str] = None) -> Dict[str, np.ndarray]:
    """Build every mapped parameter from ``src`` and cast floats to ``dtype`` (default the
    config's dtype) (pi0_loader.py:174-203).  With ``named_params`` ([(name, param)] as
    ``PiZeroRunner.named_params``), every listed name must be built with the listed shape;
    extra built names (the vision tower when only the backbone is compiled) are allowed."""
    target = np.dtype(dtype or config.dtype)
    params: Dict[str, np.ndarray] = {}
    for name, spec in build_name_map(config).items():
        a = spec.build(src)
        params[name] = a if np.issubdtype(a.dtype, np.integer) else a.astype(target, copy=False)
    if named_params is not None:
        missing = [n for n, _ in named_params if n not in params]
        if missing:
            raise KeyError(f"the loader builds no {len(missing)} listed parameter(s), e.g. {missing[:5]}")
        for n, p in named_params:
            want, got = tuple(int(s) for s in p.shape), tuple(params[n].shape)
            if want != got:
                raise ValueError(f"parameter {n}: loader shape {got} vs model shape {want}")
    return params
