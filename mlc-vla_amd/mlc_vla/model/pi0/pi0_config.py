"""Configuration of the pi0.5 model (drop-in for mlc_vla.model.pi0.pi0_config).

Same fields, defaults, derived sizes and checks as the reference
(python/mlc_vla/model/pi0/pi0_config.py:15-170).  One extension: an expert
variant may be given as a ``GemmaExpertConfig`` instance (or one of the extra
named variants below) so that shapes outside the reference's three variants,
such as the 2-layer width-256/128 model used as the CPU-sized case, can be
described without new code.
"""

from __future__ import annotations

import dataclasses
import json
import os
from typing import Dict, List, Tuple, Union


@dataclasses.dataclass
class GemmaExpertConfig:
    """One Gemma expert (openpi ``gemma.Config``), pi0_config.py:15-44.

    The two experts must share head_dim / num_heads / num_kv_heads / depth for
    the joint attention.
    """

    width: int
    depth: int
    mlp_dim: int
    num_heads: int
    num_kv_heads: int
    head_dim: int

    @staticmethod
    def from_variant(variant: Union[str, "GemmaExpertConfig"]) -> "GemmaExpertConfig":
        if isinstance(variant, GemmaExpertConfig):
            return variant
        if variant in _VARIANTS:
            return dataclasses.replace(_VARIANTS[variant])
        raise ValueError(f"Unknown gemma variant: {variant}")


_VARIANTS: Dict[str, GemmaExpertConfig] = {
    # reference variants (pi0_config.py:30-44)
    "gemma_2b": GemmaExpertConfig(width=2048, depth=18, mlp_dim=16_384, num_heads=8, num_kv_heads=1, head_dim=256),
    "gemma_300m": GemmaExpertConfig(width=1024, depth=18, mlp_dim=4096, num_heads=8, num_kv_heads=1, head_dim=256),
    "dummy": GemmaExpertConfig(width=64, depth=4, mlp_dim=128, num_heads=8, num_kv_heads=1, head_dim=16),
    # 2-layer CPU-sized model: prefix expert width 256 / MLP 1024, action expert width 128 / MLP 512
    "tiny_vlm": GemmaExpertConfig(width=256, depth=2, mlp_dim=1024, num_heads=2, num_kv_heads=1, head_dim=64),
    "tiny_action": GemmaExpertConfig(width=128, depth=2, mlp_dim=512, num_heads=2, num_kv_heads=1, head_dim=64),
}


@dataclasses.dataclass
class SiglipConfig:
    """SigLIP So400m/14 (only its patch count enters prefix_len here)."""

    image_size: int = 224
    patch_size: int = 14
    num_channels: int = 3
    hidden_size: int = 1152
    intermediate_size: int = 4304
    num_hidden_layers: int = 27
    num_attention_heads: int = 16
    layer_norm_eps: float = 1e-6
    projection_dim: int = 2048

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def num_patches(self) -> int:
        side = self.image_size // self.patch_size
        return side * side


@dataclasses.dataclass
class Pi0Config:
    """pi0.5 top-level configuration (pi0_config.py:72-170)."""

    paligemma_variant: Union[str, GemmaExpertConfig] = "gemma_2b"
    action_expert_variant: Union[str, GemmaExpertConfig] = "gemma_300m"

    action_dim: int = 32
    action_horizon: int = 10
    max_token_len: int = 200

    pi05: bool = True
    siglip: SiglipConfig = dataclasses.field(default_factory=SiglipConfig)
    image_keys: Tuple[str, ...] = ("base_0_rgb", "left_wrist_0_rgb", "right_wrist_0_rgb")

    dtype: str = "float32"
    attn_logits_dtype: str = "float32"
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10_000.0
    attn_neg_inf: float = -2.3819763e38
    time_min_period: float = 4e-3
    time_max_period: float = 4.0

    num_denoise_steps: int = 10

    kwargs: Dict[str, object] = dataclasses.field(default_factory=dict)

    @property
    def vlm(self) -> GemmaExpertConfig:
        return GemmaExpertConfig.from_variant(self.paligemma_variant)

    @property
    def action_expert(self) -> GemmaExpertConfig:
        return GemmaExpertConfig.from_variant(self.action_expert_variant)

    @property
    def num_images(self) -> int:
        return len(self.image_keys)

    @property
    def prefix_len(self) -> int:
        """image tokens + language tokens (pi0_config.py:129-131)."""
        return self.num_images * self.siglip.num_patches + self.max_token_len

    @property
    def suffix_len(self) -> int:
        """pi0.5 suffix = action tokens only (pi0_config.py:134-136)."""
        return self.action_horizon

    def experts(self) -> List[GemmaExpertConfig]:
        return [self.vlm, self.action_expert]

    @classmethod
    def from_openpi_config(cls, path: str, **overrides) -> "Pi0Config":
        """Read action_dim / action_horizon / variants from a checkpoint's config.json
        (directory or file), then apply ``overrides`` (pi0_config.py:141-163)."""
        if os.path.isdir(path):
            path = os.path.join(path, "config.json")
        with open(path) as f:
            raw = json.load(f)
        kw: Dict[str, object] = {}
        for key in ("action_dim", "action_horizon", "paligemma_variant", "action_expert_variant"):
            if key in raw:
                kw[key] = raw[key]
        kw.update(overrides)
        return cls(**kw)

    def __post_init__(self):
        a, b = self.vlm, self.action_expert
        assert a.head_dim == b.head_dim, "dual experts must share head_dim"
        assert a.num_heads == b.num_heads, "dual experts must share num_heads"
        assert a.num_kv_heads == b.num_kv_heads, "dual experts must share num_kv_heads"
        assert a.depth == b.depth, "dual experts must share depth"
