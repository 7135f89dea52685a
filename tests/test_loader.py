"""openpi checkpoint loader (pi0_loader.py) on a synthetic PI0Pytorch-style safetensors file.

The fixture lists the checkpoint's key names and shapes for the tiny model. Each tensor
holds distinct random values, so every mapping is checked by value: gate/up stacking order,
adaRMS dense -> modulation, norms copied without +1, the patch conv -> Linear element order,
the tied embedding, and the bf16 / dtype casts.
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from conftest import TINY_KWARGS
from mlc_vla.model.pi0 import Pi0Config, SiglipConfig
from mlc_vla.model.pi0.pi0_loader import build_name_map, load_params, load_safetensors
from mlc_vla.model.pi0.pi0_model import named_params

SIG = SiglipConfig(image_size=28, patch_size=14, hidden_size=16, intermediate_size=24, num_hidden_layers=2,
                   num_attention_heads=2)
PWE = "paligemma_with_expert."
LM = PWE + "paligemma.model.language_model."
EXP = PWE + "gemma_expert.model."
VIS = PWE + "paligemma.model.vision_tower.vision_model."


def _config(**kw) -> Pi0Config:
    return Pi0Config(**{**TINY_KWARGS, "dtype": "float32", "siglip": SIG, **kw})


def _checkpoint(cfg: Pi0Config) -> dict:
    """PI0Pytorch state_dict keys and shapes, written out from the checkpoint format."""
    vlm, ae = cfg.vlm, cfg.action_expert
    hd, nq, nkv = vlm.head_dim, vlm.num_heads, vlm.num_kv_heads
    shapes = {}
    for L in range(vlm.depth):
        for root, ex, ada in ((LM, vlm, False), (EXP, ae, cfg.pi05)):
            p = f"{root}layers.{L}."
            shapes[p + "self_attn.q_proj.weight"] = (nq * hd, ex.width)
            shapes[p + "self_attn.k_proj.weight"] = (nkv * hd, ex.width)
            shapes[p + "self_attn.v_proj.weight"] = (nkv * hd, ex.width)
            shapes[p + "self_attn.o_proj.weight"] = (ex.width, nq * hd)
            shapes[p + "mlp.gate_proj.weight"] = (ex.mlp_dim, ex.width)
            shapes[p + "mlp.up_proj.weight"] = (ex.mlp_dim, ex.width)
            shapes[p + "mlp.down_proj.weight"] = (ex.width, ex.mlp_dim)
            for ln in ("input_layernorm", "post_attention_layernorm"):
                if ada:
                    shapes[f"{p}{ln}.dense.weight"] = (3 * ex.width, ex.width)
                    shapes[f"{p}{ln}.dense.bias"] = (3 * ex.width,)
                else:
                    shapes[f"{p}{ln}.weight"] = (ex.width,)
    shapes[LM + "norm.weight"] = (vlm.width,)
    shapes[EXP + "norm.dense.weight"] = (3 * ae.width, ae.width)
    shapes[EXP + "norm.dense.bias"] = (3 * ae.width,)
    for name, (n, k) in {"action_in_proj": (ae.width, cfg.action_dim), "action_out_proj": (cfg.action_dim, ae.width),
                         "time_mlp_in": (ae.width, ae.width), "time_mlp_out": (ae.width, ae.width)}.items():
        shapes[f"{name}.weight"] = (n, k)
        shapes[f"{name}.bias"] = (n,)
    s = cfg.siglip
    shapes[VIS + "embeddings.patch_embedding.weight"] = (s.hidden_size, s.num_channels, s.patch_size, s.patch_size)
    shapes[VIS + "embeddings.patch_embedding.bias"] = (s.hidden_size,)
    shapes[VIS + "embeddings.position_embedding.weight"] = (s.num_patches, s.hidden_size)
    for i in range(s.num_hidden_layers):
        p = f"{VIS}encoder.layers.{i}."
        for proj in ("q_proj", "k_proj", "v_proj", "out_proj"):
            shapes[f"{p}self_attn.{proj}.weight"] = (s.hidden_size, s.hidden_size)
            shapes[f"{p}self_attn.{proj}.bias"] = (s.hidden_size,)
        shapes[p + "mlp.fc1.weight"], shapes[p + "mlp.fc1.bias"] = (s.intermediate_size, s.hidden_size), (s.intermediate_size,)
        shapes[p + "mlp.fc2.weight"], shapes[p + "mlp.fc2.bias"] = (s.hidden_size, s.intermediate_size), (s.hidden_size,)
        for ln in ("layer_norm1", "layer_norm2"):
            shapes[f"{p}{ln}.weight"], shapes[f"{p}{ln}.bias"] = (s.hidden_size,), (s.hidden_size,)
    shapes[VIS + "post_layernorm.weight"], shapes[VIS + "post_layernorm.bias"] = (s.hidden_size,), (s.hidden_size,)
    proj = PWE + "paligemma.model.multi_modal_projector.linear."
    shapes[proj + "weight"], shapes[proj + "bias"] = (s.projection_dim, s.hidden_size), (s.projection_dim,)
    shapes[PWE + "paligemma.lm_head.weight"] = (257152 // 1024, vlm.width)
    g = torch.Generator().manual_seed(0)
    return {k: torch.randn(v, generator=g) for k, v in shapes.items()}


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    cfg = _config()
    sd = _checkpoint(cfg)
    # the backbone in bf16 as openpi stores it; the heads in float32
    stored = {k: (v.to(torch.bfloat16) if k.startswith(PWE) else v) for k, v in sd.items()}
    path = tmp_path_factory.mktemp("ckpt") / "model.safetensors"
    save_file(stored, str(path))
    return cfg, stored, str(path)


def test_every_named_param_is_built_with_its_shape(ckpt):
    cfg, stored, path = ckpt
    src = load_safetensors(path)
    assert all(a.dtype == np.float32 for a in src.values())
    out = load_params(_config(dtype="float16"), src, named_params=named_params(_config(dtype="float16")))
    names = [n for n, _ in named_params(cfg)]
    assert set(names) <= set(out) and len(names) == len(set(names))
    assert all(out[n].dtype == np.float16 for n in names)
    assert "vision.layers.1.mlp.fc2.weight" in out and "embed_tokens.weight" in out


def test_transforms_by_value(ckpt):
    cfg, stored, path = ckpt
    src = load_safetensors(path)
    out = load_params(cfg, src)
    f32 = lambda k: stored[k].to(torch.float32).numpy()  # noqa: E731
    L = cfg.vlm.depth - 1
    for e, root in ((0, LM), (1, EXP)):
        p = f"{root}layers.{L}."
        gu = out[f"backbone.layers.{L}.mlp.{e}.gate_up_proj.weight"]
        np.testing.assert_array_equal(gu[: gu.shape[0] // 2], f32(p + "mlp.gate_proj.weight"))  # gate first
        np.testing.assert_array_equal(gu[gu.shape[0] // 2:], f32(p + "mlp.up_proj.weight"))
        np.testing.assert_array_equal(out[f"backbone.layers.{L}.self_attn.experts.{e}.k_proj.weight"],
                                      f32(p + "self_attn.k_proj.weight"))
    # expert 0: plain RMSNorm scale as stored (no +1); expert 1 (pi0.5): adaRMS dense -> modulation
    np.testing.assert_array_equal(out[f"backbone.layers.{L}.input_layernorm.0.weight"],
                                  f32(f"{LM}layers.{L}.input_layernorm.weight"))
    np.testing.assert_array_equal(out[f"backbone.layers.{L}.post_attention_layernorm.1.modulation.bias"],
                                  f32(f"{EXP}layers.{L}.post_attention_layernorm.dense.bias"))
    np.testing.assert_array_equal(out["backbone.final_norm.1.modulation.weight"], f32(EXP + "norm.dense.weight"))
    np.testing.assert_array_equal(out["backbone.final_norm.0.weight"], f32(LM + "norm.weight"))
    np.testing.assert_array_equal(out["embed_tokens.weight"], f32(PWE + "paligemma.lm_head.weight"))
    np.testing.assert_array_equal(out["time_mlp_out.bias"], stored["time_mlp_out.bias"].numpy())
    # patch conv [h, c, p, p] -> Linear [h, p*p*c]: column (i*p + j)*c + ch holds conv[h, ch, i, j]
    conv = f32(VIS + "embeddings.patch_embedding.weight")
    lin = out["vision.patch_embedding.weight"]
    h, c, p, _ = conv.shape
    assert lin.shape == (h, p * p * c)
    for (hh, ch, i, j) in [(0, 0, 0, 0), (3, 2, 5, 11), (h - 1, c - 1, p - 1, p - 1), (7, 1, 13, 0)]:
        assert lin[hh, (i * p + j) * c + ch] == conv[hh, ch, i, j]


def test_pi0_without_adarms_maps_plain_norms():
    cfg = _config(pi05=False)
    m = build_name_map(cfg)
    assert "backbone.layers.0.input_layernorm.1.weight" in m
    assert not any(k.endswith("modulation.weight") for k in m)


def test_missing_key_and_wrong_shape_fail_loudly(ckpt):
    cfg, stored, path = ckpt
    src = load_safetensors(path)
    dropped = dict(src)
    del dropped[f"{EXP}layers.0.mlp.up_proj.weight"]
    with pytest.raises(KeyError):
        load_params(cfg, dropped)
    bad = dict(src)
    k = f"{LM}layers.0.self_attn.o_proj.weight"
    bad[k] = bad[k][:, :-1]
    with pytest.raises(ValueError):
        load_params(cfg, bad, named_params=named_params(cfg))


def test_from_openpi_config(tmp_path):
    (tmp_path / "config.json").write_text(json.dumps(
        {"action_dim": 32, "action_horizon": 10, "paligemma_variant": "gemma_2b",
         "action_expert_variant": "gemma_300m", "precision": "bfloat16"}))
    cfg = Pi0Config.from_openpi_config(str(tmp_path), dtype="float16")
    assert (cfg.action_dim, cfg.action_horizon, cfg.dtype) == (32, 10, "float16")
    assert cfg.vlm.width == 2048 and cfg.action_expert.width == 1024
    cfg2 = Pi0Config.from_openpi_config(str(tmp_path / "config.json"), action_horizon=50)
    assert cfg2.action_horizon == 50
