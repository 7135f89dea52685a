"""Host-side contract of the drop-in API (no GPU): helpers bit-equal to the oracle,
the Pi0Config contract (as python/tests/test_config_interface.py:21-73), parameter
naming against the oracle's independent spec, and loud failure without the HIP path."""

from __future__ import annotations

import json

import numpy as np
import pytest

from conftest import DUMMY_KWARGS, TINY_KWARGS
from mlc_vla import openpi_ref, sample
from mlc_vla.compile import compile_model
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.model.pi0.pi0_model import get_default_spec, named_params, quantized_named_params
from oracle import pi0_oracle as O
from oracle import q4_oracle as Q


@pytest.mark.parametrize("n,w", [(10, 1024), (3, 64), (7, 128)])
def test_time_embs_match_oracle(n, w):
    for a, b in zip(sample.make_time_embs(n, w), O.make_time_embs(n, w)):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("L,hd,off", [(50, 256, 968), (8, 64, 32), (4, 16, 0)])
def test_rope_tables_match_oracle(L, hd, off):
    for a, b in zip(sample.make_rope_np(L, hd, 10_000.0, off), O.make_rope_np(L, hd, 10_000.0, off)):
        np.testing.assert_array_equal(a, b)


def test_prefix_masks_match_oracle():
    pad = np.array([1, 1, 0, 1, 0, 0, 1, 0], np.float32)
    for kw in ({}, {"num_valid": 5}, {"pad_mask": pad}, {"num_valid": 2, "pad_mask": pad}):
        np.testing.assert_array_equal(sample.make_prefix_mask_np(8, **kw), O.make_prefix_mask_np(8, **kw))


def test_euler_and_joint_mask_match_oracle():
    rng = np.random.default_rng(0)
    x0 = rng.standard_normal((1, 4, 32)).astype(np.float32)
    vs = [rng.standard_normal((1, 4, 32)).astype(np.float32) for _ in range(5)]
    np.testing.assert_array_equal(sample.euler_loop(lambda x, i: vs[i] * x, x0, 5),
                                  O.euler_loop(lambda x, i: vs[i] * x, x0, 5))
    np.testing.assert_array_equal(openpi_ref.build_joint_additive_mask(6, 3),
                                  O.build_additive_mask(6, 3, -2.3819763e38, np.float32))


def test_default_config_derived_shapes():
    cfg = Pi0Config()
    assert cfg.num_images == 3
    assert cfg.prefix_len == 3 * 256 + 200 == 968
    assert cfg.suffix_len == cfg.action_horizon == 10
    assert cfg.attn_logits_dtype == "float32"
    assert cfg.vlm.head_dim == cfg.action_expert.head_dim


def test_from_openpi_config_reads_json_and_overrides(tmp_path):
    (tmp_path / "config.json").write_text(json.dumps({
        "action_dim": 7, "action_horizon": 5, "paligemma_variant": "dummy",
        "action_expert_variant": "dummy", "precision": "bfloat16"}))
    cfg = Pi0Config.from_openpi_config(str(tmp_path), dtype="float16", attn_logits_dtype="float16")
    assert (cfg.action_dim, cfg.action_horizon, cfg.paligemma_variant) == (7, 5, "dummy")
    assert cfg.dtype == "float16" and cfg.attn_logits_dtype == "float16" and cfg.suffix_len == 5
    assert Pi0Config.from_openpi_config(str(tmp_path / "config.json")).action_dim == 7


def test_dual_expert_mismatch_rejected():
    with pytest.raises(AssertionError):
        Pi0Config(paligemma_variant="gemma_2b", action_expert_variant="dummy")


def test_tiny_config_shapes():
    cfg = Pi0Config(**TINY_KWARGS)
    assert cfg.prefix_len == 32 and cfg.suffix_len == 8
    assert (cfg.vlm.width, cfg.vlm.mlp_dim, cfg.action_expert.width, cfg.action_expert.mlp_dim) == (256, 1024, 128, 512)
    assert (cfg.vlm.num_heads, cfg.vlm.num_kv_heads, cfg.vlm.head_dim, cfg.vlm.depth) == (2, 1, 64, 2)


@pytest.mark.parametrize("kw", [DUMMY_KWARGS, TINY_KWARGS, dict(dtype="float16")], ids=["dummy", "tiny", "pi05"])
def test_named_params_match_oracle_specs(kw):
    cfg = Pi0Config(**kw)
    npar = named_params(cfg)
    specs = O.param_specs(O.dims_from_config(cfg))
    assert [(n, tuple(p.shape)) for n, p in npar] == [(n, tuple(s)) for n, s in specs]
    assert all(p.dtype == "float16" for _, p in npar)
    assert len(npar) == 18 * cfg.vlm.depth + 11  # 335 for pi0.5
    qn = quantized_named_params(cfg)
    assert [(n, tuple(p.shape), p.dtype) for n, p in qn] == [(n, tuple(s), t) for n, s, t in Q.quantized_specs(specs)]


def test_default_spec_signatures():
    cfg = Pi0Config(dtype="float16", action_horizon=50)
    s = get_default_spec(cfg)
    assert s["denoise_step_kv"]["keys"].shape == (18, 1, 1, 968, 256)
    assert s["denoise_step_kv"]["keys"].dtype == "float32"
    assert s["denoise_step_kv"]["values"].dtype == "float16"
    assert s["denoise_step_kv"]["suffix_cos"].shape == (1, 50, 1, 128)
    assert s["denoise_loop_kv"]["x0"].dtype == "float32"
    assert s["denoise_loop_kv"]["time_embs"].shape == (10, 1024)
    assert s["prefill"]["prefix_embs"].shape == (1, 968, 2048)


def test_compile_targets_and_dtypes():
    """CPU targets are refused; float32 models (the reference's default dtype) build the M1
    functions, float16 ones every function, and q4f16_1 quantizes float16 models only."""
    from mlc_vla.compile_quant import compile_model_quant

    with pytest.raises(NotImplementedError):
        compile_model(Pi0Config(**DUMMY_KWARGS), "c")
    f32 = Pi0Config(**{**DUMMY_KWARGS, "dtype": "float32"})
    ex, npar = compile_model(f32, "rocm")
    assert ex.functions == ("prefill", "denoise_step_kv", "denoise_loop_kv")
    assert all(sp.dtype == "float32" for _, sp in npar)
    assert ex.c_config().dtype == 2  # MLCV_DTYPE_F32
    with pytest.raises(NotImplementedError):
        compile_model(f32, "rocm", functions=["denoise_step"])
    with pytest.raises(NotImplementedError):
        compile_model_quant(f32, "rocm", None, "q4f16_1")
    with pytest.raises(NotImplementedError):
        compile_model(Pi0Config(**{**DUMMY_KWARGS, "dtype": "bfloat16"}), "rocm")
    ex, npar = compile_model(Pi0Config(**DUMMY_KWARGS), "rocm")
    assert len(npar) == 18 * 4 + 11 and ex.functions == ("prefill", "denoise_step_kv", "denoise_loop_kv")
    assert ex.c_config().dtype == 1  # MLCV_DTYPE_F16
