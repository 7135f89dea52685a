"""The C ABI library: loads, exports every entry point include/mlcvla.h declares, and
answers host-only queries.  No kernel is launched here (no GPU needed)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT
from mlc_vla import _native as N
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.runtime import Executable

HEADER = os.path.join(ROOT, "include", "mlcvla.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlcv_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = N.load()
    names = _declared()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(N.SIGNATURES)


def test_last_error_and_param_count():
    lib = N.load()
    assert lib.mlcv_last_error() is not None
    for kw, quant in ((dict(dtype="float16"), 0), (dict(dtype="float16"), 1),
                      (dict(paligemma_variant="dummy", action_expert_variant="dummy", dtype="float16"), 0)):
        cfg = Pi0Config(**kw)
        ex = Executable(cfg, ("prefill",), [], "q4f16_1" if quant else None)
        c = ex.c_config()
        n = ctypes.c_int32()
        N.call("mlcv_param_count", ctypes.byref(c), ctypes.byref(n))
        d = cfg.vlm.depth
        want = 18 * d + 11 + (14 * d + 5 if quant else 0)
        assert n.value == want


def test_invalid_config_is_rejected_with_message():
    cfg = Pi0Config(dtype="float16")
    c = Executable(cfg, ("prefill",), []).c_config()
    c.head_dim = 48  # unsupported
    h = ctypes.c_void_p()
    rc = N.load().mlcv_create(ctypes.byref(c), ctypes.byref(h))
    assert rc != 0
    assert b"head_dim" in N.load().mlcv_last_error()


def test_null_arguments_fail_cleanly():
    lib = N.load()
    assert lib.mlcv_prefill(None, None, None, None, None, None) != 0
    assert b"null" in lib.mlcv_last_error()
    with pytest.raises(N.MlcvError):
        N.call("mlcv_denoise_step_kv", *([None] * 10))


def test_vision_and_embedding_queries_and_argument_checks():
    """embed_image's host queries (parameter count, workspace bytes) and the argument checks of
    the newer entry points, all answered before any device call."""
    lib = N.load()
    vc = N.VisionConfig(image_size=224, patch_size=14, num_channels=3, hidden_size=1152, intermediate_size=4304,
                        num_hidden_layers=27, num_attention_heads=16, projection_dim=2048, layer_norm_eps=1e-6)
    n = ctypes.c_int32()
    N.call("mlcv_vision_param_count", ctypes.byref(vc), ctypes.byref(n))
    assert n.value == 3 + 16 * 27 + 4
    nb = ctypes.c_size_t()
    N.call("mlcv_embed_image_workspace", ctypes.byref(vc), ctypes.byref(nb))
    np_, kp = 256, 592
    assert nb.value >= 2 * (np_ * kp + 1152 * kp + np_ * 1152 * 7 + np_ * 4304)
    arr = (ctypes.c_void_p * n.value)()
    with pytest.raises(N.MlcvError, match="null"):
        N.call("mlcv_embed_image", ctypes.byref(vc), arr, n.value, None, None, None, 0, None)
    one = ctypes.c_void_p(16)
    with pytest.raises(N.MlcvError, match="parameter count"):
        N.call("mlcv_embed_image", ctypes.byref(vc), arr, n.value - 1, one, one, one, 0, None)
    with pytest.raises(N.MlcvError, match="null vision parameter"):
        N.call("mlcv_embed_image", ctypes.byref(vc), arr, n.value, one, one, one, nb.value, None)
    with pytest.raises(N.MlcvError, match="bad argument"):
        N.call("mlcv_embed_language", None, 4, None, 10, 8, None, None)
    with pytest.raises(N.MlcvError, match="null"):
        N.call("mlcv_denoise_step", None, None, None, None, None, None)
    with pytest.raises(N.MlcvError, match="bad argument"):
        N.call("mlcv_tile_linear", None, 4, 8, None, 8, None, 0, 0, -1, None)
