"""Pins of the SigLIP oracle (oracle/siglip_oracle.py) against torch library routines in float64:
patch flatten + Linear == stride-p conv2d with the checkpoint's conv weight (through the
loader's conversion), layer_norm == F.layer_norm, attention == scaled_dot_product_attention."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from mlc_vla.model.pi0 import SiglipConfig
from mlc_vla.model.pi0.pi0_loader import build_name_map
from oracle import siglip_oracle as S

SMALL = SiglipConfig(image_size=28, patch_size=14, hidden_size=144, intermediate_size=200, num_hidden_layers=2,
                     num_attention_heads=2, projection_dim=64)


def test_patch_linear_equals_conv2d():
    rng = np.random.default_rng(0)
    size, p, c, h = 56, 14, 3, 10
    conv_w = rng.standard_normal((h, c, p, p))
    image = rng.standard_normal((size, size, c))
    # the loader's conversion of the checkpoint conv weight
    from mlc_vla.model.pi0.pi0_loader import _patch_conv_as_linear
    lin_w = _patch_conv_as_linear(conv_w)
    ours = S.patchify(image, p) @ lin_w.T
    ref = F.conv2d(torch.from_numpy(image).permute(2, 0, 1)[None], torch.from_numpy(conv_w), stride=p)[0]
    ref = ref.permute(1, 2, 0).reshape(-1, h).numpy()  # patches row-major over (py, px)
    np.testing.assert_allclose(ours, ref, rtol=1e-12, atol=1e-10)


def test_layer_norm_equals_torch():
    rng = np.random.default_rng(1)
    x, w, b = rng.standard_normal((7, 144)) * 3 + 1, rng.standard_normal(144), rng.standard_normal(144)
    ref = F.layer_norm(torch.from_numpy(x), (144,), torch.from_numpy(w), torch.from_numpy(b), eps=1e-6).numpy()
    np.testing.assert_allclose(S.layer_norm(x, w, b, 1e-6, "f64"), ref, rtol=1e-10, atol=1e-12)


def test_attention_equals_sdpa():
    rng = np.random.default_rng(2)
    t, heads, hd = 9, 2, 72
    q, k, v = (rng.standard_normal((t, heads * hd)) for _ in range(3))
    th = lambda a: torch.from_numpy(a).reshape(t, heads, hd).permute(1, 0, 2)  # noqa: E731
    ref = F.scaled_dot_product_attention(th(q), th(k), th(v)).permute(1, 0, 2).reshape(t, heads * hd).numpy()
    np.testing.assert_allclose(S.attention(q, k, v, heads, "f64"), ref, rtol=1e-10, atol=1e-12)


def test_vision_param_names_match_the_loader():
    from mlc_vla.model.pi0 import Pi0Config
    cfg = Pi0Config(dtype="float16", siglip=SMALL)
    names = [n for n, _ in S.vision_param_specs(SMALL)]
    loader = [n for n in build_name_map(cfg) if n.startswith("vision.")]
    assert sorted(names) == sorted(loader) and len(names) == 3 + 16 * SMALL.num_hidden_layers + 4


def test_f16_mode_tracks_f64():
    P = S.make_vision_params(SMALL, 3)
    img = np.random.default_rng(4).standard_normal((28, 28, 3)).astype(np.float16)
    a, b = S.embed_image(P, SMALL, img, "f16"), S.embed_image(P, SMALL, img, "f64")
    assert a.shape == (SMALL.num_patches, SMALL.projection_dim)
    cos = float((a * b).sum() / np.sqrt((a * a).sum() * (b * b).sum()))
    assert cos > 0.9999 and np.abs(a - b).max() < 2e-2 * np.abs(b).max()
