"""Shared fixtures.  GPU tests are marked ``@pytest.mark.gpu``; everything else runs on CPU."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mlc-vla_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

# The reference's test model (python/tests/conftest.py:21-28) in float16: dummy experts
# (width 64, depth 4, mlp 128, 8 heads, 1 kv head, head_dim 16), prefix 776, horizon 4, 3 steps.
DUMMY_KWARGS = dict(
    paligemma_variant="dummy",
    action_expert_variant="dummy",
    max_token_len=8,
    action_horizon=4,
    num_denoise_steps=3,
    dtype="float16",
)

# The 2-layer CPU-sized model: prefix expert width 256 / MLP 1024, action expert 128 / 512,
# 2 query heads, 1 kv head, head_dim 64, prefix 32, horizon 8, action_dim 32, 10 steps.
TINY_KWARGS = dict(
    paligemma_variant="tiny_vlm",
    action_expert_variant="tiny_action",
    image_keys=(),
    max_token_len=32,
    action_horizon=8,
    action_dim=32,
    num_denoise_steps=10,
    dtype="float16",
)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))
