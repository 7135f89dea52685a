"""Host-side input builders shared with openpi (drop-in for the helpers of
mlc_vla.openpi_ref that the M1 path uses)."""

from __future__ import annotations

import math

import numpy as np

_ATTN_NEG_INF = -2.3819763e38  # openpi big_neg


def sinusoidal_time_emb(timestep: float, dim: int, min_period: float = 4e-3,
                        max_period: float = 4.0) -> np.ndarray:
    """[1, dim] float32 = [sin(w t), cos(w t)], w = 2*pi / (min * (max/min)^f), f in linspace(0,1,dim/2).

    Computed in float64 and rounded once (openpi_ref.py:49-58).
    """
    if dim % 2:
        raise ValueError("dim must be even")
    half = dim // 2
    # fractions as numpy's linspace forms them (i * step, last one exactly 1)
    frac = np.arange(half, dtype=np.float64) * (1.0 / (half - 1)) if half > 1 else np.zeros(1)
    frac[-1] = 1.0
    period = min_period * (max_period / min_period) ** frac
    # same operation order as the reference: (1/period * 2) * pi, then * t
    ang = (1.0 / period * 2 * math.pi) * float(timestep)
    out = np.empty((1, dim), np.float64)
    out[0, :half] = np.sin(ang)
    out[0, half:] = np.cos(ang)
    return out.astype(np.float32)


def build_joint_additive_mask(prefix_len: int, suffix_len: int) -> np.ndarray:
    """Joint [1,1,T,T] mask: prefix rows see the prefix, suffix rows see all (openpi_ref.py:61-69)."""
    total = prefix_len + suffix_len
    is_suffix = np.arange(total) >= prefix_len
    allow = is_suffix[:, None] | ~is_suffix[None, :]
    return np.where(allow, 0.0, _ATTN_NEG_INF).astype(np.float32).reshape(1, 1, total, total)
