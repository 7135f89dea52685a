"""Host orchestration of the M1 path: prefill once, then N Euler steps (drop-in for mlc_vla.sample).

    runner = PiZeroRunner(Pi0Config(dtype="float16"), "rocm")
    params = runner.to_params(arrays)               # numpy, in runner.named_params order
    actions = runner.sample(params, prefix_embs)    # [1, horizon, action_dim] float32
    actions = runner.sample_graph(params, prefix_embs)

Flow-matching Euler integration as in openpi's sample_actions: dt = -1/N, x = noise,
t = 1; v = velocity(x, t); x = x + dt*v; t += dt (python/mlc_vla/sample.py:1-14,
67-74).  ``sample`` runs the loop on the host around ``denoise_step_kv``;
``sample_graph`` runs it on the device (``denoise_loop_kv``, one captured graph).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple

import numpy as np

from . import runtime
from .compile import _device_for, compile_model
from .model.pi0.pi0_model import KV_FUNCS
from .openpi_ref import sinusoidal_time_emb

_KV_FUNCS = list(KV_FUNCS)


def make_time_embs(num_steps: int, ae_width: int) -> List[np.ndarray]:
    """Sinusoidal embedding of t = 1, 1+dt, ... (t accumulated as a Python float), [1, W] f32 each."""
    dt = -1.0 / num_steps
    out = []
    t = 1.0
    for _ in range(num_steps):
        out.append(sinusoidal_time_emb(t, ae_width))
        t += dt
    return out


def make_rope_np(num_positions: int, head_dim: int, theta: float, offset: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """RoPE tables [1, L, 1, hd/2] f32: angle = pos / theta^((2/hd) i), evaluated in float64."""
    half = head_dim // 2
    pos = offset + np.arange(num_positions, dtype=np.float64)
    inv_ts = theta ** ((2.0 / head_dim) * np.arange(half, dtype=np.float64))
    ang = pos[:, None] / inv_ts[None, :]
    shape = (1, num_positions, 1, half)
    return np.cos(ang).astype(np.float32).reshape(shape), np.sin(ang).astype(np.float32).reshape(shape)


def make_prefix_mask_np(prefix_len: int, num_valid: Optional[int] = None, pad_mask=None,
                        neg: float = -1e9) -> np.ndarray:
    """Additive prefix mask [1,1,1,P] f32: 0 for valid tokens, ``neg`` for padding.

    ``pad_mask`` (0/1 or bool per token) takes precedence over ``num_valid`` (first
    ``num_valid`` tokens valid); with neither, every token is valid.
    """
    if pad_mask is not None:
        valid = np.asarray(pad_mask, dtype=np.float32).reshape(-1)[:prefix_len] > 0
    elif num_valid is not None:
        valid = np.arange(prefix_len) < int(num_valid)
    else:
        valid = np.ones(prefix_len, dtype=bool)
    out = np.full(prefix_len, np.float32(neg), dtype=np.float32)
    out[valid] = 0.0
    return out.reshape(1, 1, 1, prefix_len)


def euler_loop(step_fn, x0: np.ndarray, num_steps: int) -> np.ndarray:
    """Integrate x <- x + dt * v(x, i) in float32 with dt = -1/num_steps."""
    dt = -1.0 / num_steps
    x = np.asarray(x0, dtype=np.float32)
    for i in range(num_steps):
        x = x + dt * np.asarray(step_fn(x, i), dtype=np.float32)
    return x


@dataclass
class _PrefixState:
    keys: "runtime.Tensor"
    values: "runtime.Tensor"
    mask: "runtime.Tensor"
    cos: "runtime.Tensor"
    sin: "runtime.Tensor"


class PiZeroRunner:
    """Prefill + denoise orchestration over the gfx950 kernels (sample.py:77-187)."""

    def __init__(self, config, target: str = "rocm", cuda_graph: bool = False, cublas=None):
        from .compile import resolve_cublas

        self.config = config
        self.target = target
        self.cuda_graph = cuda_graph
        self.cublas = resolve_cublas(cublas, "rocm")
        self.ex, self.named_params = compile_model(config, target, functions=_KV_FUNCS, cuda_graph=cuda_graph,
                                                   cublas=cublas)
        self.dev = _device_for(target)
        self.vm = runtime.VirtualMachine(self.ex, self.dev)

    def to_params(self, arrays):
        """numpy weights (named_params order) -> device tensors."""
        return [runtime.tensor(a, self.dev) for a in arrays]

    def _prefix_state(self, params, prefix_embs: np.ndarray, prefix_pad) -> "_PrefixState":
        """Everything the denoise steps of one chunk read: the prefix K/V cache from prefill,
        the additive prefix mask and the suffix RoPE tables, whose positions start after the
        valid prefix tokens (no pad mask: all of them)."""
        cfg = self.config
        on_dev = lambda a: runtime.tensor(a, self.dev)  # noqa: E731
        mask_np = make_prefix_mask_np(cfg.prefix_len, pad_mask=prefix_pad)
        first_suffix_pos = int(np.count_nonzero(mask_np == 0.0))
        cos_np, sin_np = make_rope_np(cfg.suffix_len, cfg.vlm.head_dim, cfg.rope_theta, offset=first_suffix_pos)
        mask = on_dev(mask_np)
        keys, values = self.vm.prefill(on_dev(np.asarray(prefix_embs, dtype=cfg.dtype)), mask, params)
        return _PrefixState(keys, values, mask, on_dev(cos_np), on_dev(sin_np))

    def _start_noise(self, noise, seed: int) -> np.ndarray:
        """x at t = 1: the caller's noise, else N(0, 1) from numpy's default_rng(seed)."""
        cfg = self.config
        if noise is None:
            noise = np.random.default_rng(seed).standard_normal((1, cfg.action_horizon, cfg.action_dim))
        return np.asarray(noise, dtype=np.float32)

    def sample(self, params, prefix_embs: np.ndarray, noise: Optional[np.ndarray] = None, num_steps: int = 10,
               seed: int = 0, prefix_pad: Optional[np.ndarray] = None) -> np.ndarray:
        """Host Euler loop: one denoise_step_kv per step, host<->device each step."""
        cfg = self.config
        dt = cfg.dtype
        st = self._prefix_state(params, prefix_embs, prefix_pad)
        te_dev = [runtime.tensor(te.astype(dt), self.dev) for te in make_time_embs(num_steps, cfg.action_expert.width)]

        def step_fn(x_np, i):
            x_dev = runtime.tensor(x_np.astype(dt), self.dev)
            v = self.vm["denoise_step_kv"](st.keys, st.values, x_dev, te_dev[i], st.cos, st.sin, st.mask, params)
            return v.numpy()

        return euler_loop(step_fn, self._start_noise(noise, seed), num_steps)

    def sample_graph(self, params, prefix_embs: np.ndarray, noise: Optional[np.ndarray] = None, seed: int = 0,
                     prefix_pad: Optional[np.ndarray] = None) -> np.ndarray:
        """Device Euler loop (denoise_loop_kv): config.num_denoise_steps steps in one call."""
        cfg = self.config
        n = cfg.num_denoise_steps
        st = self._prefix_state(params, prefix_embs, prefix_pad)
        x0 = runtime.tensor(self._start_noise(noise, seed), self.dev)
        tes = np.concatenate(make_time_embs(n, cfg.action_expert.width), axis=0).astype(cfg.dtype)
        out = self.vm["denoise_loop_kv"](st.keys, st.values, x0, runtime.tensor(tes, self.dev), st.cos, st.sin,
                                         st.mask, params)
        return out.numpy()
