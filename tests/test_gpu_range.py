"""denoise_step_kv at realistic magnitudes against the float32 oracle (gemma_dual.py:60-88
adaRMS, which normalises in fp32 before the modulation).

Random N(0, 0.02) weights keep the residual stream near 1, where no fp16 range question
arises.  Here:
- the residual stream sits near 1e4: action_in_proj's weights are scaled by 5e4, so the
  input projection alone puts the rows' largest entries near 2e4;
- every adaRMS scale lies in [2, 4] (the scale third of each modulation bias), so the
  pre-scaled adaRMS input x * (1 + scale) of the fragment-major path goes past fp16's 65504
  (the test checks that it does) -- the per-norm power-of-two prescale keeps it finite;
- the stand-in prefix keys are 300 x N(0, 1) (entries up to about 1.3e3), so the logits are
  in the hundreds and the softmax is sharply peaked.
The launch chain, the persistent step and the XCD tensor-parallel step, at the tiny size and the full
pi0.5 shape (the XCD step at full size only).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import TINY_KWARGS
from gates import action_gate
from mlc_vla import runtime
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.sample import PiZeroRunner, make_prefix_mask_np, make_rope_np
from oracle import pi0_oracle as O

pytestmark = pytest.mark.gpu

F32 = O.Prec("f32")


def _is_ae(name: str) -> bool:
    return not (".experts.0." in name or ".mlp.0." in name or name.endswith("layernorm.0.weight")
                or name == "backbone.final_norm.0.weight")


class BigStep:
    """One denoise_step_kv with large residuals, adaRMS scales in [2, 4] and large keys."""

    def __init__(self, kw, seed=7):
        self.cfg = Pi0Config(**kw)
        self.d = d = O.dims_from_config(self.cfg)
        self.runner = PiZeroRunner(self.cfg, "rocm")
        g = torch.Generator(device="cuda").manual_seed(seed)
        W = d.ae_width
        p = {}
        for n, s in O.param_specs(d):
            if not _is_ae(n):
                p[n] = torch.empty(s, dtype=torch.float16, device="cuda")  # the step never reads them
                continue
            t = 0.02 * torch.randn(s, generator=g, device="cuda")
            if n == "action_in_proj.weight":
                t = t * 5e4
            elif n.endswith("modulation.bias"):
                t[:W] = 2.0 + 2.0 * torch.rand(W, generator=g, device="cuda")
            p[n] = t.half()
        self.p = p
        self.params = [p[n] for n, _ in self.runner.named_params]
        torch.cuda.synchronize()
        self.host = {n: t.float().cpu().numpy() for n, t in p.items() if _is_ae(n)}
        rng = np.random.default_rng(seed)
        P, hd, kv, D, T, A = d.prefix_len, d.head_dim, d.num_kv_heads, d.depth, d.suffix_len, d.action_dim
        self.keys = (300.0 * rng.standard_normal((D, 1, kv, P, hd))).astype(np.float32)
        self.values = rng.standard_normal((D, 1, kv, P, hd)).astype(np.float16)
        self.x_t = rng.standard_normal((1, T, A)).astype(np.float16)
        self.te = O.sinusoidal_time_emb(0.3, d.ae_width).astype(np.float16)
        valid = P - P // 7
        self.pm = make_prefix_mask_np(P, num_valid=valid)
        self.cos, self.sin = make_rope_np(T, hd, self.cfg.rope_theta, offset=valid)

    def run(self, form: str) -> np.ndarray:
        vm = self.runner.vm
        vm.set_step_form(form)
        dv = lambda a: runtime.tensor(a, self.runner.dev)  # noqa: E731
        args = [dv(a) for a in (self.keys, self.values, self.x_t, self.te, self.cos, self.sin, self.pm)]
        return vm["denoise_step_kv"](*args, self.params).numpy()

    def oracle(self) -> np.ndarray:
        return O.denoise_step_kv(self.host, self.d, self.keys, self.values.astype(np.float32),
                                 self.x_t.astype(np.float32), self.te.astype(np.float32), self.cos, self.sin,
                                 self.pm, F32)


@pytest.fixture(scope="module")
def tiny_big():
    print("range: tiny model", flush=True)
    return BigStep(TINY_KWARGS)


@pytest.fixture(scope="module")
def full_big():
    print("range: full pi0.5 shape", flush=True)
    return BigStep(dict(dtype="float16", action_horizon=50))


@pytest.mark.parametrize("form", ["chain", "persistent", "xtp"])
@pytest.mark.parametrize("which", ["tiny", "full"])
def test_step_at_large_magnitudes_vs_oracle(which, form, tiny_big, full_big):
    if which == "tiny" and form == "xtp":
        pytest.skip("the XCD tensor-parallel step is built for the pi0.5 action expert's shape only")
    s = tiny_big if which == "tiny" else full_big
    print(f"range: {which} {form}", flush=True)
    ref = s.oracle()
    # the setting is what the test says: residual rows near 1e4, and layer 0's pre-scaled
    # adaRMS input x * (1 + scale) past fp16's range
    h = s.host
    x0 = s.x_t.astype(np.float32)[0] @ h["action_in_proj.weight"].T + h["action_in_proj.bias"]
    cond = O.time_cond(h, s.te.astype(np.float32).reshape(1, -1), F32)
    mn = "backbone.layers.0.input_layernorm.1.modulation"
    scale = (cond @ h[mn + ".weight"].T + h[mn + ".bias"])[0, : s.d.ae_width]
    assert 5e3 < np.abs(x0).max() < 6e4
    assert np.abs(x0 * (1.0 + scale)).max() > 65504
    got = s.run(form)
    assert np.all(np.isfinite(got))
    ok, st = action_gate(got, ref)
    print(which, form, st, flush=True)
    assert ok, st
