"""The parity gates can fail: mistakes planted in the oracle (on the CPU) are rejected by the
same gates the GPU results pass (``tests/gates.py``).

At the 2-layer and dummy sizes the attention branch is too small for the action gate to see
(a zeroed attention moves the velocity by about 2e-3), so the gates that carry the
attention's parity are the full-size ones:
- the action gate of the full-size step (config 3 shape) rejects a zeroed attention;
- the per-layer attention-output gate of the full-size step rejects the attention scaled by
  1.1 and the attention reading another layer's K / V (the per-layer residual gate does not see
  the 1.1 scale: with random-init adaRMS gates the attention branch is a few percent of the
  residual stream);
- the per-layer K / V gate of the full-width prefill (P = 968, 800 valid) rejects a zeroed or
  1.1-scaled prefill attention and a key mask that lets the padded keys in;
- the per-kernel gate rejects a joint attention scaled by 1.1 or without its key mask.
Each planted run is in the fp16 cast-point mode, so it carries the rounding noise a GPU
result has, and is compared against the float32 oracle like the GPU result.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gates import action_gate, kernel_gate, kv_gate, rel_gate
from oracle import pi0_oracle as O

F32, F16 = O.Prec("f32"), O.Prec("f16")


def _params(specs, seed):
    g = torch.Generator().manual_seed(seed)
    return {n: (0.02 * torch.randn(s, generator=g)).half().numpy() for n, s in specs}


@pytest.fixture(scope="module")
def step_case():
    """Full pi0.5 action expert (18 layers, width 1024, T = 50) over N(0,1) stand-in K/V, P = 968."""
    d = O.Dims(vlm_width=2048, vlm_mlp=16384, ae_width=1024, ae_mlp=4096, depth=18, num_heads=8,
               num_kv_heads=1, head_dim=256, prefix_len=968, suffix_len=50, action_dim=32)
    ae = [(n, s) for n, s in O.param_specs(d)
          if not (".experts.0." in n or ".mlp.0." in n or n.endswith(".0.weight"))]
    p = _params(ae, 5)
    rng = np.random.default_rng(5)
    keys = rng.standard_normal((18, 1, 1, 968, 256)).astype(np.float32)
    values = rng.standard_normal((18, 1, 1, 968, 256)).astype(np.float16)
    x_t = rng.standard_normal((1, 50, 32)).astype(np.float16)
    te = O.sinusoidal_time_emb(1.0, 1024).astype(np.float16)
    pm = O.make_prefix_mask_np(968)
    cos, sin = O.make_rope_np(50, 256, 10_000.0, offset=968)

    def run(prec, plant=None, k=keys, v=values):
        """velocity, per-layer residual stream and per-layer attention output; ``plant`` maps
        the attention output of every layer (the planted mistake)."""
        xs, att = [], []
        sdpa = O.sdpa

        def hooked(*a, **kw):
            o = sdpa(*a, **kw)
            o = o if plant is None else plant(o)
            att.append(o.copy())
            return o

        O.sdpa = hooked
        try:
            out = O.denoise_step_kv(p, d, k, v, x_t, te, cos, sin, pm, prec,
                                    layer_hook=lambda L, x: xs.append(x.copy()))
        finally:
            O.sdpa = sdpa
        return out, xs, att

    return run, run(F32), (keys, values)


def _layers_fail(xs, ref_xs):
    return [L for L, (a, b) in enumerate(zip(xs, ref_xs)) if not rel_gate(a, b)[0]]


def test_step_gates_pass_an_unplanted_fp16_run(step_case):
    run, (ref, ref_xs, ref_att), _ = step_case
    out, xs, att = run(F16)
    assert action_gate(out, ref)[0], action_gate(out, ref)[1]
    assert _layers_fail(xs, ref_xs) == []
    assert _layers_fail(att, ref_att) == []


def test_step_gates_reject_planted_attention_mistakes(step_case):
    """A zeroed attention fails the action gate; the attention scaled by 1.1 or reading the
    next layer's K / V fails the per-layer attention-output gate in every layer.  (The
    per-layer residual gate alone does not see the 1.1 scale with random-init gates: the
    attention branch is a few percent of the residual stream.)"""
    run, (ref, ref_xs, ref_att), (keys, values) = step_case
    out, _, _ = run(F16, plant=np.zeros_like)
    ok, st = action_gate(out, ref)
    assert not ok, st
    out, xs, att = run(F16, plant=lambda a: (a.astype(np.float32) * 1.1).astype(a.dtype))
    assert _layers_fail(att, ref_att) == list(range(18))
    out, xs, att = run(F16, k=np.roll(keys, 1, axis=0), v=np.roll(values, 1, axis=0))
    assert _layers_fail(att, ref_att) == list(range(18))
    assert not action_gate(out, ref)[0]


@pytest.fixture(scope="module")
def prefill_case():
    """Three layers of the Gemma-2B-shaped prefix expert at P = 968 with 800 valid tokens."""
    d = O.Dims(vlm_width=2048, vlm_mlp=16384, ae_width=1024, ae_mlp=4096, depth=3, num_heads=8,
               num_kv_heads=1, head_dim=256, prefix_len=968, suffix_len=50, action_dim=32)
    e0 = [(n, s) for n, s in O.param_specs(d) if ".experts.0." in n or ".mlp.0." in n or n.endswith(".0.weight")]
    p = _params(e0, 11)
    prefix = np.random.default_rng(3).standard_normal((1, 968, 2048)).astype(np.float16)
    pm = O.make_prefix_mask_np(968, num_valid=800)
    ref = O.prefill(p, d, prefix, pm, F32)
    return d, p, prefix, pm, ref


def _kv_layers_fail(kv, ref):
    return [L for L in range(ref[0].shape[0])
            if not (kv_gate(kv[0][L], ref[0][L])[0] and kv_gate(kv[1][L], ref[1][L])[0])]


def test_prefill_gate_passes_an_unplanted_fp16_run(prefill_case):
    d, p, prefix, pm, ref = prefill_case
    assert _kv_layers_fail(O.prefill(p, d, prefix, pm, F16), ref) == []


@pytest.mark.parametrize("mistake", ["zero", "scale", "nomask"])
def test_prefill_gate_rejects_planted_attention_mistakes(prefill_case, monkeypatch, mistake):
    d, p, prefix, pm, ref = prefill_case
    sdpa = O.sdpa
    if mistake == "zero":
        monkeypatch.setattr(O, "sdpa", lambda *a, **k: np.zeros_like(sdpa(*a, **k)))
    elif mistake == "scale":
        monkeypatch.setattr(O, "sdpa", lambda *a, **k: (sdpa(*a, **k).astype(np.float32) * 1.1).astype(np.float16))
    else:
        monkeypatch.setattr(O, "sdpa", lambda q, k, v, mask, *a, **kw: sdpa(q, k, v, None, *a, **kw))
    fails = _kv_layers_fail(O.prefill(p, d, prefix, pm, F16), ref)
    assert fails and fails[0] == 1, fails  # layer 0's K/V do not see the attention; layer 1's do


def test_kernel_gate_rejects_planted_attention_mistakes():
    """The isolated joint attention at the config-2 shape (8 heads, hd 256, 968 prefix keys with
    900 valid, 50 suffix keys): x 1.1 and a dropped key mask fail the per-kernel gate, the
    fp16 cast-point oracle passes it."""
    rng = np.random.default_rng(2)
    s = 1.0 / 16.0
    q = rng.standard_normal((50, 8, 256)) * s
    k = np.concatenate([rng.standard_normal((968, 1, 256)), rng.standard_normal((50, 1, 256))]) * s
    v = np.concatenate([rng.standard_normal((968, 1, 256)), rng.standard_normal((50, 1, 256))]) * s
    mask = np.concatenate([np.where(np.arange(968) < 900, 0.0, -1e9), np.zeros(50)])
    F64 = O.Prec("f64")
    ref = O.sdpa(q, k, v, mask, F64)
    f16 = O.sdpa(q.astype(np.float32), k.astype(np.float32), v.astype(np.float16), mask, F16)
    assert kernel_gate(f16, ref)[0], kernel_gate(f16, ref)[1]
    assert not kernel_gate(1.1 * ref, ref)[0]
    assert not kernel_gate(O.sdpa(q, k, v, None, F64), ref)[0]
