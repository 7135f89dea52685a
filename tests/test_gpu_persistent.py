"""The persistent step (one launch per denoise_step_kv, csrc/step_persistent.hip) against the
oracle, op by op and layer by layer, through the probes of the last step's intermediates.

Per op, the oracle is fed the GPU's own inputs of that op, so each check isolates the kernel
code of one phase (pi0_model.py:142-163; gemma_dual.py:60-94 adaRMS / gated residual,
:97-122 _sdpa, :125-135 GeGLU MLP, :255-275 attn_decode_e1, :343-351 decode_e1):
- q / k / v: adaRMS (input) + projections + RoPE on the GPU's residual and modulations;
- attention: float64 SDPA over [prefix K/V ; the GPU's suffix k/v] with the GPU's q (the
  per-kernel gate);
- o_proj / down: the gated residual on the GPU's attention / GeGLU output;
- gate_up: adaRMS (post) + GeGLU on the GPU's residual;
- head: final adaRMS + action_out.
Then the whole chain: every layer's residual stream and attention output against the float32
oracle's (the gates the ablation tests show reject a zeroed, 1.1-scaled or misrouted
attention), and the velocity against the action gate.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import TINY_KWARGS, cosine, max_abs
from gates import action_gate, kernel_gate, rel_gate
from mlc_vla import _native as N
from mlc_vla import runtime
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.sample import PiZeroRunner, make_prefix_mask_np, make_rope_np, make_time_embs
from oracle import pi0_oracle as O

pytestmark = pytest.mark.gpu

F32, F16, F64 = O.Prec("f32"), O.Prec("f16"), O.Prec("f64")


def _is_ae(name: str) -> bool:
    return not (".experts.0." in name or ".mlp.0." in name or name.endswith("layernorm.0.weight")
                or name == "backbone.final_norm.0.weight")


class Step:
    """One denoise_step_kv on the GPU with random-init weights and N(0,1) stand-in K/V."""

    def __init__(self, kw, seed=3, kv_seed=5):
        self.cfg = Pi0Config(**kw)
        self.d = O.dims_from_config(self.cfg)
        self.runner = PiZeroRunner(self.cfg, "rocm")
        self.runner.vm.set_persist(True)
        d = self.d
        g = torch.Generator(device="cuda").manual_seed(seed)
        specs = O.param_specs(d)
        self.p = {n: ((0.02 * torch.randn(s, generator=g, device="cuda")).half() if _is_ae(n)
                      else torch.empty(s, dtype=torch.float16, device="cuda")) for n, s in specs}
        self.params = [self.p[n] for n, _ in self.runner.named_params]
        torch.cuda.synchronize()
        self.host = {n: t.cpu().numpy() for n, t in self.p.items() if _is_ae(n)}
        rng = np.random.default_rng(kv_seed)
        P, hd, kv, D, T, A = d.prefix_len, d.head_dim, d.num_kv_heads, d.depth, d.suffix_len, d.action_dim
        self.keys = rng.standard_normal((D, 1, kv, P, hd)).astype(np.float32)
        self.values = rng.standard_normal((D, 1, kv, P, hd)).astype(np.float16)
        self.x_t = rng.standard_normal((1, T, A)).astype(np.float16)
        self.te = O.sinusoidal_time_emb(0.6, d.ae_width).astype(np.float16)
        valid = P - P // 9
        self.pm = make_prefix_mask_np(P, num_valid=valid)
        self.cos, self.sin = make_rope_np(T, hd, self.cfg.rope_theta, offset=valid)
        dv = lambda a: runtime.tensor(a, self.runner.dev)  # noqa: E731
        self.args = [dv(a) for a in (self.keys, self.values, self.x_t, self.te, self.cos, self.sin, self.pm)]

    def run(self):
        return self.runner.vm["denoise_step_kv"](*self.args, self.params).numpy()

    def probe(self, what, layer):
        d, T = self.d, self.d.suffix_len
        nq, nkv = d.num_heads * d.head_dim, d.num_kv_heads * d.head_dim
        shape, dt = {"x": ((T, d.ae_width), np.float16), "x_mid": ((T, d.ae_width), np.float16),
                     "q": ((T, nq), np.float32), "k": ((T, nkv), np.float32), "v": ((T, nkv), np.float16),
                     "attn": ((T, nq), np.float16), "h": ((T, d.ae_mlp), np.float16),
                     "mod": ((2 * d.depth + 1, 3 * d.ae_width), np.float16)}[what]
        return self.runner.vm.probe(what, layer, shape, dt)


def _per_op_checks(s: Step, v_gpu):
    d, T = s.d, s.d.suffix_len
    n, kv, hd = d.num_heads, d.num_kv_heads, d.head_dim
    P = s.host
    mods = s.probe("mod", 0)
    ref_mods = O.all_modulations(P, d, O.time_cond(P, s.te.reshape(1, -1), F32), F32)
    ok, st = rel_gate(mods, np.concatenate(ref_mods, 0), rel=2e-3, cos=0.99999)
    assert ok, ("modulations", st)
    cos = s.cos.reshape(T, hd // 2)
    sin = s.sin.reshape(T, hd // 2)
    mask = np.concatenate([s.pm.reshape(-1), np.zeros(T, np.float32)])
    worst = {}

    def note(name, L, st):
        if name not in worst or st["cos"] < worst[name][1]["cos"]:
            worst[name] = (L, st)

    for L in range(d.depth):
        a = f"backbone.layers.{L}.self_attn.experts.1."
        x = s.probe("x", L)
        xn, gate = O.ada_rms_norm(x.astype(np.float32), mods[2 * L:2 * L + 1].astype(np.float32), d.eps, F32)
        q_ref = O.apply_rope(O.linear(xn, P, a + "q_proj", F32).reshape(T, n, hd), cos, sin, F32) * np.float32(hd ** -0.5)
        k_ref = O.apply_rope(O.linear(xn, P, a + "k_proj", F32).reshape(T, kv, hd), cos, sin, F32)
        v_ref = O.linear(xn, P, a + "v_proj", F32)
        q, k, v = s.probe("q", L), s.probe("k", L), s.probe("v", L)
        for name, got, ref in (("q", q, q_ref.reshape(T, -1)), ("k", k, k_ref.reshape(T, -1)), ("v", v, v_ref)):
            ok, st = rel_gate(got, ref, rel=1e-2, cos=0.99999)
            note(name, L, st)
            assert ok, (name, L, st)
        # attention on the GPU's own q / k / v, float64
        kf = np.concatenate([s.keys[L, 0].transpose(1, 0, 2), k.reshape(T, kv, hd)], 0).astype(np.float64)
        vf = np.concatenate([s.values[L, 0].transpose(1, 0, 2), v.reshape(T, kv, hd)], 0).astype(np.float64)
        att_ref = O.sdpa(q.reshape(T, n, hd).astype(np.float64), kf, vf, mask.astype(np.float64), F64)
        att = s.probe("attn", L)
        ok, st = kernel_gate(att, att_ref)
        note("attention", L, st)
        assert ok, ("attention", L, st)
        # o_proj + gated residual on the GPU's attention output (fp16 cast points)
        xm_ref = O.gated_residual(x, O.linear(att, P, a + "o_proj", F16), gate.astype(np.float16), F16)
        xm = s.probe("x_mid", L)
        ok, st = rel_gate(xm, xm_ref, rel=2e-3, cos=0.999999)
        note("o_proj", L, st)
        assert ok, ("o_proj", L, st)
        # adaRMS (post) + gate_up + GeGLU on the GPU's residual
        xn2, gate2 = O.ada_rms_norm(xm.astype(np.float32), mods[2 * L + 1:2 * L + 2].astype(np.float32), d.eps, F32)
        gu = O.linear(xn2, P, f"backbone.layers.{L}.mlp.1.gate_up_proj", F32)
        F = gu.shape[-1] // 2
        h_ref = O.gelu_tanh(gu[:, :F]) * gu[:, F:]
        h = s.probe("h", L)
        ok, st = rel_gate(h, h_ref, rel=1e-2, cos=0.99999)
        note("gate_up", L, st)
        assert ok, ("gate_up", L, st)
        # down + gated residual on the GPU's GeGLU output
        xo_ref = O.gated_residual(xm, O.linear(h, P, f"backbone.layers.{L}.mlp.1.down_proj", F16),
                                  gate2.astype(np.float16), F16)
        ok, st = rel_gate(s.probe("x", L + 1), xo_ref, rel=2e-3, cos=0.999999)
        note("down", L, st)
        assert ok, ("down", L, st)
    xf, _ = O.ada_rms_norm(s.probe("x", d.depth).astype(np.float32), mods[2 * d.depth:].astype(np.float32), d.eps, F32)
    v_ref = O.linear(xf, P, "action_out_proj", F32, bias=True).reshape(v_gpu.shape)
    ok, st = rel_gate(v_gpu, v_ref, rel=1e-2, cos=0.99999)
    assert ok, ("head", st)
    print("per-op worst (layer, stats):", {k_: (v_[0], round(v_[1]["cos"], 8), round(v_[1].get("rel", 0), 5))
                                          for k_, v_ in worst.items()}, flush=True)


def _chain_checks(s: Step, v_gpu):
    """The whole step against the float32 oracle: per-layer residual and attention output."""
    d = s.d
    xs, att = [], []
    sdpa = O.sdpa

    def hooked(*a, **kw):
        o = sdpa(*a, **kw)
        att.append(o.copy())
        return o

    O.sdpa = hooked
    try:
        ref = O.denoise_step_kv(s.host, d, s.keys, s.values, s.x_t, s.te, s.cos, s.sin, s.pm, F32,
                                layer_hook=lambda L, x: xs.append(x.copy()))
    finally:
        O.sdpa = sdpa
    for L in range(d.depth):
        ok, st = rel_gate(s.probe("x", L + 1), xs[L])
        assert ok, ("residual after layer", L, st)
        ok, st = rel_gate(s.probe("attn", L), att[L])
        assert ok, ("attention output of layer", L, st)
    ok, st = action_gate(v_gpu, ref)
    print("chain velocity:", st, flush=True)
    assert ok, st
    return ref


@pytest.fixture(scope="module")
def tiny_step():
    print("persistent step: tiny model", flush=True)
    return Step(TINY_KWARGS)


@pytest.fixture(scope="module")
def full_step():
    print("persistent step: full pi0.5 shape", flush=True)
    return Step(dict(dtype="float16", action_horizon=50))


@pytest.mark.parametrize("which", ["tiny", "full"])
def test_persistent_step_per_op_and_chain(which, tiny_step, full_step):
    s = tiny_step if which == "tiny" else full_step
    v = s.run()
    _per_op_checks(s, v)
    _chain_checks(s, v)


@pytest.mark.parametrize("which", ["tiny", "full"])
def test_persistent_step_matches_launch_chain(which, tiny_step, full_step):
    """The persistent kernel and the one-launch-per-op path compute the same step (the
    summation orders of the row statistics differ, so they agree to fp16 rounding)."""
    s = tiny_step if which == "tiny" else full_step
    a = s.run()
    s.runner.vm.set_persist(False)
    try:
        b = s.run()
    finally:
        s.runner.vm.set_persist(True)
    assert np.all(np.isfinite(a)) and np.all(np.isfinite(b))
    assert cosine(a, b) >= 0.99999 and max_abs(a, b) <= 5e-3, (cosine(a, b), max_abs(a, b))


def test_persistent_graph_replays_and_repeats(tiny_step):
    """Replays of the captured step (progress words advance across launches) with eager work
    in between give the same velocity every time, and a loop of steps equals the host loop."""
    s = tiny_step
    v0 = s.run()
    for i in range(4):
        torch.randn(1000, device="cuda").sum().item()  # eager work between the replays
        np.testing.assert_array_equal(s.run(), v0)
    prefix = np.random.default_rng(1).standard_normal((1, s.cfg.prefix_len, s.cfg.vlm.width)).astype(np.float16)
    noise = np.random.default_rng(2).standard_normal((1, s.cfg.action_horizon, s.cfg.action_dim)).astype(np.float32)
    params0 = [s.p[n] if _is_ae(n) else torch.zeros_like(s.p[n]) for n, _ in s.runner.named_params]
    graph = s.runner.sample_graph(params0, prefix, noise=noise)
    host = s.runner.sample(params0, prefix, noise=noise, num_steps=s.cfg.num_denoise_steps)
    np.testing.assert_array_equal(graph, host)


def test_persistent_wait_timeout_is_reported_and_recovered(tiny_step):
    """A wait between phases that gives up (forced from the host with a spin limit of zero
    polls, every kernel still exits) is reported by mlcv_sync / the output's .numpy(), and
    the context computes correctly again after it."""
    s = tiny_step
    good = s.run()
    s.runner.vm.set_persist_spin(0)
    try:
        out = s.runner.vm["denoise_step_kv"](*s.args, s.params)
        with pytest.raises(N.MlcvError, match="gave up"):
            out.numpy()
    finally:
        s.runner.vm.set_persist_spin(1 << 22)
    np.testing.assert_array_equal(s.run(), good)


def test_persistent_loop_and_chunk_vs_oracle():
    """denoise_loop_kv and the chunk (prefill + loop) on the persistent step, tiny model."""
    cfg = Pi0Config(**TINY_KWARGS)
    d = O.dims_from_config(cfg)
    runner = PiZeroRunner(cfg, "rocm", cuda_graph=True)
    runner.vm.set_persist(True)
    p16 = O.make_params(O.param_specs(d), 0, "float16")
    params = runner.to_params([p16[n] for n, _ in runner.named_params])
    rng = np.random.default_rng(9)
    prefix = rng.standard_normal((1, cfg.prefix_len, cfg.vlm.width)).astype(np.float16)
    noise = rng.standard_normal((1, cfg.action_horizon, cfg.action_dim)).astype(np.float32)
    pad = (np.arange(cfg.prefix_len) < cfg.prefix_len - 6).astype(np.float32)
    got = runner.sample_graph(params, prefix, noise=noise, prefix_pad=pad)
    ref = O.sample({k: v.astype(np.float32) for k, v in p16.items()}, d, prefix, noise, F32, prefix_pad=pad, graph=True)
    ok, st = action_gate(got, ref)
    assert ok, st
    pm = make_prefix_mask_np(cfg.prefix_len, pad_mask=pad)
    cos, sin = make_rope_np(cfg.suffix_len, cfg.vlm.head_dim, cfg.rope_theta, offset=int(pad.sum()))
    tes = np.concatenate(make_time_embs(cfg.num_denoise_steps, cfg.action_expert.width), 0).astype(np.float16)
    dv = lambda a: runtime.tensor(a, runner.dev)  # noqa: E731
    chunk = runner.vm["chunk"](dv(prefix), dv(pm), dv(noise), dv(tes), dv(cos), dv(sin), params).numpy()
    np.testing.assert_array_equal(chunk, got)
