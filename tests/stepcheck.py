"""Shared checks of one denoise_step_kv against the oracle, op by op and along the whole
chain, on the intermediates a step exposes through probes (mlcv_step_probe): the persistent
step keeps every layer's; the launch chain's are recorded by replaying its operations one at a
time (ChainReplay).

Per op, the oracle is fed the GPU's own inputs of that op, so each check isolates the kernel
code of one operation (pi0_model.py:142-163; gemma_dual.py:60-94 adaRMS / gated residual,
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
import torch

from gates import action_gate, kernel_gate, rel_gate
from mlc_vla import runtime
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.sample import PiZeroRunner, make_prefix_mask_np, make_rope_np
from oracle import pi0_oracle as O

F32, F16, F64 = O.Prec("f32"), O.Prec("f16"), O.Prec("f64")


def is_ae(name: str) -> bool:
    return not (".experts.0." in name or ".mlp.0." in name or name.endswith("layernorm.0.weight")
                or name == "backbone.final_norm.0.weight")


class Step:
    """One denoise_step_kv on the GPU with random-init weights and N(0,1) stand-in K/V, run in
    the given form: "persistent" (one launch per step), "xtp" (two launches per layer over the
    XCDs) or "chain" (one launch per operation)."""

    def __init__(self, kw, seed=3, kv_seed=5, form="persistent"):
        self.cfg = Pi0Config(**kw)
        self.d = O.dims_from_config(self.cfg)
        self.runner = PiZeroRunner(self.cfg, "rocm")
        self.form = form
        self.runner.vm.set_step_form(form)
        if form == "xtp":
            self.runner.vm.set_xtp_keep(True)  # every layer's intermediates for the probes
        d = self.d
        g = torch.Generator(device="cuda").manual_seed(seed)
        specs = O.param_specs(d)
        self.p = {n: ((0.02 * torch.randn(s, generator=g, device="cuda")).half() if is_ae(n)
                      else torch.empty(s, dtype=torch.float16, device="cuda")) for n, s in specs}
        self.params = [self.p[n] for n, _ in self.runner.named_params]
        torch.cuda.synchronize()
        self.host = {n: t.cpu().numpy() for n, t in self.p.items() if is_ae(n)}
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


def per_op_checks(s: Step, v_gpu):
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


def chain_checks(s: Step, v_gpu):
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


class ChainReplay:
    """The launch chain's intermediates of one step: after a denoise_step_kv on the chain, its
    operations run again one at a time (mlcv_bench_op: the same kernels with the same
    arguments) and each output is read between them.  Exposes the Step interface."""

    def __init__(self, s: Step):
        self.s = s
        vm = s.runner.vm
        d, T = s.d, s.d.suffix_len
        nq, nkv = d.num_heads * d.head_dim, d.num_kv_heads * d.head_dim
        shapes = {"x": ((T, d.ae_width), np.float16), "x_mid": ((T, d.ae_width), np.float16),
                  "q": ((T, nq), np.float32), "k": ((T, nkv), np.float32), "v": ((T, nkv), np.float16),
                  "attn": ((T, nq), np.float16), "h": ((T, d.ae_mlp), np.float16),
                  "mod": ((2 * d.depth + 1, 3 * d.ae_width), np.float16), "vout": ((T, d.action_dim), np.float32)}
        rec = {}

        def grab(what, L):
            rec[(what, L)] = vm.probe(what, 0, *shapes[what])

        keys, values = s.args[0], s.args[1]
        vm.run_op("time_mod")
        grab("mod", 0)
        vm.run_op("action_in")
        grab("x", 0)
        for L in range(d.depth):
            vm.run_op("qkv", L)
            for w in ("q", "k", "v"):
                grab(w, L)
            vm.run_op("attention", L, keys, values)
            grab("attn", L)
            vm.run_op("o_proj", L)
            grab("x_mid", L)
            vm.run_op("gate_up", L)
            grab("h", L)
            vm.run_op("down", L)
            grab("x", L + 1)
        vm.run_op("head")
        grab("vout", 0)
        self.rec = rec

    def probe(self, what, layer):
        return self.rec[(what, layer)]

    def __getattr__(self, name):
        return getattr(self.s, name)
