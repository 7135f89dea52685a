"""The persistent step (one launch per denoise_step_kv, csrc/step_persistent.hip) against the
oracle, op by op and layer by layer (stepcheck.per_op_checks / chain_checks, through the probes
of every layer's intermediates), against the launch chain, across graph replays, and with a
wait that gives up."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import TINY_KWARGS, cosine, max_abs
from gates import action_gate
from mlc_vla import _native as N
from mlc_vla import runtime
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.sample import PiZeroRunner, make_prefix_mask_np, make_rope_np, make_time_embs
from oracle import pi0_oracle as O
from stepcheck import Step, chain_checks, is_ae, per_op_checks

pytestmark = pytest.mark.gpu

F32 = O.Prec("f32")


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
    per_op_checks(s, v)
    chain_checks(s, v)


@pytest.mark.parametrize("which", ["tiny", "full"])
def test_persistent_step_matches_launch_chain(which, tiny_step, full_step):
    """The persistent kernel and the one-launch-per-op path compute the same step (the
    summation orders of the row statistics differ, so they agree to fp16 rounding)."""
    s = tiny_step if which == "tiny" else full_step
    a = s.run()
    s.runner.vm.set_step_form("chain")
    try:
        b = s.run()
    finally:
        s.runner.vm.set_step_form("persistent")
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
    params0 = [s.p[n] if is_ae(n) else torch.zeros_like(s.p[n]) for n, _ in s.runner.named_params]
    graph = s.runner.sample_graph(params0, prefix, noise=noise)
    host = s.runner.sample(params0, prefix, noise=noise, num_steps=s.cfg.num_denoise_steps)
    np.testing.assert_array_equal(graph, host)


def test_persistent_progress_words_wrap(full_step):
    """Progress words started just below 2**32 wrap inside the next launches (92 phases each at
    this shape): every launch compares them against its own start value, and the attention's
    row-block counters start each launch at 0, so the steps equal those from words at 0 bit for
    bit (a launch index derived from the words would jump at the wrap)."""
    s = full_step
    s.runner.vm.set_sync_words(0)
    good = s.run()
    s.runner.vm.set_sync_words(2**32 - 40)
    for _ in range(4):
        np.testing.assert_array_equal(s.run(), good)


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
