"""The XCD tensor-parallel step (csrc/step_xtp.hip: each decoder layer as two launches of one
workgroup per CU, tensor-parallel over the 8 XCDs, pi0_model.py:142-163 / gemma_dual.py:343-351)
at the full pi0.5 shape: against the oracle op by op and layer by layer (every layer's
intermediates kept, MLCV_OPT_XTP_KEEP), the 8 XCDs' copies of the residual stream, against the
launch chain, with the default reused buffers, across graph replays and the device loop, with
the masked-chunk skip against the same step without it, with barrier words that wrap, and with
a barrier wait that gives up."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import cosine, max_abs
from mlc_vla import _native as N
from mlc_vla import runtime
from mlc_vla.sample import make_prefix_mask_np, make_rope_np
from stepcheck import Step, chain_checks, is_ae, per_op_checks

pytestmark = pytest.mark.gpu

FULL = dict(dtype="float16", action_horizon=50)


@pytest.fixture(scope="module")
def xstep():
    print("XCD step: full pi0.5 shape", flush=True)
    return Step(FULL, form="xtp")


def test_xtp_step_per_op_and_chain(xstep):
    v = xstep.run()
    per_op_checks(xstep, v)
    chain_checks(xstep, v)


def test_xtp_xcd_copies_of_the_residual_stream_are_identical(xstep):
    """Every XCD adds the 8 partials of its own copy in the same order: the copies agree bit for bit."""
    xstep.run()
    T, W = xstep.d.suffix_len, xstep.d.ae_width
    for L in (0, 1, 9, xstep.d.depth - 1):
        xs = [xstep.runner.vm.probe("xcd_x", 8 * L + x, (T, W), np.float16) for x in range(8)]
        for x in range(1, 8):
            np.testing.assert_array_equal(xs[0], xs[x], err_msg=f"layer {L} XCD {x}")


def test_xtp_matches_reused_buffers_and_launch_chain(xstep):
    vm = xstep.runner.vm
    a = xstep.run()
    vm.set_xtp_keep(False)  # the default: one set of buffers for every layer
    try:
        b = xstep.run()
    finally:
        vm.set_xtp_keep(True)
    np.testing.assert_array_equal(a, b)
    vm.set_step_form("chain")
    try:
        c = xstep.run()
    finally:
        vm.set_step_form("xtp")
        vm.set_xtp_keep(True)
    assert np.all(np.isfinite(c))
    assert cosine(a, c) >= 0.99999 and max_abs(a, c) <= 5e-3, (cosine(a, c), max_abs(a, c))


def test_xtp_graph_replays_and_device_loop(xstep):
    """Replays of the captured step (barrier words advance across launches) with eager work in
    between give the same velocity as the direct launches, and the in-graph 10-step loop equals
    the host loop."""
    s = xstep
    s.runner.vm.set_xtp_keep(False)
    try:
        v0 = s.run()
        s.runner.vm.set_step_graph(True)
        try:
            for _ in range(4):
                torch.randn(1000, device="cuda").sum().item()
                np.testing.assert_array_equal(s.run(), v0)
        finally:
            s.runner.vm.set_step_graph(False)
        prefix = np.random.default_rng(1).standard_normal((1, s.cfg.prefix_len, s.cfg.vlm.width)).astype(np.float16)
        noise = np.random.default_rng(2).standard_normal((1, s.cfg.action_horizon, s.cfg.action_dim)).astype(np.float32)
        params0 = [s.p[n] if is_ae(n) else torch.zeros_like(s.p[n]) for n, _ in s.runner.named_params]
        graph = s.runner.sample_graph(params0, prefix, noise=noise)
        host = s.runner.sample(params0, prefix, noise=noise, num_steps=s.cfg.num_denoise_steps)
        assert np.all(np.isfinite(graph))
        np.testing.assert_array_equal(graph, host)
    finally:
        s.runner.vm.set_xtp_keep(True)


def test_xtp_masked_chunk_skip_is_exact(xstep):
    """With 800 of 968 prefix keys valid, 5 of the 32 key chunks are all padding (mask -1e9):
    skipping them gives bit-identical velocities (their softmax weights are exactly 0 in fp32,
    gemma_dual.py:97-122; the pad invariance of compare_pad.py:62-91)."""
    s = xstep
    P, T, hd = s.d.prefix_len, s.d.suffix_len, s.d.head_dim
    pm = make_prefix_mask_np(P, num_valid=800)
    cos, sin = make_rope_np(T, hd, s.cfg.rope_theta, offset=800)
    dv = lambda a: runtime.tensor(a, s.runner.dev)  # noqa: E731
    args = [dv(a) for a in (s.keys, s.values, s.x_t, s.te, cos, sin, pm)]
    vm = s.runner.vm
    skipped = vm["denoise_step_kv"](*args, s.params).numpy()
    N.call("mlcv_set_option", vm._ctx, N.MLCV_OPT_XTP, 2)
    try:
        full = vm["denoise_step_kv"](*args, s.params).numpy()
    finally:
        vm.set_xtp(True)
        vm.set_xtp_keep(True)
    assert np.all(np.isfinite(skipped))
    np.testing.assert_array_equal(skipped, full)


def test_xtp_barrier_words_wrap(xstep):
    """Barrier words started just below 2**32 wrap in the first layers' launches (4 barriers
    per attention launch, 2 per MLP launch): the waits compare against each launch's start value
    with wrapping arithmetic, so the steps equal those from words at 0 bit for bit."""
    s = xstep
    s.runner.vm.set_sync_words(0)
    good = s.run()
    s.runner.vm.set_sync_words(2**32 - 3)
    for _ in range(3):
        np.testing.assert_array_equal(s.run(), good)


def test_xtp_wait_timeout_is_reported_and_recovered(xstep):
    """A barrier wait that gives up (forced from the host with a spin limit of zero polls; every
    kernel still exits) is reported by mlcv_sync / the output's .numpy(), and the context
    computes correctly again after it."""
    s = xstep
    good = s.run()
    s.runner.vm.set_persist_spin(0)
    try:
        out = s.runner.vm["denoise_step_kv"](*s.args, s.params)
        with pytest.raises(N.MlcvError, match="gave up"):
            out.numpy()
    finally:
        s.runner.vm.set_persist_spin(1 << 22)
    np.testing.assert_array_equal(s.run(), good)
