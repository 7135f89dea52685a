"""Sampling through the worker process (mlc_vla/worker.py, the evaluation worker of
M1.md:55-72) against the in-process runner on the same synthetic weights: the device loop
and the host loop, with and without a prefix pad mask, bit for bit."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import TINY_KWARGS
from mlc_vla import worker as W
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.sample import PiZeroRunner

pytestmark = pytest.mark.gpu


def test_worker_sample_matches_in_process_runner(tmp_path):
    cfg = Pi0Config(**TINY_KWARGS)
    print("worker: tiny model, seed 11", flush=True)
    runner = PiZeroRunner(cfg, "rocm")
    params = runner.to_params(W.random_params(runner.named_params, 11))
    rng = np.random.default_rng(5)
    prefix = rng.standard_normal((1, cfg.prefix_len, cfg.vlm.width)).astype(np.float16)
    noise = rng.standard_normal((1, cfg.action_horizon, cfg.action_dim)).astype(np.float32)
    pad = np.ones(cfg.prefix_len, bool)
    pad[-5:] = False
    want_graph = runner.sample_graph(params, prefix, noise=noise)
    want_pad = runner.sample_graph(params, prefix, noise=noise, prefix_pad=pad)
    want_host = runner.sample(params, prefix, noise=noise, num_steps=3)
    with W.WorkerClient(TINY_KWARGS, str(tmp_path / "cfg.json"), random_weights=11) as c:
        p = c.ping()
        assert p["ready"], p.get("error")
        got = c.sample(prefix, noise=noise)
        assert got.shape == (1, cfg.action_horizon, cfg.action_dim) and np.all(np.isfinite(got))
        np.testing.assert_array_equal(got, want_graph)
        np.testing.assert_array_equal(c.sample(prefix, noise=noise, prefix_pad=pad), want_pad)
        np.testing.assert_array_equal(c.sample(prefix, noise=noise, graph=False, num_steps=3), want_host)
        with pytest.raises(W.WorkerError):
            c.sample(prefix[:, :3], noise=noise)  # a wrong prefix length is an error reply
        np.testing.assert_array_equal(c.sample(prefix, noise=noise), want_graph)  # and the worker goes on
    assert c.proc.returncode == 0
