"""The HIP path against the committed golden fixtures (tests/golden/): q4f16_1
quantize/dequantize bit-exact, isolated joint attention at the pi0.5 head shape,
and the 2-layer model end to end through PiZeroRunner (prefill K/V, v at t=1,
10-step host and in-graph actions).

The fixtures are float32 / float64; the device path computes with fp16 weights
(the float32 weights rounded once), so model outputs are held to the action
tolerance: max_abs <= 1e-2 and cosine >= 0.999.
"""

from __future__ import annotations

import ctypes
import os
import sys

import numpy as np
import pytest
import torch

from conftest import ROOT, TINY_KWARGS, cosine, max_abs
from mlc_vla import _native as N
from mlc_vla import runtime
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.sample import PiZeroRunner, make_prefix_mask_np

GOLDEN = os.path.join(ROOT, "tests", "golden")
if GOLDEN not in sys.path:
    sys.path.insert(0, GOLDEN)
import make_golden as G  # noqa: E402

pytestmark = pytest.mark.gpu


def _load(name):
    return np.load(os.path.join(GOLDEN, name))


def _st():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _tol(got, ref, atol=1e-2, cos=0.999):
    assert np.all(np.isfinite(got))
    assert max_abs(got, ref) <= atol, max_abs(got, ref)
    assert cosine(got, ref) >= cos, cosine(got, ref)


def test_q4_fixture_bitexact():
    print("golden q4 16x128", flush=True)
    fx = _load("q4_kat.npz")
    w = fx["w"]
    n, k = w.shape
    wd = _dev(w)
    qw = torch.zeros((n, k // 8), dtype=torch.int32, device="cuda")
    qs = torch.zeros((n, k // 32), dtype=torch.float16, device="cuda")
    N.call("mlcv_q4_quantize", _p(wd), _p(qw), _p(qs), n, k, _st())
    out = torch.empty((n, k), dtype=torch.float16, device="cuda")
    N.call("mlcv_q4_dequantize", _p(qw), _p(qs), _p(out), n, k, _st())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(qw.cpu().numpy().view(np.uint32), fx["q_weight"])
    np.testing.assert_array_equal(qs.cpu().numpy().view(np.uint16), fx["q_scale"].view(np.uint16))
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16), fx["deq_bits"])


def test_attention_fixture():
    print("golden attention Tq=50 H=8 hd=256 Sp=96 valid=72 Ts=50", flush=True)
    fx = _load("attn_isolated.npz")
    q, kp, vp, ks, vs, mask = G.attn_inputs(**G.ATTN)
    tq, h, hd = q.shape[0], G.ATTN["h"], G.ATTN["hd"]
    out = torch.empty((tq, h * hd), dtype=torch.float16, device="cuda")
    qd, kpd, vpd, ksd, vsd, md = _dev(q), _dev(kp.astype(np.float32)), _dev(vp), _dev(ks), _dev(vs), _dev(mask)
    N.call("mlcv_joint_attention", _p(qd), tq, h, 1, hd, _p(kpd), 1, _p(vpd), kp.shape[1], _p(md), _p(ksd),
           _p(vsd), ks.shape[0], _p(out), _st())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = fx["out_f64"]
    scale = float(np.abs(ref).max())
    assert max_abs(got, ref) <= 2e-3 * scale + 2e-4, (max_abs(got, ref), scale)
    assert cosine(got, ref) > 0.99999


@pytest.fixture(scope="module")
def tiny_model():
    cfg = Pi0Config(**TINY_KWARGS)
    runner = PiZeroRunner(cfg, "rocm")
    specs, params, prefix, noise = G.tiny_inputs()
    assert [n for n, _ in specs] == [n for n, _ in runner.named_params]
    dev_params = runner.to_params([params[n].astype(np.float16) for n, _ in runner.named_params])
    return cfg, runner, dev_params, prefix, noise, _load("tiny_e2e.npz")


def test_tiny_prefill_fixture(tiny_model):
    print("golden tiny prefill", flush=True)
    cfg, runner, params, prefix, _, fx = tiny_model
    pm = make_prefix_mask_np(cfg.prefix_len)
    k, v = runner.vm["prefill"](runtime.tensor(prefix.astype(np.float16), runner.dev),
                                runtime.tensor(pm, runner.dev), params)
    for L in range(2):
        _tol(k.numpy()[L], fx["keys"][L], atol=2e-2 * np.abs(fx["keys"][L]).max(), cos=0.9999)
        _tol(v.numpy()[L], fx["values"][L], atol=2e-2 * np.abs(fx["values"][L]).max(), cos=0.9999)


def test_tiny_step_fixture(tiny_model):
    print("golden tiny denoise_step_kv t=1", flush=True)
    cfg, runner, params, prefix, noise, fx = tiny_model
    d = G.TINY_DIMS
    pm = make_prefix_mask_np(cfg.prefix_len)
    dev = lambda a: runtime.tensor(np.ascontiguousarray(a), runner.dev)  # noqa: E731
    k, v = runner.vm["prefill"](dev(prefix.astype(np.float16)), dev(pm), params)
    cos, sin = G.O.make_rope_np(d.suffix_len, d.head_dim, d.theta, offset=d.prefix_len)
    te = G.O.sinusoidal_time_emb(1.0, d.ae_width).astype(np.float16)
    v1 = runner.vm["denoise_step_kv"](k, v, dev(noise.astype(np.float16)), dev(te), dev(cos), dev(sin), dev(pm),
                                      params)
    _tol(v1.numpy(), fx["v1"])
    _tol(v1.numpy(), fx["v1_f64"])


def test_tiny_actions_fixture(tiny_model):
    print("golden tiny sample / sample_graph", flush=True)
    _, runner, params, prefix, noise, fx = tiny_model
    host = runner.sample(params, prefix, noise=noise, num_steps=10)
    _tol(host, fx["actions"])
    _tol(host, fx["actions_f64"])
    graph = runner.sample_graph(params, prefix, noise=noise)
    _tol(graph, fx["actions_graph"])
    _tol(graph, fx["actions_graph_f64"])


# ---- the float32 model (Pi0Config(dtype="float32"), the reference's default dtype) ----------
# The fixtures are the float32 oracle (and its float64 twin) on float32 weights; the float32
# model computes with those weights unrounded, so it is held to float32 accuracy: the tolerance
# the CPU fixture test gives two float32 BLAS builds (tests/test_golden.py: rtol 2e-4, atol
# 2e-5 of the largest value), which fp16 weights miss by two orders of magnitude.
def _f32_tol(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.all(np.isfinite(got)), what
    np.testing.assert_allclose(got, ref, rtol=2e-4, atol=2e-5 * float(np.abs(ref).max()), err_msg=what)
    assert cosine(got, ref) >= 0.9999999, (what, cosine(got, ref))


@pytest.fixture(scope="module")
def tiny_f32():
    cfg = Pi0Config(**{**TINY_KWARGS, "dtype": "float32"})
    runner = PiZeroRunner(cfg, "rocm")
    specs, params, prefix, noise = G.tiny_inputs()
    assert [n for n, _ in specs] == [n for n, _ in runner.named_params]
    dev_params = runner.to_params([params[n].astype(np.float32) for n, _ in runner.named_params])
    return cfg, runner, dev_params, prefix, noise, _load("tiny_e2e.npz")


def test_tiny_f32_prefill_and_step_fixture(tiny_f32):
    print("golden tiny float32 model: prefill, denoise_step_kv t=1", flush=True)
    cfg, runner, params, prefix, noise, fx = tiny_f32
    d = G.TINY_DIMS
    dev = lambda a: runtime.tensor(np.ascontiguousarray(a), runner.dev)  # noqa: E731
    pm = make_prefix_mask_np(cfg.prefix_len)
    k, v = runner.vm["prefill"](dev(prefix.astype(np.float32)), dev(pm), params)
    assert k.dtype == "float32" and v.dtype == "float32"
    for L in range(2):
        _f32_tol(k.numpy()[L], fx["keys"][L], f"keys[{L}]")
        _f32_tol(v.numpy()[L], fx["values"][L], f"values[{L}]")
    cos, sin = G.O.make_rope_np(d.suffix_len, d.head_dim, d.theta, offset=d.prefix_len)
    te = G.O.sinusoidal_time_emb(1.0, d.ae_width).astype(np.float32)
    v1 = runner.vm["denoise_step_kv"](k, v, dev(noise.astype(np.float32)), dev(te), dev(cos), dev(sin), dev(pm), params)
    _f32_tol(v1.numpy(), fx["v1"], "v1")
    _f32_tol(v1.numpy(), fx["v1_f64"], "v1 (float64 truth)")


def test_tiny_f32_actions_fixture(tiny_f32):
    print("golden tiny float32 model: sample / sample_graph", flush=True)
    _, runner, params, prefix, noise, fx = tiny_f32
    host = runner.sample(params, prefix, noise=noise, num_steps=10)
    _f32_tol(host, fx["actions"], "actions")
    _f32_tol(host, fx["actions_f64"], "actions (float64 truth)")
    graph = runner.sample_graph(params, prefix, noise=noise)
    _f32_tol(graph, fx["actions_graph"], "actions_graph")
    _f32_tol(graph, fx["actions_graph_f64"], "actions_graph (float64 truth)")


def test_dummy_f32_model_vs_oracle():
    """The reference's dummy configuration (pi0_config.py: paligemma and action expert
    "dummy") in float32 against the float32 oracle on the same weights: sample and sample_graph."""
    from conftest import DUMMY_KWARGS
    from oracle import pi0_oracle as O

    cfg = Pi0Config(**{**DUMMY_KWARGS, "dtype": "float32"})
    d = O.dims_from_config(cfg)
    print(f"dummy float32 model: {d}", flush=True)
    runner = PiZeroRunner(cfg, "rocm")
    p = O.make_params(O.param_specs(d), 3, "float32")
    params = runner.to_params([p[n] for n, _ in runner.named_params])
    rng = np.random.default_rng(4)
    prefix = rng.standard_normal((1, cfg.prefix_len, cfg.vlm.width)).astype(np.float32)
    noise = rng.standard_normal((1, cfg.action_horizon, cfg.action_dim)).astype(np.float32)
    got = runner.sample(params, prefix, noise=noise, num_steps=cfg.num_denoise_steps)
    ref = O.sample(p, d, prefix, noise, O.Prec("f32"))
    _f32_tol(got, ref, "dummy sample")
    graph = runner.sample_graph(params, prefix, noise=noise)
    refg = O.sample(p, d, prefix, noise, O.Prec("f32"), graph=True)
    _f32_tol(graph, refg, "dummy sample_graph")


def test_f32_tolerance_rejects_the_fp16_model(tiny_model):
    """The float32 tolerance above discriminates: the float16 model (the same weights rounded
    to fp16) passes the action tolerance on this fixture but not the float32 one."""
    cfg, runner, params, prefix, noise, fx = tiny_model
    d = G.TINY_DIMS
    dev = lambda a: runtime.tensor(np.ascontiguousarray(a), runner.dev)  # noqa: E731
    pm = make_prefix_mask_np(cfg.prefix_len)
    k, v = runner.vm["prefill"](dev(prefix.astype(np.float16)), dev(pm), params)
    cos, sin = G.O.make_rope_np(d.suffix_len, d.head_dim, d.theta, offset=d.prefix_len)
    te = G.O.sinusoidal_time_emb(1.0, d.ae_width).astype(np.float16)
    v1 = runner.vm["denoise_step_kv"](k, v, dev(noise.astype(np.float16)), dev(te), dev(cos), dev(sin), dev(pm),
                                      params).numpy()
    _tol(v1, fx["v1"])
    with pytest.raises(AssertionError):
        _f32_tol(v1, fx["v1"], "fp16 model v1")
