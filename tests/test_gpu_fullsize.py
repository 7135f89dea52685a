"""Full-size parity of the two configurations the step benchmark does not cover by itself:

- the action chunk (prefill of the Gemma-2B-shaped prefix expert at P = 968 with 800 valid
  tokens, then the 10-step in-graph Euler loop of the pi0.5 action expert), against the
  float32 oracle: every layer's prefix K / V, then the actions (pi0_model.py:128-194,
  gemma_dual.py:398-415; the pad recipe of compare_pad.py:62-91);
- the q4f16_1 ``denoise_step_kv`` at the full shape (the XCD step, and the launch chain it is
  checked against), against the oracle on the same dequantized weights and against the fp16
  step (compare_quant.py:76-117, cos >= 0.97 at :115).

Weights are 0.02 N(0, 1) drawn on the GPU with a seeded torch generator (drawing the 2.4 G
parameters with numpy on the host would take minutes); the oracle reads the same fp16 values.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gates import action_gate, kv_gate
from mlc_vla import _native as N
from mlc_vla import runtime
from mlc_vla.compile_quant import compile_model_quant
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.sample import PiZeroRunner, make_prefix_mask_np, make_rope_np, make_time_embs
from oracle import pi0_oracle as O

pytestmark = pytest.mark.gpu

F32 = O.Prec("f32")


def _gpu_params(specs, seed, keep=lambda n: True):
    """0.02 N(0,1) fp16 device tensors for the kept names (empty tensors for the others)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    out = {}
    for name, shape in specs:
        if keep(name):
            out[name] = (0.02 * torch.randn(shape, generator=g, device="cuda")).half()
        else:
            out[name] = torch.empty(shape, dtype=torch.float16, device="cuda")
    return out


def _host(params, names):
    torch.cuda.synchronize()
    return {n: params[n].cpu().numpy() for n in names}


def _is_ae(name: str) -> bool:
    return not (".experts.0." in name or ".mlp.0." in name or name.endswith("layernorm.0.weight")
                or name == "backbone.final_norm.0.weight")


def test_fullsize_chunk_800_valid_vs_oracle():
    cfg = Pi0Config(dtype="float16", action_horizon=50)
    assert (cfg.prefix_len, cfg.vlm.width, cfg.vlm.mlp_dim, cfg.vlm.depth) == (968, 2048, 16384, 18)
    d = O.dims_from_config(cfg)
    print("full-size chunk: drawing 2.4 G parameters on the GPU", flush=True)
    runner = PiZeroRunner(cfg, "rocm", cuda_graph=True)
    p = _gpu_params(O.param_specs(d), seed=11)
    params = [p[n] for n, _ in runner.named_params]
    host = _host(p, [n for n, _ in O.param_specs(d)])
    rng = np.random.default_rng(3)
    prefix = rng.standard_normal((1, 968, 2048)).astype(np.float16)
    pad = (np.arange(968) < 800).astype(np.float32)
    noise = np.random.default_rng(0).standard_normal((1, 50, 32)).astype(np.float32)
    pm = make_prefix_mask_np(968, pad_mask=pad)
    dv = lambda a: runtime.tensor(a, runner.dev)  # noqa: E731

    print("full-size chunk: GPU prefill", flush=True)
    k, v = runner.vm["prefill"](dv(prefix), dv(pm), params)
    kg, vg = k.numpy(), v.numpy()
    print("full-size chunk: oracle prefill (float32)", flush=True)
    kr, vr = O.prefill(host, d, prefix, pm, F32)
    worst = []
    for L in range(d.depth):
        okk, sk = kv_gate(kg[L], kr[L])
        okv, sv = kv_gate(vg[L], vr[L])
        worst.append((L, sk["rel"], sk["cos"], sv["rel"], sv["cos"]))
        assert okk and okv, (L, sk, sv)
    print("per-layer K/V (layer, K rel, K cos, V rel, V cos), worst three by K cos:",
          sorted(worst, key=lambda w: w[2])[:3], flush=True)

    print("full-size chunk: GPU loop + chunk graph", flush=True)
    x = runner.sample_graph(params, prefix, noise=noise, prefix_pad=pad)
    cos, sin = make_rope_np(50, 256, cfg.rope_theta, offset=800)
    tes = np.concatenate(make_time_embs(10, 1024), 0).astype(np.float16)
    chunk = runner.vm["chunk"](dv(prefix), dv(pm), dv(noise), dv(tes), dv(cos), dv(sin), params).numpy()
    np.testing.assert_array_equal(chunk, x)  # one graph == prefill graph + loop graph
    print("full-size chunk: oracle loop (float32)", flush=True)
    ref = O.denoise_loop_kv(host, d, kr, vr, noise, tes, cos, sin, pm, F32)
    ok, st = action_gate(x, ref)
    print(f"full-size chunk actions: {st}", flush=True)
    assert ok, st


def _q4_quantize_gpu(w: torch.Tensor):
    n, k = w.shape
    qw = torch.empty((n, k // 8), dtype=torch.int32, device="cuda")
    qs = torch.empty((n, k // 32), dtype=torch.float16, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    N.call("mlcv_q4_quantize", ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(qw.data_ptr()),
           ctypes.c_void_p(qs.data_ptr()), n, k, st)
    deq = torch.empty_like(w)
    N.call("mlcv_q4_dequantize", ctypes.c_void_p(qw.data_ptr()), ctypes.c_void_p(qs.data_ptr()),
           ctypes.c_void_p(deq.data_ptr()), n, k, st)
    return qw, qs, deq


def test_fullsize_q4_step_vs_oracle_and_fp16():
    cfg = Pi0Config(dtype="float16", action_horizon=50)
    d = O.dims_from_config(cfg)
    specs = O.param_specs(d)
    print("full-size q4 step: drawing the action-expert weights", flush=True)
    p = _gpu_params(specs, seed=21, keep=_is_ae)
    ex, qnp, qmap, _quant = compile_model_quant(cfg, "rocm", None, "q4f16_1")
    vm = runtime.VirtualMachine(ex, runtime.device())
    qt, deq = {}, {}
    for base, (qwn, qsn) in ((b[: -len(".weight")], qn) for b, qn in qmap.param_map.items()):
        w = p[base + ".weight"]
        if _is_ae(base + ".weight"):
            qt[qwn], qt[qsn], deq[base + ".weight"] = _q4_quantize_gpu(w)
        else:  # the prefix expert: not read by denoise_step_kv
            qt[qwn] = torch.empty((w.shape[0], w.shape[1] // 8), dtype=torch.int32, device="cuda")
            qt[qsn] = torch.zeros((w.shape[0], w.shape[1] // 32), dtype=torch.float16, device="cuda")
    qparams = [qt[n] if n in qt else p[n] for n, _ in qnp]
    runner = PiZeroRunner(cfg, "rocm")
    fparams = [p[n] for n, _ in runner.named_params]
    rng = np.random.default_rng(5)
    keys = rng.standard_normal((18, 1, 1, 968, 256)).astype(np.float32)
    values = rng.standard_normal((18, 1, 1, 968, 256)).astype(np.float16)
    x_t = rng.standard_normal((1, 50, 32)).astype(np.float16)
    te = O.sinusoidal_time_emb(1.0, 1024).astype(np.float16)
    pm = make_prefix_mask_np(968)
    cos, sin = make_rope_np(50, 256, 10_000.0, offset=968)
    dv = lambda a: runtime.tensor(a, runner.dev)  # noqa: E731
    args = [dv(a) for a in (keys, values, x_t, te, cos, sin, pm)]
    print("full-size q4 step: GPU q4 (XCD step and launch chain) and fp16 steps", flush=True)
    vq = vm["denoise_step_kv"](*args, qparams).numpy()  # the default form: the XCD step
    vm.set_step_form("chain")
    vqc = vm["denoise_step_kv"](*args, qparams).numpy()
    vm.set_step_form("xtp")
    cq = float(np.dot(vq.ravel().astype(np.float64), vqc.ravel()) /
               (np.linalg.norm(vq.astype(np.float64)) * np.linalg.norm(vqc.astype(np.float64))))
    mq = float(np.max(np.abs(vq.astype(np.float64) - vqc)))
    print(f"q4 XCD step vs q4 launch chain: cos {cq:.8f} max_abs {mq:.3e}", flush=True)
    assert np.all(np.isfinite(vq)) and cq >= 0.99999 and mq <= 5e-3, (cq, mq)
    vf = runner.vm["denoise_step_kv"](*args, fparams).numpy()
    ae_names = [n for n, _ in specs if _is_ae(n)]
    host = _host(p, ae_names)
    hostq = dict(host)
    hostq.update(_host(deq, list(deq)))
    print("full-size q4 step: oracle on the dequantized weights", flush=True)
    ref = O.denoise_step_kv(hostq, d, keys, values, x_t, te, cos, sin, pm, F32)
    ok, st = action_gate(vq, ref)
    print(f"q4 step vs oracle on the dequantized weights: {st}", flush=True)
    assert ok, st
    c = float(np.dot(vq.ravel().astype(np.float64), vf.ravel()) /
              (np.linalg.norm(vq.astype(np.float64)) * np.linalg.norm(vf.astype(np.float64))))
    print(f"q4 step vs fp16 step: cos {c:.5f}", flush=True)
    assert c >= 0.97


def test_masked_chunk_skip_is_bit_exact_at_800_valid():
    """Prefill and the step attentions skip the 32-key chunks whose keys are all masked
    (MLCV_OPT_MASK_SKIP, default on): at 800 valid of 968 prefix keys (6 of the prefill's 31 key
    chunks), every layer's K / V and the velocity of each step form are bit-identical to the same
    calls computing those chunks (gemma_dual.py:97-122: exp of a -1e9 logit is 0 in fp32)."""
    cfg = Pi0Config(dtype="float16", action_horizon=50)
    d = O.dims_from_config(cfg)
    print("mask skip: drawing the full-size parameters on the GPU", flush=True)
    runner = PiZeroRunner(cfg, "rocm", cuda_graph=True)
    p = _gpu_params(O.param_specs(d), seed=7)
    params = [p[n] for n, _ in runner.named_params]
    rng = np.random.default_rng(4)
    prefix = rng.standard_normal((1, 968, 2048)).astype(np.float16)
    pm = make_prefix_mask_np(968, num_valid=800)
    cos, sin = make_rope_np(50, 256, cfg.rope_theta, offset=800)
    x_t = rng.standard_normal((1, 50, 32)).astype(np.float16)
    te = O.sinusoidal_time_emb(0.7, d.ae_width).astype(np.float16)
    dv = lambda a: runtime.tensor(a, runner.dev)  # noqa: E731
    args = [dv(a) for a in (x_t, te, cos, sin, pm)]
    forms = ["chain", "persistent", "xtp"]

    def run(skip):
        runner.vm.set_mask_skip(skip)
        k, v = runner.vm["prefill"](dv(prefix), args[4], params)
        out = {"keys": k.numpy(), "values": v.numpy()}
        for form in forms:
            runner.vm.set_step_form(form)
            out[form] = runner.vm["denoise_step_kv"](k, v, *args, params).numpy()
        runner.vm.set_step_form("xtp")
        return out

    print("mask skip: with the skip", flush=True)
    a = run(True)
    print("mask skip: without the skip", flush=True)
    b = run(False)
    runner.vm.set_mask_skip(True)
    for name in ["keys", "values"] + forms:
        assert np.all(np.isfinite(a[name])), name
        np.testing.assert_array_equal(a[name], b[name], err_msg=name)


def test_prefill_tile_major_weights_bit_exact(monkeypatch):
    """The prefill's gate_up and down read tile-major copies of their weights (made at bind) and
    tile-major activations (the post-attention norm's output, gate_up's GeGLU output): one
    contiguous 1 KB per DMA instruction of 16 rows x 32 k.  The same fp16 values land in the same
    LDS slots as with the row-major operands, so every layer's K / V is bit-identical
    (gemma_dual.py:125-135, the prefix expert's GeGLU MLP at P = 968 with its 8 pad rows)."""
    cfg = Pi0Config(dtype="float16", action_horizon=50)
    d = O.dims_from_config(cfg)
    runner = PiZeroRunner(cfg, "rocm", cuda_graph=True)
    p = _gpu_params(O.param_specs(d), seed=9)
    params = [p[n] for n, _ in runner.named_params]
    rng = np.random.default_rng(6)
    prefix = runtime.tensor(rng.standard_normal((1, 968, 2048)).astype(np.float16), runner.dev)
    pm = runtime.tensor(make_prefix_mask_np(968, num_valid=800), runner.dev)
    out = {}
    for wt in ("1", "0"):  # read at bind: each pass binds the parameters again
        monkeypatch.setenv("MLCV_PF_WTILE", wt)
        runner.vm._bound = None  # the binding is cached by pointer: force the bind to run again
        print(f"prefill with MLCV_PF_WTILE={wt}", flush=True)
        k, v = runner.vm["prefill"](prefix, pm, params)
        out[wt] = (k.numpy(), v.numpy())
    assert np.all(np.isfinite(out["1"][0])) and np.all(np.isfinite(out["1"][1]))
    np.testing.assert_array_equal(out["1"][0], out["0"][0])
    np.testing.assert_array_equal(out["1"][1], out["0"][1])
