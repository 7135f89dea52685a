"""Model-level parity on the GPU through the drop-in API (PiZeroRunner / VM functions),
mirroring the reference's e2e tests (python/tests/test_compile_and_run.py,
test_numerical_gates.py, test_pizero_runner.py) and its CLI gates (compare_kv,
compare_loop, compare_pad, compare_quant), each checked against the oracle.

Tolerance on actions / velocities (fp16 kernels vs the float32 oracle on the same
fp16-valued weights): max_abs <= 1e-2 and cosine >= 0.999.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest

from conftest import DUMMY_KWARGS, TINY_KWARGS, cosine, max_abs
from mlc_vla import runtime
from mlc_vla.compile_quant import compile_model_quant, quantize_params
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.model.pi0.pi0_config import GemmaExpertConfig
from mlc_vla.sample import PiZeroRunner, make_prefix_mask_np, make_rope_np, make_time_embs
from oracle import m0_torch
from oracle import pi0_oracle as O
from oracle import q4_oracle as Q

pytestmark = pytest.mark.gpu

F32 = O.Prec("f32")
F16 = O.Prec("f16")


def _tol(got, ref, atol=1e-2, cos=0.999):
    assert np.all(np.isfinite(got))
    assert max_abs(got, ref) <= atol, max_abs(got, ref)
    assert cosine(got, ref) >= cos, cosine(got, ref)


class Model:
    def __init__(self, kw, seed=0):
        self.cfg = Pi0Config(**kw)
        self.d = O.dims_from_config(self.cfg)
        print(f"model {kw.get('paligemma_variant')} P={self.cfg.prefix_len} T={self.cfg.suffix_len}", flush=True)
        self.runner = PiZeroRunner(self.cfg, "rocm")
        specs = O.param_specs(self.d)
        self.p16 = O.make_params(specs, seed, "float16")
        self.p32 = {k: v.astype(np.float32) for k, v in self.p16.items()}
        self.params = self.runner.to_params([self.p16[n] for n, _ in self.runner.named_params])
        rng = np.random.default_rng(1)
        self.prefix = rng.standard_normal((1, self.cfg.prefix_len, self.cfg.vlm.width)).astype(np.float16)
        self.x_t = rng.standard_normal((1, self.cfg.action_horizon, self.cfg.action_dim)).astype(np.float16)
        self.noise = rng.standard_normal((1, self.cfg.action_horizon, self.cfg.action_dim)).astype(np.float32)

    def dev(self, a):
        return runtime.tensor(np.asarray(a), self.runner.dev)


@pytest.fixture(scope="module")
def tiny():
    return Model(TINY_KWARGS)


@pytest.fixture(scope="module")
def dummy():
    return Model(DUMMY_KWARGS)


def _prefill(m: Model, pmask_np):
    k, v = m.runner.vm["prefill"](m.dev(m.prefix), m.dev(pmask_np), m.params)
    return k, v


def test_prefill_kv_vs_oracle(tiny):
    m = tiny
    pm = make_prefix_mask_np(m.cfg.prefix_len)
    k, v = _prefill(m, pm)
    assert k.shape == (2, 1, 1, 32, 64) and k.dtype == "float32" and v.dtype == "float16"
    k_ref, v_ref = O.prefill(m.p32, m.d, m.prefix, pm, F32)
    for L in range(m.d.depth):  # every layer's cache, so layer L-1's attention/MLP is exercised
        _tol(k.numpy()[L], k_ref[L], atol=2e-2 * np.abs(k_ref[L]).max(), cos=0.99995)
        _tol(v.numpy()[L], v_ref[L], atol=2e-2 * np.abs(v_ref[L]).max(), cos=0.99995)


@pytest.mark.parametrize("which", ["tiny", "dummy"])
def test_denoise_step_kv_vs_oracle(which, tiny, dummy):
    m = tiny if which == "tiny" else dummy
    pm = make_prefix_mask_np(m.cfg.prefix_len)
    k, v = _prefill(m, pm)
    cos, sin = make_rope_np(m.cfg.suffix_len, m.cfg.vlm.head_dim, m.cfg.rope_theta, offset=m.cfg.prefix_len)
    te = make_time_embs(m.cfg.num_denoise_steps, m.cfg.action_expert.width)[0].astype(np.float16)
    vel = m.runner.vm["denoise_step_kv"](k, v, m.dev(m.x_t), m.dev(te), m.dev(cos), m.dev(sin), m.dev(pm), m.params)
    got = vel.numpy()
    assert got.shape == (1, m.cfg.action_horizon, m.cfg.action_dim) and got.dtype == np.float32
    k_ref, v_ref = O.prefill(m.p32, m.d, m.prefix, pm, F32)
    ref = O.denoise_step_kv(m.p32, m.d, k_ref, v_ref, m.x_t, te, cos, sin, pm, F32)
    _tol(got, ref)


def test_long_horizon_rowmajor_path():
    """Action horizon 72 (two 64-row blocks): the row-major kernels with the per-element
    adaRMS prologue instead of the fragment-major path, for one step and the graph loop."""
    m = Model(dict(TINY_KWARGS, action_horizon=72))
    pm = make_prefix_mask_np(m.cfg.prefix_len)
    k, v = _prefill(m, pm)
    cos, sin = make_rope_np(m.cfg.suffix_len, m.cfg.vlm.head_dim, m.cfg.rope_theta, offset=m.cfg.prefix_len)
    te = make_time_embs(m.cfg.num_denoise_steps, m.cfg.action_expert.width)[3].astype(np.float16)
    got = m.runner.vm["denoise_step_kv"](k, v, m.dev(m.x_t), m.dev(te), m.dev(cos), m.dev(sin), m.dev(pm),
                                         m.params).numpy()
    k_ref, v_ref = O.prefill(m.p32, m.d, m.prefix, pm, F32)
    _tol(got, O.denoise_step_kv(m.p32, m.d, k_ref, v_ref, m.x_t, te, cos, sin, pm, F32))
    graph = m.runner.sample_graph(m.params, m.prefix, noise=m.noise)
    _tol(graph, O.sample(m.p32, m.d, m.prefix, m.noise, F32, graph=True))


def test_m1_vs_m0_joint_forward(tiny):
    """compare_kv: the GPU M1 path against the float64 joint (M0) forward."""
    m = tiny
    pm = make_prefix_mask_np(m.cfg.prefix_len)
    k, v = _prefill(m, pm)
    cos, sin = make_rope_np(m.cfg.suffix_len, m.cfg.vlm.head_dim, m.cfg.rope_theta, offset=m.cfg.prefix_len)
    te = np.random.default_rng(4).standard_normal((1, m.cfg.action_expert.width)).astype(np.float16)
    got = m.runner.vm["denoise_step_kv"](k, v, m.dev(m.x_t), m.dev(te), m.dev(cos), m.dev(sin), m.dev(pm),
                                         m.params).numpy()
    ref = m0_torch.denoise_step_m0({k_: v_.astype(np.float64) for k_, v_ in m.p16.items()}, m.d,
                                   m.prefix.astype(np.float64), m.x_t.astype(np.float64), te.astype(np.float64))
    _tol(got, ref)


@pytest.mark.parametrize("which", ["tiny", "dummy"])
def test_denoise_step_joint_vs_m0_oracle_and_m1(which, tiny, dummy):
    """vm["denoise_step"] (Pi0Model.denoise_step, the joint prefix + suffix forward, all prefix
    tokens valid) against the float64 torch joint forward, and against the M1 path on the GPU
    (prefill + denoise_step_kv with suffix RoPE positions P..P+T-1): compare_kv's gate.  The M1
    tables come from numpy's float64 cos/sin and the joint forward's from the C library, which
    may differ in the last float32 ulp, so M1 is compared to a tight tolerance, not bitwise."""
    m = tiny if which == "tiny" else dummy
    te = np.random.default_rng(6).standard_normal((1, m.cfg.action_expert.width)).astype(np.float16)
    got = m.runner.vm["denoise_step"](m.dev(m.prefix), m.dev(m.x_t), m.dev(te), m.params).numpy()
    assert got.shape == (1, m.cfg.action_horizon, m.cfg.action_dim) and got.dtype == np.float32
    ref = m0_torch.denoise_step_m0({k_: v_.astype(np.float64) for k_, v_ in m.p16.items()}, m.d,
                                   m.prefix.astype(np.float64), m.x_t.astype(np.float64), te.astype(np.float64))
    _tol(got, ref)
    pm = make_prefix_mask_np(m.cfg.prefix_len)
    k, v = _prefill(m, pm)
    cos, sin = make_rope_np(m.cfg.suffix_len, m.cfg.vlm.head_dim, m.cfg.rope_theta, offset=m.cfg.prefix_len)
    m1 = m.runner.vm["denoise_step_kv"](k, v, m.dev(m.x_t), m.dev(te), m.dev(cos), m.dev(sin), m.dev(pm),
                                        m.params).numpy()
    assert cosine(got, m1) >= 0.999999
    assert max_abs(got, m1) <= 1e-3 * max(1.0, float(np.abs(m1).max()))
    # a second call replays the joint graph with new inputs staged into it
    x2 = np.random.default_rng(13).standard_normal(m.x_t.shape).astype(np.float16)
    got2 = m.runner.vm["denoise_step"](m.dev(m.prefix), m.dev(x2), m.dev(te), m.params).numpy()
    ref2 = m0_torch.denoise_step_m0({k_: v_.astype(np.float64) for k_, v_ in m.p16.items()}, m.d,
                                    m.prefix.astype(np.float64), x2.astype(np.float64), te.astype(np.float64))
    _tol(got2, ref2)
    assert not np.array_equal(got2, got)


def test_vm_embed_language(tiny):
    """vm["embed_language"] from compile_model(functions=["embed_language"]): the parameter list
    is [embed_tokens.weight] at the PaliGemma vocabulary; bit-exact against the oracle."""
    from mlc_vla.compile import compile_model
    from mlc_vla.runtime import VirtualMachine

    cfg = tiny.cfg
    ex, npar = compile_model(cfg, "rocm", functions=["embed_language"])
    assert [n for n, _ in npar] == ["embed_tokens.weight"] and npar[0][1].shape == (257152, cfg.vlm.width)
    vm = VirtualMachine(ex, tiny.runner.dev)
    rng = np.random.default_rng(12)
    table = rng.standard_normal(npar[0][1].shape, dtype=np.float32).astype(np.float16)
    ids = rng.integers(0, 257152, size=(1, cfg.max_token_len)).astype(np.int32)
    got = vm["embed_language"](tiny.dev(ids), [tiny.dev(table)]).numpy()
    assert got.shape == (1, cfg.max_token_len, cfg.vlm.width) and got.dtype == np.float16
    np.testing.assert_array_equal(got.view(np.uint16), O.embed_language(table, ids).view(np.uint16))
    with pytest.raises(KeyError):
        vm["prefill"]


@pytest.mark.parametrize("sig", [
    dict(image_size=28, patch_size=14, hidden_size=144, intermediate_size=200, num_hidden_layers=2,
         num_attention_heads=2, projection_dim=64),
    dict(image_size=56, patch_size=14, hidden_size=128, intermediate_size=96, num_hidden_layers=1,
         num_attention_heads=2, projection_dim=32),
    dict(num_hidden_layers=1),  # one layer of So400m/14 at 224 x 224: 256 patches, hd 72, projector to 2048
    dict(),  # the whole So400m/14 tower (27 layers) + projector, as pi0.5 runs it
], ids=["hd72", "hd64", "so400m_1layer", "so400m_27layers"])
def test_vm_embed_image_vs_oracle(sig, tiny):
    """vm["embed_image"] (SigLIP tower + projector, siglip.py:20-120, pi0_model.py:97-99) against
    the oracle at the reference's fp16 cast points (siglip_oracle, pinned to torch conv2d /
    layer_norm / SDPA in float64), up to the full 27-layer So400m/14 tower."""
    print(f"embed_image {sig}", flush=True)
    from mlc_vla.compile import compile_model
    from mlc_vla.model.pi0 import Pi0Config, SiglipConfig
    from mlc_vla.runtime import VirtualMachine
    from oracle import siglip_oracle as S

    sc = SiglipConfig(**sig)
    cfg = Pi0Config(**{**TINY_KWARGS, "siglip": sc})
    ex, npar = compile_model(cfg, "rocm", functions=["embed_image"])
    assert [n for n, _ in npar] == [n for n, _ in S.vision_param_specs(sc)]
    vm = VirtualMachine(ex, tiny.runner.dev)
    P = S.make_vision_params(sc, 7)
    img = np.random.default_rng(8).standard_normal((sc.image_size, sc.image_size, sc.num_channels)).astype(np.float16)
    got = vm["embed_image"](tiny.dev(img[None]), [tiny.dev(P[n]) for n, _ in npar]).numpy()
    assert got.shape == (1, sc.num_patches, sc.projection_dim) and got.dtype == np.float16
    ref = S.embed_image(P, sc, img, "f16")
    g = got[0].astype(np.float64)
    print(f"embed_image: cos {cosine(g, ref):.7f} max_abs {max_abs(g, ref):.3e} max|ref| {np.abs(ref).max():.3f}",
          flush=True)
    assert np.all(np.isfinite(g))
    assert cosine(g, ref) >= 0.9999, cosine(g, ref)
    assert max_abs(g, ref) <= 2e-2 * float(np.abs(ref).max()), (max_abs(g, ref), float(np.abs(ref).max()))
    # the second call replays the captured graph: the new image is staged into it
    img2 = np.random.default_rng(9).standard_normal(img.shape).astype(np.float16)
    params = [tiny.dev(P[n]) for n, _ in npar]
    got2 = vm["embed_image"](tiny.dev(img2[None]), params).numpy()[0].astype(np.float64)
    again = vm["embed_image"](tiny.dev(img[None]), params).numpy()[0]
    ref2 = S.embed_image(P, sc, img2, "f16")
    assert cosine(got2, ref2) >= 0.9999 and max_abs(got2, ref2) <= 2e-2 * float(np.abs(ref2).max())
    np.testing.assert_array_equal(again, got[0])


def test_sample_vs_oracle_and_graph_loop(tiny):
    """sample (host loop) vs the oracle; sample_graph (device loop) vs sample (compare_loop)."""
    m = tiny
    host = m.runner.sample(m.params, m.prefix, noise=m.noise, num_steps=m.cfg.num_denoise_steps)
    graph = m.runner.sample_graph(m.params, m.prefix, noise=m.noise)
    assert host.shape == graph.shape == (1, m.cfg.action_horizon, m.cfg.action_dim)
    assert cosine(host, graph) >= 0.99999
    np.testing.assert_array_equal(host, graph)  # same kernels, same fp32 Euler update
    ref = O.sample(m.p32, m.d, m.prefix, m.noise, F32, num_steps=m.cfg.num_denoise_steps)
    _tol(host, ref)


def test_graph_capture_equals_eager(tiny):
    m = tiny
    x_graph = m.runner.sample_graph(m.params, m.prefix, noise=m.noise)
    m.runner.vm.set_graph(False)
    try:
        x_eager = m.runner.sample_graph(m.params, m.prefix, noise=m.noise)
        m.runner.vm.set_hoist(False)
        x_nohoist = m.runner.sample_graph(m.params, m.prefix, noise=m.noise)
    finally:
        m.runner.vm.set_graph(True)
        m.runner.vm.set_hoist(True)
    np.testing.assert_array_equal(x_graph, x_eager)
    np.testing.assert_array_equal(x_graph, x_nohoist)
    # replay the captured graph several times with eager work in between
    for _ in range(3):
        np.testing.assert_array_equal(m.runner.sample_graph(m.params, m.prefix, noise=m.noise), x_graph)


def test_chunk_equals_prefill_plus_loop(tiny):
    m = tiny
    cfg = m.cfg
    pm = make_prefix_mask_np(cfg.prefix_len)
    cos, sin = make_rope_np(cfg.suffix_len, cfg.vlm.head_dim, cfg.rope_theta, offset=cfg.prefix_len)
    tes = np.concatenate(make_time_embs(cfg.num_denoise_steps, cfg.action_expert.width), 0).astype(np.float16)
    x = m.runner.vm["chunk"](m.dev(m.prefix), m.dev(pm), m.dev(m.noise), m.dev(tes), m.dev(cos), m.dev(sin),
                             m.params).numpy()
    np.testing.assert_array_equal(x, m.runner.sample_graph(m.params, m.prefix, noise=m.noise))


def test_prefix_pad_invariance():
    """compare_pad: padded prefix (garbage x10 in the padding, masked) == truncated prefix."""
    pad = 5
    base = dict(TINY_KWARGS)
    full = Model({**base, "max_token_len": 32})
    trunc_cfg = Pi0Config(**{**base, "max_token_len": 32 - pad})
    trunc = PiZeroRunner(trunc_cfg, "rocm")
    params_t = trunc.to_params([full.p16[n] for n, _ in trunc.named_params])
    rng = np.random.default_rng(0)
    prefix = (0.02 * rng.standard_normal((1, 32, 256))).astype(np.float16)
    prefix[:, 32 - pad:] = (10.0 * rng.standard_normal((1, pad, 256))).astype(np.float16)
    pad_mask = (np.arange(32) < 32 - pad).astype(np.float32)
    noise = rng.standard_normal((1, 8, 32)).astype(np.float32)
    a = full.runner.sample(full.params, prefix, noise=noise, num_steps=3, prefix_pad=pad_mask)
    b = trunc.sample(params_t, prefix[:, :32 - pad], noise=noise, num_steps=3)
    assert cosine(a, b) >= 0.9999 and max_abs(a, b) < 1e-2
    leak = full.runner.sample(full.params, prefix, noise=noise, num_steps=3)  # no mask: garbage leaks
    assert max_abs(leak, b) > max_abs(a, b)


def test_reference_dummy_contract(dummy):
    """test_compile_and_run / test_pizero_runner on the reference's dummy test model."""
    m = dummy
    cfg = m.cfg
    pm = make_prefix_mask_np(cfg.prefix_len)
    k, v = _prefill(m, pm)
    assert cfg.prefix_len in k.shape and cfg.vlm.head_dim in k.shape
    assert np.all(np.isfinite(k.numpy())) and np.all(np.isfinite(v.numpy().astype(np.float32)))
    out = m.runner.sample(m.params, m.prefix, num_steps=cfg.num_denoise_steps, seed=7)
    assert out.shape == (1, cfg.action_horizon, cfg.action_dim) and out.dtype == np.float32
    half = np.zeros(cfg.prefix_len, np.float32)
    half[: cfg.prefix_len // 2] = 1.0
    out2 = m.runner.sample(m.params, m.prefix, num_steps=cfg.num_denoise_steps, seed=1, prefix_pad=half)
    assert np.all(np.isfinite(out2))
    ref = O.sample(m.p32, m.d, m.prefix, np.random.default_rng(1).standard_normal(
        (1, cfg.action_horizon, cfg.action_dim)).astype(np.float32), F32, num_steps=cfg.num_denoise_steps,
        prefix_pad=half)
    _tol(out2, ref)


def test_q4_path_vs_oracle_and_vs_fp(tiny):
    """compare_quant: q4f16_1 weights (quantized on the GPU) vs the fp path (cos >= 0.97),
    and vs the oracle run on the same quantized weights (tight)."""
    m = tiny
    ex, qnp, qmap, quant = compile_model_quant(m.cfg, "rocm", None, "q4f16_1")
    src = {n: v for n, v in m.p16.items()}
    qparams = quantize_params(quant, src, qnp, qmap)
    qref = Q.quantize_params(src, O.param_specs(m.d))
    for name in qref:
        np.testing.assert_array_equal(np.asarray(qparams[name]).view(np.uint8), np.asarray(qref[name]).view(np.uint8))
    vm = runtime.VirtualMachine(ex, m.runner.dev)
    tp = [runtime.tensor(qparams[n], m.runner.dev) for n, _ in qnp]
    cfg = m.cfg
    pm = make_prefix_mask_np(cfg.prefix_len)
    cos, sin = make_rope_np(cfg.suffix_len, cfg.vlm.head_dim, cfg.rope_theta, offset=cfg.prefix_len)
    te = O.sinusoidal_time_emb(0.7, cfg.action_expert.width).astype(np.float16)
    kq, vq = vm["prefill"](m.dev(m.prefix), m.dev(pm), tp)
    vel_q = vm["denoise_step_kv"](kq, vq, m.dev(m.x_t), m.dev(te), m.dev(cos), m.dev(sin), m.dev(pm), tp).numpy()
    k, v = _prefill(m, pm)
    vel_fp = m.runner.vm["denoise_step_kv"](k, v, m.dev(m.x_t), m.dev(te), m.dev(cos), m.dev(sin), m.dev(pm),
                                            m.params).numpy()
    assert cosine(vel_q, vel_fp) >= 0.97
    q32 = {n: (a if a.dtype == np.uint32 else a.astype(np.float32)) for n, a in qref.items()}
    kr, vr = O.prefill(q32, m.d, m.prefix, pm, F32)
    ref = O.denoise_step_kv(q32, m.d, kr, vr, m.x_t, te, cos, sin, pm, F32)
    _tol(vel_q, ref)


@pytest.mark.parametrize("kw", [TINY_KWARGS, DUMMY_KWARGS], ids=["tiny", "dummy"])
def test_multi_slab_tiles_bit_identical(kw, monkeypatch):
    """32-row fragment-major tiles (every wave multiplies its X fragments by both 16-row
    weight slabs) split K over the same 4 waves and sum the k groups in the same order as
    16-row tiles: with equal K slices the step and the graph loop are bit-identical (gate_up
    defaults to 32-row tiles for fp16, so the variant runs it on 16)."""
    ref = Model(kw)
    monkeypatch.setenv("MLCV_TILING", "o=32:2,gu=16:1,down=32:4")
    alt = Model(kw)
    monkeypatch.delenv("MLCV_TILING")
    pm = make_prefix_mask_np(ref.cfg.prefix_len)
    cos, sin = make_rope_np(ref.cfg.suffix_len, ref.cfg.vlm.head_dim, ref.cfg.rope_theta,
                            offset=ref.cfg.prefix_len)
    te = make_time_embs(ref.cfg.num_denoise_steps, ref.cfg.action_expert.width)[2].astype(np.float16)
    outs = []
    for m in (ref, alt):
        k, v = _prefill(m, pm)
        step = m.runner.vm["denoise_step_kv"](k, v, m.dev(m.x_t), m.dev(te), m.dev(cos), m.dev(sin), m.dev(pm),
                                              m.params).numpy()
        outs.append((step, m.runner.sample_graph(m.params, m.prefix, noise=m.noise)))
    assert np.all(np.isfinite(outs[0][0])) and np.all(np.isfinite(outs[0][1]))
    np.testing.assert_array_equal(outs[1][0], outs[0][0])
    np.testing.assert_array_equal(outs[1][1], outs[0][1])


# one layer with 8 heads of 256: o_proj has K = 2048, which 4 m groups take in one round of
# 16 chunks (two rounds of 8 otherwise)
_WIDE = GemmaExpertConfig(width=256, depth=1, mlp_dim=512, num_heads=8, num_kv_heads=1, head_dim=256)
WIDE_HEADS_KWARGS = dict(TINY_KWARGS, paligemma_variant=_WIDE, action_expert_variant=_WIDE, action_horizon=50)


@pytest.mark.parametrize("kw", [dict(TINY_KWARGS, action_horizon=50), DUMMY_KWARGS, WIDE_HEADS_KWARGS],
                         ids=["tiny_h50", "dummy", "wide_heads"])
def test_m_group_tiles_bit_identical(kw, monkeypatch):
    """o_proj and down with their 16-row weight slabs shared out over 1, 2 or 4 workgroups
    (each multiplying 4, 2 or 1 of the 64-row block's m tiles over the same K slices and k
    groups; with 4 groups a K of 2048 runs as one 16-chunk round laid out as two 8-chunk ones):
    the step and the graph loop are bit-identical whatever the m groups."""
    outs = []
    for til in ("o=16:1:1,down=16:4:1", "o=16:1:2,down=16:4:2", "o=16:1:4,down=16:4:4", None):
        if til:
            monkeypatch.setenv("MLCV_TILING", til)
        m = Model(kw)
        if til:
            monkeypatch.delenv("MLCV_TILING")
        pm = make_prefix_mask_np(m.cfg.prefix_len)
        cos, sin = make_rope_np(m.cfg.suffix_len, m.cfg.vlm.head_dim, m.cfg.rope_theta, offset=m.cfg.prefix_len)
        te = make_time_embs(m.cfg.num_denoise_steps, m.cfg.action_expert.width)[2].astype(np.float16)
        k, v = _prefill(m, pm)
        step = m.runner.vm["denoise_step_kv"](k, v, m.dev(m.x_t), m.dev(te), m.dev(cos), m.dev(sin), m.dev(pm),
                                              m.params).numpy()
        outs.append((step, m.runner.sample_graph(m.params, m.prefix, noise=m.noise)))
    assert np.all(np.isfinite(outs[0][0])) and np.all(np.isfinite(outs[0][1]))
    for step, chunk in outs[1:]:
        np.testing.assert_array_equal(step, outs[0][0])
        np.testing.assert_array_equal(chunk, outs[0][1])


@pytest.mark.parametrize("kw", [dict(TINY_KWARGS, action_horizon=50), WIDE_HEADS_KWARGS], ids=["tiny_h50", "wide_heads"])
def test_attention_task_order_bit_identical(kw, monkeypatch):
    """The step attention's workgroups in the XCD-grouped order (every row block of a key split
    on one XCD) and in grid order run the same tasks: bit-identical steps and chunks."""
    outs = []
    for xg in ("0", None):
        if xg:
            monkeypatch.setenv("MLCV_ATTN_XG", xg)
        m = Model(kw)
        if xg:
            monkeypatch.delenv("MLCV_ATTN_XG")
        pm = make_prefix_mask_np(m.cfg.prefix_len)
        cos, sin = make_rope_np(m.cfg.suffix_len, m.cfg.vlm.head_dim, m.cfg.rope_theta, offset=m.cfg.prefix_len)
        te = make_time_embs(m.cfg.num_denoise_steps, m.cfg.action_expert.width)[4].astype(np.float16)
        k, v = _prefill(m, pm)
        step = m.runner.vm["denoise_step_kv"](k, v, m.dev(m.x_t), m.dev(te), m.dev(cos), m.dev(sin), m.dev(pm),
                                              m.params).numpy()
        outs.append((step, m.runner.sample_graph(m.params, m.prefix, noise=m.noise)))
    assert np.all(np.isfinite(outs[0][0])) and np.all(np.isfinite(outs[0][1]))
    np.testing.assert_array_equal(outs[1][0], outs[0][0])
    np.testing.assert_array_equal(outs[1][1], outs[0][1])


def test_side_stream_modulations_bit_identical(tiny, monkeypatch):
    """The modulations as one launch over all 2 D + 1 norms (default) and as two pieces on
    a second stream (MLCV_FORK_MOD=1, layer 0 first) run the same tiles: the step and the
    graph loop are bit-identical."""
    monkeypatch.setenv("MLCV_FORK_MOD", "1")
    alt = Model(TINY_KWARGS)
    monkeypatch.delenv("MLCV_FORK_MOD")
    ref = tiny
    pm = make_prefix_mask_np(ref.cfg.prefix_len)
    cos, sin = make_rope_np(ref.cfg.suffix_len, ref.cfg.vlm.head_dim, ref.cfg.rope_theta,
                            offset=ref.cfg.prefix_len)
    te = make_time_embs(ref.cfg.num_denoise_steps, ref.cfg.action_expert.width)[3].astype(np.float16)
    outs = []
    for m in (ref, alt):
        k, v = _prefill(m, pm)
        step = m.runner.vm["denoise_step_kv"](k, v, m.dev(m.x_t), m.dev(te), m.dev(cos), m.dev(sin), m.dev(pm),
                                              m.params).numpy()
        outs.append((step, m.runner.sample_graph(m.params, m.prefix, noise=m.noise)))
    assert np.all(np.isfinite(outs[0][0])) and np.all(np.isfinite(outs[0][1]))
    np.testing.assert_array_equal(outs[1][0], outs[0][0])
    np.testing.assert_array_equal(outs[1][1], outs[0][1])


def test_full_size_step_vs_oracle():
    """One fp16 denoise_step_kv at the full pi0.5 shape (18 layers, width 1024, P=968, T=50)
    against the float32 oracle, with N(0,1) stand-in prefix K/V."""
    cfg = Pi0Config(dtype="float16", action_horizon=50)
    d = O.dims_from_config(cfg)
    runner = PiZeroRunner(cfg, "rocm")
    names = [n for n, _ in runner.named_params]
    is_ae = lambda n: not (".experts.0." in n or ".mlp.0." in n)  # noqa: E731
    p16 = O.make_params([(n, s) for n, s in O.param_specs(d) if is_ae(n)], 0, "float16")
    dummy0 = {}
    params = []
    for n, p in runner.named_params:  # expert-0 weights are not read by denoise_step_kv
        if n in p16:
            params.append(runtime.tensor(p16[n], runner.dev))
        else:
            dummy0[n] = runtime.empty(p.shape, "float16", runner.dev)
            params.append(dummy0[n])
    rng = np.random.default_rng(5)
    keys = rng.standard_normal((18, 1, 1, 968, 256)).astype(np.float32)
    values = rng.standard_normal((18, 1, 1, 968, 256)).astype(np.float16)
    x_t = rng.standard_normal((1, 50, 32)).astype(np.float16)
    te = O.sinusoidal_time_emb(1.0, 1024).astype(np.float16)
    pm = make_prefix_mask_np(968)
    cos, sin = make_rope_np(50, 256, 10_000.0, offset=968)
    dv = lambda a: runtime.tensor(a, runner.dev)  # noqa: E731
    got = runner.vm["denoise_step_kv"](dv(keys), dv(values), dv(x_t), dv(te), dv(cos), dv(sin), dv(pm),
                                       params).numpy()
    p32 = {n: v.astype(np.float32) for n, v in p16.items()}
    ref = O.denoise_step_kv(p32, d, keys, values, x_t, te, cos, sin, pm, F32)
    _tol(got, ref)
    assert len(names) == 335
