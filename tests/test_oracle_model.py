"""Pins the numpy oracle (oracle/pi0_oracle.py) against independent checks.

Each check is chosen so that a plausible slip in the oracle fails it: library
routines in float64 (torch rms_norm / scaled_dot_product_attention / gelu),
closed forms (time embedding at t=0, constant-velocity Euler), invariants (RoPE
norm and relative position), brute force (masks), and the reference's own gates
(M1 == M0 against an independently written torch joint forward, loop == host
loop, padded == truncated prefix).  Planted mistakes show the gates bite.
"""

from __future__ import annotations

import dataclasses
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F  # noqa: N812

from conftest import cosine, max_abs
from oracle import m0_torch
from oracle import pi0_oracle as O

F64 = O.Prec("f64")

SMALL = O.Dims(vlm_width=64, vlm_mlp=128, ae_width=48, ae_mlp=96, depth=3, num_heads=4, num_kv_heads=1,
               head_dim=16, prefix_len=12, suffix_len=5, action_dim=7, num_steps=3)
HD64 = O.Dims(vlm_width=128, vlm_mlp=256, ae_width=64, ae_mlp=128, depth=2, num_heads=2, num_kv_heads=1,
              head_dim=64, prefix_len=20, suffix_len=6, action_dim=32, num_steps=4)
GQA_FULL = dataclasses.replace(SMALL, num_kv_heads=4)


def _inputs(d: O.Dims, seed=1):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((1, d.prefix_len, d.vlm_width)), rng.standard_normal((1, d.suffix_len, d.action_dim)),
            rng.standard_normal((1, d.ae_width)))


def _m1(params, d, prefix, x_t, te, P=F64, pmask=None, offset=None, rope_offset=None):
    pmask = O.make_prefix_mask_np(d.prefix_len) if pmask is None else pmask
    k, v = O.prefill(params, d, prefix, pmask, P)
    off = d.prefix_len if rope_offset is None else rope_offset
    cos, sin = O.make_rope_np(d.suffix_len, d.head_dim, d.theta, offset=off)
    return O.denoise_step_kv(params, d, k, v, x_t, te, cos, sin, pmask, P)


# ---------------------------------------------------------------- host helpers


def test_time_emb_closed_forms():
    e0 = O.sinusoidal_time_emb(0.0, 64)
    assert np.all(e0[0, :32] == 0.0) and np.all(e0[0, 32:] == 1.0)
    t, dim = 0.7, 1024
    e = O.sinusoidal_time_emb(t, dim)
    half = dim // 2
    for i in (0, 1, 17, half - 1):
        period = math.exp(math.log(4e-3) + (i / (half - 1)) * (math.log(4.0) - math.log(4e-3)))
        ang = 2 * math.pi * t / period
        assert abs(e[0, i] - math.sin(ang)) < 2e-6
        assert abs(e[0, half + i] - math.cos(ang)) < 2e-6


def test_time_grid_is_one_to_one_over_n():
    embs = O.make_time_embs(10, 32)
    ts = [1.0 - 0.1 * i for i in range(10)]
    for e, t in zip(embs, ts):
        np.testing.assert_allclose(e, O.sinusoidal_time_emb(t, 32), atol=1e-6)


def test_rope_tables_norm_and_relative_position():
    hd, theta = 64, 10_000.0
    cos, sin = O.make_rope_np(40, hd, theta, offset=3)
    c, s = cos.reshape(40, hd // 2).astype(np.float64), sin.reshape(40, hd // 2).astype(np.float64)
    np.testing.assert_allclose(c * c + s * s, 1.0, atol=1e-6)
    rng = np.random.default_rng(0)
    q, k = rng.standard_normal((1, 1, hd)), rng.standard_normal((1, 1, hd))
    cf, sf = O.make_rope_np(60, hd, theta, offset=0)
    cf, sf = cf.reshape(60, hd // 2), sf.reshape(60, hd // 2)

    def rot(x, p):
        return O.apply_rope(x, cf[p:p + 1], sf[p:p + 1], F64)

    d1 = float(np.sum(rot(q, 10) * rot(k, 4)))
    d2 = float(np.sum(rot(q, 36) * rot(k, 30)))
    assert abs(d1 - d2) < 1e-5  # q.k depends only on the position difference
    xr = rot(q, 21)
    np.testing.assert_allclose(np.linalg.norm(xr), np.linalg.norm(q), rtol=1e-6)


def test_rope_matches_rotate_half_form():
    hd, L = 16, 9
    x = np.random.default_rng(3).standard_normal((L, 2, hd))
    cos, sin = O.make_rope_np(L, hd, 10_000.0, offset=5)
    got = O.apply_rope(x, cos.reshape(L, hd // 2), sin.reshape(L, hd // 2), F64)
    c = np.concatenate([cos.reshape(L, hd // 2)] * 2, axis=-1)[:, None, :].astype(np.float64)
    s = np.concatenate([sin.reshape(L, hd // 2)] * 2, axis=-1)[:, None, :].astype(np.float64)
    rh = np.concatenate([-x[..., hd // 2:], x[..., :hd // 2]], axis=-1)
    np.testing.assert_allclose(got, x * c + rh * s, atol=1e-12)


def test_prefix_mask_brute_force():
    m = O.make_prefix_mask_np(7, num_valid=4).ravel()
    assert list(m) == [0, 0, 0, 0, -1e9, -1e9, -1e9]
    pad = np.array([1, 0, 1, 1, 0, 0, 1])
    m = O.make_prefix_mask_np(7, num_valid=2, pad_mask=pad).ravel()  # pad_mask wins
    assert [float(v) for v in m] == [0.0 if p else -1e9 for p in pad]
    assert np.all(O.make_prefix_mask_np(5) == 0)


def test_joint_mask_brute_force():
    P, T = 4, 3
    m = O.build_additive_mask(P, T, -5.0, np.float32)[0, 0]
    for i in range(P + T):
        for j in range(P + T):
            allowed = (i >= P) or (j < P)
            assert m[i, j] == (0.0 if allowed else -5.0)
    assert np.isneginf(O.build_additive_mask(P, T, -2.3819763e38, np.float16)).sum() == P * T


def test_euler_constant_velocity():
    x0 = np.ones((1, 2, 3), np.float32)
    out = O.euler_loop(lambda x, i: np.full_like(x, 2.0), x0, 4)
    np.testing.assert_allclose(out, x0 - 2.0, atol=1e-6)


# ---------------------------------------------------------------- model pieces vs torch


def test_rms_norms_vs_torch():
    rng = np.random.default_rng(5)
    x, w = rng.standard_normal((6, 32)), rng.standard_normal(32) * 0.1
    ref = F.rms_norm(torch.tensor(x), (32,), eps=1e-6).numpy() * (1 + w)
    np.testing.assert_allclose(O.rms_norm(x, w, 1e-6, F64), ref, atol=1e-12)
    mod = rng.standard_normal((1, 96)) * 0.1
    out, gate = O.ada_rms_norm(x, mod, 1e-6, F64)
    ref2 = F.rms_norm(torch.tensor(x), (32,), eps=1e-6).numpy() * (1 + mod[:, :32]) + mod[:, 32:64]
    np.testing.assert_allclose(out, ref2, atol=1e-12)
    np.testing.assert_array_equal(gate, mod[:, 64:])


@pytest.mark.parametrize("kv", [1, 4])
def test_sdpa_vs_torch(kv):
    rng = np.random.default_rng(7)
    tq, ts, n, hd = 5, 11, 4, 16
    q = rng.standard_normal((tq, n, hd))
    k = rng.standard_normal((ts, kv, hd))
    v = rng.standard_normal((ts, kv, hd))
    mask = np.where(rng.random(ts) < 0.3, -1e9, 0.0)
    mask[0] = 0.0
    got = O.sdpa(q, k, v, mask, F64)
    qt = torch.tensor(q).permute(1, 0, 2)
    kt = torch.tensor(k).permute(1, 0, 2).expand(n, ts, hd)
    vt = torch.tensor(v).permute(1, 0, 2).expand(n, ts, hd)
    ref = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=torch.tensor(mask)[None, None, :].expand(n, tq, ts),
                                         scale=1.0)
    np.testing.assert_allclose(got, ref.permute(1, 0, 2).reshape(tq, n * hd).numpy(), atol=1e-12)


def test_gelu_tanh_vs_torch():
    x = np.linspace(-6, 6, 101)
    np.testing.assert_allclose(O.gelu_tanh(x), F.gelu(torch.tensor(x), approximate="tanh").numpy(), atol=1e-14)


def test_param_specs_count_and_shapes():
    specs = O.param_specs(SMALL)
    assert len(specs) == 18 * SMALL.depth + 11
    d = dict(specs)
    assert d["backbone.layers.0.mlp.1.gate_up_proj.weight"] == (2 * SMALL.ae_mlp, SMALL.ae_width)
    assert d["backbone.layers.2.input_layernorm.1.modulation.weight"] == (3 * SMALL.ae_width, SMALL.ae_width)
    assert d["action_out_proj.weight"] == (SMALL.action_dim, SMALL.ae_width)
    assert len(set(n for n, _ in specs)) == len(specs)


# ---------------------------------------------------------------- the reference's gates


@pytest.mark.parametrize("d", [SMALL, HD64, GQA_FULL], ids=["hd16", "hd64", "kv_eq_heads"])
def test_m1_equals_m0_fp64(d):
    """compare_kv.py:39-116 in float64: prefill + suffix decode == joint forward."""
    params = O.make_params(O.param_specs(d), 0, "float64")
    prefix, x_t, te = _inputs(d)
    v1 = _m1(params, d, prefix, x_t, te)
    v0 = m0_torch.denoise_step_m0(params, d, prefix, x_t, te)
    assert max_abs(v1, v0) < 1e-10 * max(1.0, np.abs(v0).max())


def test_m1_equals_m0_detects_planted_mistakes():
    d = SMALL
    params = O.make_params(O.param_specs(d), 0, "float64")
    prefix, x_t, te = _inputs(d)
    v0 = m0_torch.denoise_step_m0(params, d, prefix, x_t, te)
    # wrong suffix RoPE offset (0 instead of the prefix length)
    assert max_abs(_m1(params, d, prefix, x_t, te, rope_offset=0), v0) > 1e-6
    # prefix K/V of the wrong layer (layers swapped)
    pm = O.make_prefix_mask_np(d.prefix_len)
    k, v = O.prefill(params, d, prefix, pm, F64)
    cos, sin = O.make_rope_np(d.suffix_len, d.head_dim, d.theta, offset=d.prefix_len)
    bad = O.denoise_step_kv(params, d, k[::-1].copy(), v[::-1].copy(), x_t, te, cos, sin, pm, F64)
    assert max_abs(bad, v0) > 1e-6


def test_loop_equals_host_loop_bitexact_f32():
    """compare_loop.py:27-61: in-graph Euler loop == host loop (float32)."""
    d = SMALL
    P = O.Prec("f32")
    params = O.make_params(O.param_specs(d), 0, "float32")
    prefix, _, _ = _inputs(d)
    noise = np.random.default_rng(3).standard_normal((1, d.suffix_len, d.action_dim)).astype(np.float32)
    host = O.sample(params, d, prefix, noise, P, num_steps=d.num_steps)
    graph = O.sample(params, d, prefix, noise, P, graph=True)
    np.testing.assert_array_equal(host, graph)


def test_pad_invariance_fp64():
    """compare_pad.py:62-91: garbage x10 in padded prefix rows is fully masked."""
    pad = 5
    d_full = dataclasses.replace(SMALL, prefix_len=16)
    d_trunc = dataclasses.replace(SMALL, prefix_len=16 - pad)
    rng = np.random.default_rng(0)
    params = O.make_params(O.param_specs(d_full), 0, "float64")
    prefix = 0.02 * rng.standard_normal((1, 16, d_full.vlm_width))
    prefix[:, 16 - pad:] = 10.0 * rng.standard_normal((1, pad, d_full.vlm_width))
    x_t = np.zeros((1, d_full.suffix_len, d_full.action_dim))
    te = O.sinusoidal_time_emb(0.7, d_full.ae_width).astype(np.float64)
    valid = 16 - pad
    v_full = _m1(params, d_full, prefix, x_t, te, pmask=O.make_prefix_mask_np(16, num_valid=valid),
                 rope_offset=valid)
    v_trunc = _m1(params, d_trunc, prefix[:, :valid], x_t, te, rope_offset=valid)
    assert max_abs(v_full, v_trunc) < 1e-10
    # without the mask the garbage leaks in
    v_leak = _m1(params, d_full, prefix, x_t, te, rope_offset=valid)
    assert max_abs(v_leak, v_trunc) > 1e-6


def test_fp16_emulation_tracks_fp64():
    d = HD64
    params = O.make_params(O.param_specs(d), 0, "float64")
    prefix, x_t, te = _inputs(d)
    truth = _m1(params, d, prefix, x_t, te)
    P = O.Prec("f16")
    p16 = {k: v.astype(np.float16) for k, v in params.items()}
    got = _m1(p16, d, P.cast(prefix), P.cast(x_t), P.cast(te), P=P)
    assert cosine(got, truth) > 0.9999
    assert max_abs(got, truth) < 5e-3


def test_embed_language_is_one_fp16_rounding_of_the_exact_product():
    """embed_language: table rows times the fp16 constant sqrt(width), rounded once to fp16.
    Checked against the float64 product rounded to fp16 over normal, subnormal and
    near-overflow entries; a float32 constant or a double rounding would differ."""
    rng = np.random.default_rng(11)
    width = 2048
    table = np.concatenate([rng.standard_normal((40, width)) * s for s in (1e-6, 1e-3, 1.0, 30.0, 1400.0)])
    table = table.astype(np.float16)
    ids = rng.integers(0, table.shape[0], size=(1, 77))
    got = O.embed_language(table, ids)
    c = np.float16(np.sqrt(width))
    assert c == np.float16(45.25)
    with np.errstate(over="ignore"):  # the largest rows overflow to inf in fp16
        exact = (table[ids].astype(np.float64) * np.float64(c)).astype(np.float16)
        wrong = (table[ids].astype(np.float32) * np.float32(np.sqrt(width))).astype(np.float16)
    np.testing.assert_array_equal(got.view(np.uint16), exact.view(np.uint16))
    assert got.shape == (1, 77, width) and got.dtype == np.float16
    assert not np.array_equal(got.view(np.uint16), wrong.view(np.uint16))
