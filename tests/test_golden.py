"""The oracle against the committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py), plus an independent library restatement of the
isolated attention fixture (torch scaled_dot_product_attention in float64)."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from conftest import ROOT, cosine, max_abs
from oracle import pi0_oracle as O
from oracle import q4_oracle as Q

GOLDEN = os.path.join(ROOT, "tests", "golden")
if GOLDEN not in sys.path:
    sys.path.insert(0, GOLDEN)
import make_golden as G  # noqa: E402


def _load(name):
    return np.load(os.path.join(GOLDEN, name))


@pytest.fixture(scope="module")
def tiny():
    return G.tiny_inputs(), _load("tiny_e2e.npz")


def test_tiny_inputs_regenerate(tiny):
    (specs, params, prefix, noise), fx = tiny
    s, ss = G.checksums(params, specs)
    np.testing.assert_allclose(s, fx["param_sum"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ss, fx["param_sumsq"], rtol=1e-12)
    np.testing.assert_array_equal(prefix, fx["prefix_embs"])
    np.testing.assert_array_equal(noise, fx["noise"])


def test_tiny_oracle_reproduces_fixture(tiny):
    (specs, params, prefix, noise), fx = tiny
    got = G.tiny_outputs(params, prefix, noise, "f32")
    for k in ("keys", "values", "v1", "actions", "actions_graph"):
        # float32 BLAS kernels differ between CPUs in summation order only
        np.testing.assert_allclose(got[k], fx[k], rtol=2e-4, atol=2e-5 * float(np.abs(fx[k]).max()), err_msg=k)
    got64 = G.tiny_outputs(params, prefix, noise, "f64")
    for k in ("v1", "actions", "actions_graph"):
        np.testing.assert_allclose(got64[k], fx[k + "_f64"], rtol=1e-9, atol=1e-12, err_msg=k)


def test_tiny_fixture_consistency(tiny):
    _, fx = tiny
    # float32 and float64 restatements agree far inside the action tolerance
    for k in ("v1", "actions", "actions_graph"):
        assert max_abs(fx[k], fx[k + "_f64"]) < 1e-4, k
        assert cosine(fx[k], fx[k + "_f64"]) > 0.999999, k
    # in-graph loop (x fed back as dt(x), dt = -1/N) == host Euler loop for float32
    np.testing.assert_allclose(fx["actions_graph"], fx["actions"], rtol=0, atol=1e-6)
    assert fx["keys"].shape == (2, 1, 1, 32, 64) and fx["v1"].shape == (1, 8, 32)


def test_attention_fixture_vs_oracle_and_torch():
    fx = _load("attn_isolated.npz")
    q, kp, vp, ks, vs, mask = G.attn_inputs(**G.ATTN)
    sums = np.array([np.sum(a.astype(np.float64)) for a in (q, kp, vp, ks, vs)])
    np.testing.assert_allclose(sums, fx["input_sums"], rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(mask, fx["mask"])
    ref = G.attn_reference(q, kp, vp, ks, vs, mask, "f64")
    np.testing.assert_allclose(ref, fx["out_f64"], rtol=1e-6, atol=1e-9)
    # independent: torch SDPA in float64, 8 query heads over the one shared kv head
    tq, h, hd = q.shape[0], 8, 256
    qt = torch.from_numpy(q.astype(np.float64).reshape(tq, h, hd).transpose(1, 0, 2).copy())
    k = np.concatenate([kp[0], ks]).astype(np.float64)
    v = np.concatenate([vp[0], vs]).astype(np.float64)
    kt = torch.from_numpy(k)[None].expand(h, -1, -1)
    vt = torch.from_numpy(v)[None].expand(h, -1, -1)
    am = torch.from_numpy(np.concatenate([mask, np.zeros(ks.shape[0], np.float32)]).astype(np.float64))
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=am, scale=1.0)
    out = out.permute(1, 0, 2).reshape(tq, h * hd).numpy()
    np.testing.assert_allclose(out, fx["out_f64"], rtol=1e-6, atol=1e-9)


def test_q4_kat_fixture():
    fx = _load("q4_kat.npz")
    w = G.q4_weight()
    np.testing.assert_array_equal(w.view(np.uint16), fx["w"].view(np.uint16))
    qw, qs = Q.quantize(w)
    np.testing.assert_array_equal(qw, fx["q_weight"])
    np.testing.assert_array_equal(qs.view(np.uint16), fx["q_scale"].view(np.uint16))
    with np.errstate(over="ignore"):
        deq = Q.dequantize(qw, qs)
    np.testing.assert_array_equal(deq.view(np.uint16), fx["deq_bits"])
    # the hand-derived words of the tie row and the zero group
    assert int(fx["q_weight"][0, 0]) == 0x97884A0E
    assert [int(x) for x in fx["q_weight"][1, :4]] == [0x77777777] * 4
    assert float(fx["q_scale"][1, 0]) == 0.0
