"""Pins the q4f16_1 oracle (oracle/q4_oracle.py): hand-computed known answers,
range/extreme-value properties, an element-by-element pure-Python restatement of
the packing, exact dequantization in float64, and the quantized name contract."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import pi0_oracle as O
from oracle import q4_oracle as Q


def test_known_answer_one_group():
    # fp16(0.7) = 0.70019531; s = fp16(0.70019531 / 7) = fp16(0.10002790) = 0.10003662 (1639 * 2^-14)
    #  0.7  : fp16(0.70019531/s)=7.0        +7 -> 14
    # -0.7  : -7.0 + 7                         -> 0
    #  0.35 : fp16(0.35009766/s)=3.5 ; 10.5 tie -> 10 (half to even)
    # -0.35 : -3.5 + 7 = 3.5 tie               -> 4
    #  0.1  : fp16(0.99939)=0.99951; fp16(7.99951)=8.0 -> 8
    #  0.05 : fp16(0.49969)=0.49976; fp16(7.49976)=7.5 tie -> 8
    #  0.0  : 7 ;  0.2 : fp16(1.99877)=1.99902; fp16(8.99902)=9.0 -> 9
    w = np.zeros((1, 32), np.float16)
    w[0, :8] = [0.7, -0.7, 0.35, -0.35, 0.1, 0.05, 0.0, 0.2]
    qw, qs = Q.quantize(w)
    assert qs.dtype == np.float16 and qs.shape == (1, 1)
    assert qs[0, 0] == np.float16(1639 * 2.0 ** -14)
    assert qw.dtype == np.uint32 and qw.shape == (1, 4)
    assert int(qw[0, 0]) == 0x97884A0E
    assert [int(x) for x in qw[0, 1:]] == [0x77777777] * 3
    deq = Q.dequantize(qw, qs)
    assert deq[0, 0] == np.float16(7 * 1639 * 2.0 ** -14)
    assert deq[0, 6] == 0.0


def test_range_extremes_and_error_bound():
    rng = np.random.default_rng(0)
    w = (0.02 * rng.standard_normal((64, 256))).astype(np.float16)
    qw, qs = Q.quantize(w)
    nib = Q.unpack_nibbles(qw, 256).reshape(64, 8, 32)
    assert nib.max() <= 14
    wg = w.astype(np.float64).reshape(64, 8, 32)
    arg = np.abs(wg).argmax(axis=-1)
    ext = np.take_along_axis(nib, arg[..., None], axis=-1)[..., 0]
    assert np.all((ext == 0) | (ext == 14))
    deq = Q.dequantize(qw, qs).astype(np.float64).reshape(64, 8, 32)
    s = qs.astype(np.float64)[..., None]
    assert np.all(np.abs(deq - wg) <= 0.5 * s * 1.01 + 1e-3 * np.abs(wg) + 1e-7)


def test_pack_unpack_bit_by_bit():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 15, size=(3, 40)).astype(np.uint32)
    packed = Q.pack(q)
    assert packed.shape == (3, 5)
    for n in range(3):
        for j in range(5):
            word = 0
            for r in range(8):
                word |= int(q[n, 8 * j + r]) << (4 * r)
            assert int(packed[n, j]) == word
    np.testing.assert_array_equal(Q.unpack_nibbles(packed, 40), q.astype(np.uint8))


def test_dequant_is_one_rounding_of_exact_product():
    rng = np.random.default_rng(2)
    qw = rng.integers(0, 2 ** 32, size=(8, 16), dtype=np.uint64).astype(np.uint32)
    qs = (0.01 * rng.random((8, 4)) + 1e-4).astype(np.float16)
    deq = Q.dequantize(qw, qs)
    for n in range(8):
        for k in range(128):
            nib = (int(qw[n, k // 8]) >> (4 * (k % 8))) & 0xF
            exact = (nib - 7) * float(qs[n, k // 32])  # exact in float64
            assert deq[n, k] == np.float16(exact)


def test_linear_q4_equals_linear_on_dequantized():
    rng = np.random.default_rng(3)
    w = (0.02 * rng.standard_normal((48, 64))).astype(np.float16)
    b = (0.02 * rng.standard_normal(48)).astype(np.float16)
    x = rng.standard_normal((5, 64)).astype(np.float16)
    qw, qs = Q.quantize(w)
    params = {"lin.q_weight": qw, "lin.q_scale": qs, "lin.bias": b}
    got = O.linear(x, params, "lin", O.Prec("f16"), bias=True)
    ref = Q.linear_q4(x, qw, qs, b)
    np.testing.assert_array_equal(got, ref)


def test_zero_group_dequantizes_to_zero():
    w = np.zeros((2, 64), np.float16)
    w[1, 32:] = 0.5
    qw, qs = Q.quantize(w)
    assert qs[0, 0] == 0 and qs[1, 0] == 0
    assert np.all(Q.dequantize(qw, qs)[:, :32] == 0)


def test_quantized_specs_contract():
    d = O.Dims(vlm_width=64, vlm_mlp=128, ae_width=64, ae_mlp=128, depth=2, num_heads=8, num_kv_heads=1,
               head_dim=16, prefix_len=8, suffix_len=4, action_dim=32)
    qs = Q.quantized_specs(O.param_specs(d))
    names = [n for n, _, _ in qs]
    lin = [n for n, s in O.param_specs(d) if n.endswith(".weight") and len(s) == 2]
    assert len(qs) == len(O.param_specs(d)) + len(lin)
    i = names.index("time_mlp_in.q_weight")
    assert names[i + 1] == "time_mlp_in.q_scale" and names[i + 2] == "time_mlp_in.bias"
    spec = {n: (s, t) for n, s, t in qs}
    assert spec["backbone.layers.1.mlp.1.down_proj.q_weight"] == ((64, 16), "uint32")
    assert spec["backbone.layers.1.mlp.1.down_proj.q_scale"] == ((64, 4), "float16")
    assert spec["backbone.final_norm.0.weight"] == ((64,), "float16")


@pytest.mark.parametrize("k", [32, 96])
def test_quantize_roundtrip_idempotent(k):
    """Quantizing a dequantized matrix reproduces the same codes and scales."""
    rng = np.random.default_rng(k)
    w = (0.05 * rng.standard_normal((16, k))).astype(np.float16)
    qw, qs = Q.quantize(w)
    qw2, qs2 = Q.quantize(Q.dequantize(qw, qs))
    np.testing.assert_array_equal(qs, qs2)
    np.testing.assert_array_equal(qw, qw2)
