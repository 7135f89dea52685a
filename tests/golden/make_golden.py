"""Writes the golden fixtures of this directory from the oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path (its tests pin relative
invariants only: python/tests/test_numerical_gates.py:15-27,
test_pizero_runner.py:63-75), so these fixtures are produced by the oracle, whose
functions are pinned independently by tests/test_oracle_*.py.  They freeze the
oracle's outputs on the seeded workloads and give the GPU tests fixed targets.

Fixtures (all seeded; parameters are regenerated from their seed and checked by
per-tensor checksums instead of being stored):

tiny_e2e.npz
    The 2-layer CPU-sized model in float32 (prefix expert width 256 / MLP 1024,
    action expert 128 / 512, 2 query heads, 1 kv head, head_dim 64, prefix 32,
    horizon 8, action_dim 32).  Weights 0.02*N(0,1) from default_rng(0) in
    named_params order (python/tests/conftest.py:47-63), prefix_embs N(0,1) from
    default_rng(1), noise from default_rng(0) (sample.py:132-137).  Holds the
    prefill K/V, v at t=1 (denoise_step_kv), the 10-step host Euler actions
    (sample) and the in-graph loop actions (sample_graph), in float32 and float64.
attn_isolated.npz
    Joint attention at the pi0.5 head shape (8 query heads, 1 kv head, head_dim
    256, 50 queries, 50 suffix keys) with the prefix cut to 96 keys of which 72
    are valid.  Inputs N(0,1)/16 in fp16 from default_rng(2), regenerated and
    checked by checksums; output in float64 truth (stored as float32).
q4_kat.npz
    q4f16_1 known answers (quant.py:217-266, 65-86, 176-193) on a 16x128 weight
    with half-even ties, zero groups, all-negative groups, subnormal values and a
    group at the fp16 maximum (its dequantized extreme, 7 * 9360, rounds to inf
    in fp16 arithmetic): q_weight, q_scale and the dequantized bits.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import pi0_oracle as O  # noqa: E402
from oracle import q4_oracle as Q  # noqa: E402

TINY_DIMS = O.Dims(vlm_width=256, vlm_mlp=1024, ae_width=128, ae_mlp=512, depth=2, num_heads=2,
                   num_kv_heads=1, head_dim=64, prefix_len=32, suffix_len=8, action_dim=32, num_steps=10)

ATTN = dict(tq=50, h=8, kv=1, hd=256, sp=96, valid=72, ts=50, seed=2)


def checksums(params, specs):
    s = np.array([np.sum(params[n].astype(np.float64)) for n, _ in specs])
    ss = np.array([np.sum(np.square(params[n].astype(np.float64))) for n, _ in specs])
    return s, ss


def tiny_inputs(d: O.Dims = TINY_DIMS):
    specs = O.param_specs(d)
    params = O.make_params(specs, 0, "float32")
    prefix = np.random.default_rng(1).standard_normal((1, d.prefix_len, d.vlm_width)).astype(np.float32)
    noise = np.random.default_rng(0).standard_normal((1, d.suffix_len, d.action_dim)).astype(np.float32)
    return specs, params, prefix, noise


def tiny_outputs(params, prefix, noise, mode: str, d: O.Dims = TINY_DIMS):
    P = O.Prec(mode)
    pmask = O.make_prefix_mask_np(d.prefix_len)
    keys, values = O.prefill(params, d, P.cast(prefix), pmask, P)
    cos, sin = O.make_rope_np(d.suffix_len, d.head_dim, d.theta, offset=d.prefix_len)
    te1 = O.sinusoidal_time_emb(1.0, d.ae_width)
    v1 = O.denoise_step_kv(params, d, keys, values, P.cast(noise), P.cast(te1), cos, sin, pmask, P)
    actions = O.sample(params, d, prefix, noise, P, num_steps=d.num_steps)
    actions_graph = O.sample(params, d, prefix, noise, P, graph=True)
    return dict(keys=keys, values=values, v1=v1, actions=actions, actions_graph=actions_graph)


def attn_inputs(tq, h, kv, hd, sp, valid, ts, seed):
    rng = np.random.default_rng(seed)
    s = 1.0 / np.sqrt(hd)
    q = (rng.standard_normal((tq, h * hd)) * s).astype(np.float16)
    kp = (rng.standard_normal((kv, sp, hd)) * s).astype(np.float16)
    vp = (rng.standard_normal((kv, sp, hd)) * s).astype(np.float16)
    ks = (rng.standard_normal((ts, kv * hd)) * s).astype(np.float16)
    vs = (rng.standard_normal((ts, kv * hd)) * s).astype(np.float16)
    mask = np.where(np.arange(sp) < valid, 0.0, -1e9).astype(np.float32)
    return q, kp, vp, ks, vs, mask


def attn_reference(q, kp, vp, ks, vs, mask, mode: str):
    """The oracle's joint attention: prefix keys then suffix keys, mask || zeros."""
    tq = q.shape[0]
    kv, sp, hd = kp.shape
    ts = ks.shape[0]
    h = q.shape[1] // hd
    P = O.Prec(mode)
    acc = np.float64 if mode == "f64" else np.float32
    qo = q.astype(acc).reshape(tq, h, hd)
    ko = np.concatenate([kp.astype(acc).transpose(1, 0, 2), ks.astype(acc).reshape(ts, kv, hd)], 0)
    vdt = np.float64 if mode == "f64" else np.float16
    vo = np.concatenate([vp.transpose(1, 0, 2), vs.reshape(ts, kv, hd)], 0).astype(vdt)
    full = np.concatenate([mask, np.zeros(ts, np.float32)]).astype(acc)
    return O.sdpa(qo, ko, vo, full, P)


def q4_weight():
    rng = np.random.default_rng(4)
    w = (0.02 * rng.standard_normal((16, 128))).astype(np.float16)
    w[0, :8] = [0.7, -0.7, 0.35, -0.35, 0.1, 0.05, 0.0, 0.2]   # half-even ties
    w[1, :32] = 0.0                                            # zero group
    w[2, 32:64] = -np.abs(w[2, 32:64])                         # all-negative group
    w[3, 64:96] = np.float16(2.0 ** -20) * np.arange(32)       # subnormal group
    w[4, 96:128] = np.float16(65504.0) * np.sign(w[4, 96:128])  # fp16 max magnitude
    return w


def main():
    specs, params, prefix, noise = tiny_inputs()
    s, ss = checksums(params, specs)
    out32 = tiny_outputs(params, prefix, noise, "f32")
    out64 = tiny_outputs(params, prefix, noise, "f64")
    np.savez_compressed(
        os.path.join(HERE, "tiny_e2e.npz"), param_sum=s, param_sumsq=ss, prefix_embs=prefix, noise=noise,
        **{k: v.astype(np.float32) for k, v in out32.items()},
        **{k + "_f64": v.astype(np.float64) for k, v in out64.items() if k in ("v1", "actions", "actions_graph")})

    q, kp, vp, ks, vs, mask = attn_inputs(**ATTN)
    ref64 = attn_reference(q, kp, vp, ks, vs, mask, "f64")
    np.savez_compressed(
        os.path.join(HERE, "attn_isolated.npz"),
        input_sums=np.array([np.sum(a.astype(np.float64)) for a in (q, kp, vp, ks, vs)]),
        out_f64=ref64.astype(np.float32), mask=mask)

    w = q4_weight()
    qw, qs = Q.quantize(w)
    deq = Q.dequantize(qw, qs)
    np.savez_compressed(os.path.join(HERE, "q4_kat.npz"), w=w, q_weight=qw, q_scale=qs, deq_bits=deq.view(np.uint16))
    for f in ("tiny_e2e.npz", "attn_isolated.npz", "q4_kat.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
