"""Kernel-level parity on the GPU, through the C ABI: q4f16_1 quantize / dequantize
bit-exact, the skinny GEMM (fp16 and q4 weights) and the joint attention against
the oracle."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import cosine, max_abs
from gates import kernel_gate
from mlc_vla import _native as N
from mlc_vla.sample import make_prefix_mask_np, make_rope_np
from oracle import pi0_oracle as O
from oracle import q4_oracle as Q

pytestmark = pytest.mark.gpu


def _st():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def _p(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr())


def _host(t: torch.Tensor, dtype=None) -> np.ndarray:
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    return a.view(dtype) if dtype is not None else a


def _ulp16(x: np.ndarray) -> np.ndarray:
    x = np.abs(np.asarray(x, np.float16))
    return (np.nextafter(x, np.float16(np.inf)) - x).astype(np.float64)


@pytest.mark.parametrize("n,k", [(1, 32), (256, 1024), (1024, 4096), (50, 96)])
def test_q4_quantize_bitexact(n, k):
    print(f"q4 quantize N={n} K={k}", flush=True)
    rng = np.random.default_rng(n + k)
    w = (0.02 * rng.standard_normal((n, k))).astype(np.float16)
    w[0, :8] = [0.7, -0.7, 0.35, -0.35, 0.1, 0.05, 0.0, 0.2]  # half-even ties (known answer)
    if n > 1:
        w[1, :32] = 0.0  # zero group
    qw_ref, qs_ref = Q.quantize(w)
    wd = _dev(w)
    qw = torch.zeros((n, k // 8), dtype=torch.int32, device="cuda")
    qs = torch.zeros((n, k // 32), dtype=torch.float16, device="cuda")
    N.call("mlcv_q4_quantize", _p(wd), _p(qw), _p(qs), n, k, _st())
    np.testing.assert_array_equal(_host(qw, np.uint32), qw_ref)
    np.testing.assert_array_equal(_host(qs).view(np.uint16), qs_ref.view(np.uint16))


@pytest.mark.parametrize("n,k", [(7, 32), (3072, 1024), (64, 4096)])
def test_q4_dequant_bitexact(n, k):
    print(f"q4 dequant N={n} K={k}", flush=True)
    rng = np.random.default_rng(k)
    qw = rng.integers(0, 2 ** 32, size=(n, k // 8), dtype=np.uint64).astype(np.uint32)  # every nibble 0..15
    qs = ((rng.random((n, k // 32)) + 0.01) * 0.02).astype(np.float16)
    out = torch.empty((n, k), dtype=torch.float16, device="cuda")
    qwd, qsd = _dev(qw), _dev(qs)
    N.call("mlcv_q4_dequantize", _p(qwd), _p(qsd), _p(out), n, k, _st())
    np.testing.assert_array_equal(_host(out).view(np.uint16), Q.dequantize(qw, qs).view(np.uint16))


# (M, K, N, epilogue): the pi0.5 prefill GEMMs at P = 968 (q/k/v, o_proj + residual, gate_up
# + GeGLU, down + residual), then ragged shapes (M and N tails, short K)
TILE_SHAPES = [(968, 2048, 2560, 0), (968, 2048, 2048, 1), (968, 2048, 16384, 2), (968, 16384, 2048, 1),
               (37, 192, 100, 0), (300, 1024, 260, 1), (300, 512, 384, 2), (1000, 4096, 512, 1), (5, 64, 128, 2),
               # K not a multiple of 64 (SigLIP fc2 and patch embedding, a ragged case)
               (256, 4304, 1152, 1), (256, 592, 1152, 0), (77, 200, 260, 1), (300, 136, 256, 2),
               # enough 256 x 64 tiles for the whole-K narrow plan, with N and K tails
               (4096, 1024, 1156, 0), (2000, 200, 1028, 1),
               # 128 x 64 tiles (128 x 128 ones would fill half the CUs), with N and K tails
               (1000, 1000, 2040, 0),
               # K >= 8192 with more 256 x 256 tiles (264) than the split workspace and meeting
               # counters hold (one per CU): planned on 256 x 128 tiles over the whole K
               (2048, 8192, 8448, 1)]


@pytest.mark.parametrize("m,k,n,epi", TILE_SHAPES)
@pytest.mark.parametrize("small", [0, 1], ids=["tile256", "tile128"])
def test_tile_linear_vs_exact(m, k, n, epi, small):
    """The prefill GEMM: exact fp16 products accumulated in fp32, one fp16 rounding (then the
    residual add, or gelu_tanh(gate) * up, in fp16), against the float64 product on the
    GPU.  The fp32 accumulation error is bounded by 8 eps32 sqrt(K) ||x_m * w_n||_2."""
    print(f"tile linear M={m} K={k} N={n} epi={epi} small={small}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(m * 31 + k + n + epi)
    rows = 2 * n if epi == 2 else n
    x = torch.randn((m, k), generator=g, device="cuda").half()
    w = (torch.randn((rows, k), generator=g, device="cuda") / k ** 0.5).half()
    y0 = torch.randn((m, n), generator=g, device="cuda").half()
    y = y0.clone() if epi == 1 else torch.empty((m, n), dtype=torch.float16, device="cuda")
    N.call("mlcv_tile_linear", _p(x), m, k, _p(w), n, _p(y), epi, small, -1, _st())
    exact = x.double() @ w.double().T
    slack = 8 * 2.0 ** -24 * k ** 0.5 * ((x.double() ** 2) @ (w.double() ** 2).T).sqrt()
    got = y.double()
    ulp = lambda t: torch.from_numpy(_ulp16(t.cpu().numpy())).cuda()  # noqa: E731
    if epi == 2:
        gate, up = exact[:, :n], exact[:, n:]
        g16, u16 = gate.half(), up.half()
        gl = torch.from_numpy(O.gelu_tanh(g16.float().cpu().numpy())).cuda().half()
        ref = (gl.double() * u16.double()).half().double()
        # one ulp of gate / up from the accumulation moves the result by about one ulp of
        # each factor's share, plus the two fp16 roundings
        bound = 2 * ulp(ref) + 2 * ulp(gl.double()) * up.abs() + 2 * ulp(g16.double()) * up.abs() * 1.2 + \
            gl.double().abs() * (ulp(u16.double()) + slack[:, n:]) + up.abs() * 1.2 * slack[:, :n]
        err = (got - ref).abs()
    else:
        pre16 = exact.half().double()
        target = exact + (y0.double() if epi == 1 else 0.0)
        bound = 0.5 * ulp(pre16) + slack + (0.5 * ulp(got) if epi == 1 else 0.0) + 0.5 * ulp(pre16)
        err = (got - target).abs()
    assert torch.isfinite(got).all()
    assert bool((err <= bound).all()), float((err / bound).max())
    assert cosine(got.cpu().numpy(), (ref if epi == 2 else target).cpu().numpy()) > 0.99999


@pytest.mark.parametrize("vocab,width,n", [(1000, 2048, 77), (300, 256, 32), (50, 100, 9)])
def test_embed_language_bitexact(vocab, width, n):
    """embed_language rows (16-byte and scalar paths) against the oracle, bit-exact; ids
    outside the table are clamped to its ends."""
    print(f"embed_language vocab={vocab} width={width} n={n}", flush=True)
    rng = np.random.default_rng(vocab + width)
    table = (rng.standard_normal((vocab, width)) * 3).astype(np.float16)
    ids = rng.integers(0, vocab, size=n).astype(np.int32)
    ids[0], ids[-1] = -5, vocab + 7
    out = torch.empty((n, width), dtype=torch.float16, device="cuda")
    idsd, tabd = _dev(ids), _dev(table)  # alive until the kernel has run
    N.call("mlcv_embed_language", _p(idsd), n, _p(tabd), vocab, width, _p(out), _st())
    ref = O.embed_language(table, np.clip(ids, 0, vocab - 1))
    np.testing.assert_array_equal(_host(out).view(np.uint16), ref.view(np.uint16))


# (M, K, N): the step's modulation, q/k/v, o_proj, down and gate_up shapes, the time MLP, action_in and
# action_out, then ragged shapes
LIN_SHAPES = [(1, 1024, 3072), (50, 1024, 2560), (50, 2048, 1024), (50, 4096, 1024), (50, 1024, 8192), (1, 1024, 1024),
              (50, 32, 1024), (8, 32, 128), (50, 1024, 32), (100, 256, 64), (4, 64, 16)]


@pytest.mark.parametrize("m,k,n", LIN_SHAPES)
@pytest.mark.parametrize("q4", [False, True], ids=["f16", "q4"])
def test_linear_vs_oracle(m, k, n, q4):
    print(f"linear M={m} K={k} N={n} q4={q4}", flush=True)
    rng = np.random.default_rng(m * 7 + k + n)
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = (0.02 * rng.standard_normal((n, k))).astype(np.float16)
    b = (0.02 * rng.standard_normal(n)).astype(np.float16)
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    xd, bd = _dev(x), _dev(b)
    if q4:
        qw, qs = Q.quantize(w)
        ref = Q.linear_q4(x, qw, qs, b)
        w_eff = Q.dequantize(qw, qs)
        qwd, qsd = _dev(qw), _dev(qs)
        N.call("mlcv_linear", _p(xd), m, k, None, _p(qwd), _p(qsd), _p(bd), _p(y), n, _st())
    else:
        ref = O.linear(x, {"l.weight": w, "l.bias": b}, "l", O.Prec("f16"), bias=True)
        w_eff = w
        wd = _dev(w)
        N.call("mlcv_linear", _p(xd), m, k, _p(wd), None, None, _p(bd), _p(y), n, _st())
    got = _host(y).astype(np.float64)
    # against the exact product: one rounding of the fp32 product to fp16, one of the fp16
    # bias add (half an ulp each), plus fp32 accumulation slack
    exact = x.astype(np.float64) @ w_eff.astype(np.float64).T
    pre16 = exact.astype(np.float16)
    bound = 0.5 * (_ulp16(pre16) + _ulp16(ref)) + 1e-6 * (1.0 + np.abs(exact))
    err = np.abs(got - (exact + b.astype(np.float64)))
    assert np.all(err <= bound + 0.5 * _ulp16(pre16)), float((err / bound).max())
    assert cosine(got, ref) > 0.99999


def _attn_case(tq, h, kv, hd, sp, ts, valid, k_f32, seed):
    rng = np.random.default_rng(seed)
    s = 1.0 / np.sqrt(hd)
    q = (rng.standard_normal((tq, h * hd)) * s).astype(np.float16)
    kp = (rng.standard_normal((kv, sp, hd)) * s).astype(np.float16)
    vp = (rng.standard_normal((kv, sp, hd)) * s).astype(np.float16)
    ks = (rng.standard_normal((ts, kv * hd)) * s).astype(np.float16)
    vs = (rng.standard_normal((ts, kv * hd)) * s).astype(np.float16)
    mask = np.where(np.arange(sp) < valid, 0.0, -1e9).astype(np.float32)
    # oracle in float64 on the same (fp16-representable) values
    qo = q.astype(np.float64).reshape(tq, h, hd)
    ko = np.concatenate([kp.astype(np.float64).transpose(1, 0, 2), ks.astype(np.float64).reshape(ts, kv, hd)], 0)
    vo = np.concatenate([vp.astype(np.float64).transpose(1, 0, 2), vs.astype(np.float64).reshape(ts, kv, hd)], 0)
    full = np.concatenate([mask, np.zeros(ts, np.float32)]).astype(np.float64)
    ref = O.sdpa(qo, ko, vo, full, O.Prec("f64"))
    out = torch.empty((tq, h * hd), dtype=torch.float16, device="cuda")
    qd, vpd = _dev(q), _dev(vp)
    kpd = _dev(kp.astype(np.float32)) if k_f32 else _dev(kp)
    md = _dev(mask)
    ksd, vsd = (_dev(ks), _dev(vs)) if ts else (None, None)
    N.call("mlcv_joint_attention", _p(qd), tq, h, kv, hd, _p(kpd), int(k_f32), _p(vpd), sp, _p(md),
           _p(ksd) if ts else None, _p(vsd) if ts else None, ts, _p(out), _st())
    return _host(out), ref


@pytest.mark.parametrize(
    "tq,h,kv,hd,sp,ts,valid,k_f32",
    [
        (50, 8, 1, 256, 968, 50, 900, True),    # isolated joint attention at the full pi0.5 shape
        (50, 8, 1, 256, 968, 50, 900, False),   # same with an fp16 prefix cache
        (8, 2, 1, 64, 32, 8, 32, True),         # 2-layer CPU-sized model
        (4, 8, 1, 16, 776, 4, 700, True),       # the reference's dummy test model
        (10, 4, 4, 32, 100, 10, 60, True),      # kv heads == q heads
        (37, 2, 1, 128, 300, 0, 250, True),     # no suffix block (prefill form)
        (50, 8, 1, 256, 968, 50, 40, True),     # most of the prefix padded: whole splits masked
    ],
)
def test_joint_attention_vs_oracle(tq, h, kv, hd, sp, ts, valid, k_f32):
    print(f"attention Tq={tq} H={h} KV={kv} hd={hd} Sp={sp} Ts={ts} valid={valid} kf32={k_f32}", flush=True)
    got, ref = _attn_case(tq, h, kv, hd, sp, ts, valid, k_f32, seed=tq + sp + hd)
    assert np.all(np.isfinite(got))
    scale = float(np.abs(ref).max())
    assert max_abs(got, ref) <= 2e-3 * scale + 2e-4, (max_abs(got, ref), scale)
    assert cosine(got, ref) > 0.99999


def test_joint_attention_logits_are_fp32_accurate():
    """Large-magnitude logits from a float32 K cache: the kernel's hi/lo split QK^T
    stays within the error the fp16 probabilities alone allow, while logits from
    fp16-rounded K (a plain fp16 QK^T) exceed that bound."""
    rng = np.random.default_rng(11)
    tq, h, hd, sp = 16, 2, 256, 128
    q = (rng.standard_normal((tq, h * hd)) * 0.3).astype(np.float16)
    kp32 = rng.standard_normal((1, sp, hd)).astype(np.float32) * 6.0  # not fp16-representable
    vp = rng.standard_normal((1, sp, hd)).astype(np.float16)
    q64 = q.astype(np.float64).reshape(tq, h, hd)
    v64 = vp.astype(np.float64).transpose(1, 0, 2)
    k64 = kp32.astype(np.float64).transpose(1, 0, 2)
    ref = O.sdpa(q64, k64, v64, None, O.Prec("f64"))
    # sum_j p_j |v_j|: scale of the error from rounding each probability to fp16
    absref = O.sdpa(q64, k64, np.abs(v64), None, O.Prec("f64"))
    bound = 2 * _ulp16(ref) + 2.0 ** -10 * absref + 1e-6
    out = torch.empty((tq, h * hd), dtype=torch.float16, device="cuda")
    qd, kd, vd = _dev(q), _dev(kp32), _dev(vp)
    N.call("mlcv_joint_attention", _p(qd), tq, h, 1, hd, _p(kd), 1, _p(vd), sp, None, None, None, 0, _p(out), _st())
    got = _host(out)
    diff = np.abs(got.astype(np.float64) - ref)
    assert np.all(diff <= bound), float((diff / bound).max())
    k16 = kp32.astype(np.float16).astype(np.float64).transpose(1, 0, 2)
    ref16 = O.sdpa(q64, k16, v64, None, O.Prec("f64"))
    assert np.any(np.abs(ref16 - ref) > bound)


def test_prefill_attention_device_scope_combine_is_bit_identical(monkeypatch):
    """The head_dim-256 prefill attention combines its key splits in the last split to arrive,
    reading the others from its XCD's L2 when every split ran on the XCD the dispatch order
    places it on, else at device scope.  MLCV_PA_DEV_COMBINE=1 forces the device-scope reads:
    the output is bit-identical (same stored partials, same arithmetic)."""
    P, h, kv, hd, valid = 968, 8, 1, 256, 800
    print("prefill attention: L2 vs device-scope combine", flush=True)
    rng = np.random.default_rng(5)
    nq, nkv = h * hd, kv * hd
    qkv = _dev(rng.standard_normal((P, nq + 2 * nkv)).astype(np.float16))
    keys = _dev(rng.standard_normal((kv, P, hd)).astype(np.float32) * 2.0)
    vals = _dev(rng.standard_normal((kv, P, hd)).astype(np.float16))
    cos, sin = (_dev(a.reshape(P, hd // 2)) for a in make_rope_np(P, hd, 10000.0))
    mask = _dev(make_prefix_mask_np(P, num_valid=valid).reshape(P))
    outs = []
    for dev_combine in ("0", "1"):
        monkeypatch.setenv("MLCV_PA_DEV_COMBINE", dev_combine)
        out = torch.empty((P, nq), dtype=torch.float16, device="cuda")
        N.call("mlcv_prefill_attention", _p(qkv), nq + 2 * nkv, _p(cos), _p(sin), P, h, kv, hd, _p(keys), _p(vals),
               _p(mask), _p(out), _st())
        outs.append(_host(out))
    assert np.all(np.isfinite(outs[0]))
    np.testing.assert_array_equal(outs[0], outs[1])


@pytest.mark.parametrize("form", ["hd256", "general"])
@pytest.mark.parametrize("P,h,kv,hd,valid", [
    (968, 8, 1, 256, 800),   # the pi0.5 prefix: 968 tokens, 800 valid
    (968, 8, 1, 256, 968),   # no padding
    (300, 8, 1, 256, 250),   # partial 128-row blocks and a partial last chunk, 8 key splits
    (200, 2, 2, 256, 37),    # one kv head per q head; a valid chunk boundary mid-split
    (100, 2, 1, 64, 77),     # a small ragged case: partial row blocks and chunks
])
def test_prefill_attention_vs_fp64(P, h, kv, hd, valid, form, monkeypatch):
    """The prefill's attention instantiation (q roped and scaled in the loader, fp32 roped
    keys from the cache, the prefix pad mask, no suffix block) through mlcv_prefill_attention,
    which builds the arguments and split plan the prefill uses, against float64 SDPA
    (gemma_dual.py:236-253,334-341; :97-122).  hd256: the head_dim-256 kernel (chunk images,
    32-row tiles, splits balanced over the valid chunks, in-kernel combine); general: the
    attention every head dim takes (MLCV_PF_ATTN=0)."""
    if form == "general":
        monkeypatch.setenv("MLCV_PF_ATTN", "0")
    elif hd != 256:
        pytest.skip("the hd256 form is for head_dim 256")
    print(f"prefill attention {form} P={P} H={h} KV={kv} hd={hd} valid={valid}", flush=True)
    rng = np.random.default_rng(P + valid + hd)
    nq, nkv = h * hd, kv * hd
    qkv = rng.standard_normal((P, nq + 2 * nkv)).astype(np.float16)  # the q/k/v GEMM output row layout
    keys = rng.standard_normal((kv, P, hd)).astype(np.float32) * 2.0
    vals = rng.standard_normal((kv, P, hd)).astype(np.float16)
    cos, sin = (a.reshape(P, hd // 2) for a in make_rope_np(P, hd, 10000.0))
    mask = make_prefix_mask_np(P, num_valid=valid).reshape(P)
    out = torch.empty((P, nq), dtype=torch.float16, device="cuda")
    qd, cd, sd, kd, vd, md = _dev(qkv), _dev(cos), _dev(sin), _dev(keys), _dev(vals), _dev(mask)
    N.call("mlcv_prefill_attention", _p(qd), nq + 2 * nkv, _p(cd), _p(sd), P, h, kv, hd, _p(kd), _p(vd), _p(md),
           _p(out), _st())
    got = _host(out)
    F64 = O.Prec("f64")
    q = O.apply_rope(qkv[:, :nq].astype(np.float64).reshape(P, h, hd), cos, sin, F64) * hd ** -0.5
    ref = O.sdpa(q, keys.astype(np.float64).transpose(1, 0, 2), vals.astype(np.float64).transpose(1, 0, 2),
                 mask.astype(np.float64), F64)
    assert np.all(np.isfinite(got))
    ok, st = kernel_gate(got, ref)
    print("prefill attention", st, flush=True)
    assert ok, st
