"""numpy restatement of mlc-vla's M1 denoise path (oracle; test infrastructure only).

Nothing in the product imports this module.  It is the checker for the HIP path
and the timed CPU baseline of ``bench.py``.

Reference functions restated here (paths relative to the reference repository):

==========================  ==============================================  =====================================
oracle function             reference                                       pinned by (tests/test_oracle_*.py)
==========================  ==============================================  =====================================
sinusoidal_time_emb         python/mlc_vla/openpi_ref.py:49-58              closed form (t=0 -> sin 0 / cos 1),
                                                                            log-space period recomputation
make_time_embs              python/mlc_vla/sample.py:27-35                  t grid equals 1, 0.9, ... (floats)
make_rope_np                python/mlc_vla/sample.py:38-47,                 norm preservation, relative-position
                            model/pi0/gemma_dual.py:24-44                   invariance, HF rotate_half form
make_prefix_mask_np         python/mlc_vla/sample.py:50-64                  brute-force enumeration
euler_loop                  python/mlc_vla/sample.py:67-74                  closed form for constant velocity
build_additive_mask         model/pi0/pi0_model.py:29-41                    brute-force block-causal rule
apply_rope                  model/pi0/gemma_dual.py:47-57                   torch rotate_half restatement (M0)
rms_norm / ada_rms_norm     model/pi0/gemma_dual.py:60-88                   torch.nn.functional.rms_norm (fp64)
gated_residual              model/pi0/gemma_dual.py:91-94                   M1==M0
sdpa                        model/pi0/gemma_dual.py:97-122                  torch scaled_dot_product_attention
gelu_tanh / mlp             model/pi0/gemma_dual.py:125-135                 torch F.gelu(approximate="tanh")
time_cond                   model/pi0/pi0_model.py:106-109                  torch F.silu / F.linear (M0)
prefill                     model/pi0/pi0_model.py:128-140,                 M1==M0 (torch fp64 joint forward),
                            gemma_dual.py:236-253,334-341,398-415           pad invariance
denoise_step_kv             model/pi0/pi0_model.py:142-163,                 M1==M0, pad invariance
                            gemma_dual.py:255-275,343-351,417-433
denoise_loop_kv             model/pi0/pi0_model.py:165-194                  loop == host euler_loop (bit-exact)
embed_language              model/pi0/pi0_model.py:101-104                  float64 product rounded once to fp16
                                                                            (all ids, every vocabulary row); the
                                                                            constant's fp16 dtype is parity unpinned
param_specs                 model/pi0/pi0_model.py:81-88,                   count 18*depth+11, shapes
                            gemma_dual.py:60-73,125-148,281-291,357-371
==========================  ==============================================  =====================================

Precision modes (``Prec``):
  "f64"  truth: every tensor float64 (used for the M1==M0 and library checks)
  "f32"  the reference with ``dtype="float32"`` (what TVM's c/llvm target computes)
  "f16"  the reference's float16 cast points: weights, GEMM outputs, residual stream,
         gates and V in fp16; RoPE, q/k, K cache, logits, softmax, RMSNorm statistics,
         the Euler state and the returned velocity in fp32.  Matmuls accumulate in fp32
         and round once to fp16 (TVM's accumulation order/dtype is parity unpinned).
"""

from __future__ import annotations

import dataclasses
import math
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

# --------------------------------------------------------------------------- #
# dims and parameters
# --------------------------------------------------------------------------- #


@dataclasses.dataclass(frozen=True)
class Dims:
    """Every size the M1 path depends on (pi0_config.py:15-170)."""

    vlm_width: int
    vlm_mlp: int
    ae_width: int
    ae_mlp: int
    depth: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    prefix_len: int
    suffix_len: int
    action_dim: int
    num_steps: int = 10
    eps: float = 1e-6
    theta: float = 10_000.0
    neg_inf: float = -2.3819763e38
    logits_dtype: str = "float32"


def dims_from_config(cfg) -> Dims:
    """Read a reference-shaped ``Pi0Config`` (pi0_config.py:72-170) into ``Dims``."""
    vlm, ae = cfg.vlm, cfg.action_expert
    return Dims(
        vlm_width=vlm.width, vlm_mlp=vlm.mlp_dim, ae_width=ae.width, ae_mlp=ae.mlp_dim,
        depth=vlm.depth, num_heads=vlm.num_heads, num_kv_heads=vlm.num_kv_heads,
        head_dim=vlm.head_dim, prefix_len=cfg.prefix_len, suffix_len=cfg.suffix_len,
        action_dim=cfg.action_dim, num_steps=cfg.num_denoise_steps, eps=cfg.rms_norm_eps,
        theta=cfg.rope_theta, neg_inf=cfg.attn_neg_inf,
        logits_dtype=getattr(cfg, "attn_logits_dtype", "float32"),
    )


def param_specs(d: Dims) -> List[Tuple[str, Tuple[int, ...]]]:
    """(name, shape) of the backbone + action-head parameters in attribute order.

    Follows the module attribute order of pi0_model.py:81-88 and gemma_dual.py:
    DualExpertBlock (:281-291) holds self_attn (experts 0,1: q,k,v,o), mlp (0,1:
    gate_up, down), input_layernorm (0: weight; 1: modulation weight,bias),
    post_attention_layernorm (same); then final_norm (:369-371); then
    action_in_proj, action_out_proj, time_mlp_in, time_mlp_out.  Linear weights are
    [out, in].  The exact TVM ``export_tvm`` order is only confirmable by import
    (parity unpinned); the count (18*depth + 11) and shapes are checked.
    """
    n, kv, hd = d.num_heads, d.num_kv_heads, d.head_dim
    widths = [d.vlm_width, d.ae_width]
    mlps = [d.vlm_mlp, d.ae_mlp]
    specs: List[Tuple[str, Tuple[int, ...]]] = []
    for L in range(d.depth):
        p = f"backbone.layers.{L}."
        for e in range(2):
            w = widths[e]
            specs.append((f"{p}self_attn.experts.{e}.q_proj.weight", (n * hd, w)))
            specs.append((f"{p}self_attn.experts.{e}.k_proj.weight", (kv * hd, w)))
            specs.append((f"{p}self_attn.experts.{e}.v_proj.weight", (kv * hd, w)))
            specs.append((f"{p}self_attn.experts.{e}.o_proj.weight", (w, n * hd)))
        for e in range(2):
            specs.append((f"{p}mlp.{e}.gate_up_proj.weight", (2 * mlps[e], widths[e])))
            specs.append((f"{p}mlp.{e}.down_proj.weight", (widths[e], mlps[e])))
        for ln in ("input_layernorm", "post_attention_layernorm"):
            specs.append((f"{p}{ln}.0.weight", (d.vlm_width,)))
            specs.append((f"{p}{ln}.1.modulation.weight", (3 * d.ae_width, d.ae_width)))
            specs.append((f"{p}{ln}.1.modulation.bias", (3 * d.ae_width,)))
    specs.append(("backbone.final_norm.0.weight", (d.vlm_width,)))
    specs.append(("backbone.final_norm.1.modulation.weight", (3 * d.ae_width, d.ae_width)))
    specs.append(("backbone.final_norm.1.modulation.bias", (3 * d.ae_width,)))
    specs.append(("action_in_proj.weight", (d.ae_width, d.action_dim)))
    specs.append(("action_in_proj.bias", (d.ae_width,)))
    specs.append(("action_out_proj.weight", (d.action_dim, d.ae_width)))
    specs.append(("action_out_proj.bias", (d.action_dim,)))
    specs.append(("time_mlp_in.weight", (d.ae_width, d.ae_width)))
    specs.append(("time_mlp_in.bias", (d.ae_width,)))
    specs.append(("time_mlp_out.weight", (d.ae_width, d.ae_width)))
    specs.append(("time_mlp_out.bias", (d.ae_width,)))
    return specs


def make_params(specs: Sequence[Tuple[str, Tuple[int, ...]]], seed: int = 0,
                dtype="float32", only: Optional[Callable[[str], bool]] = None) -> Dict[str, np.ndarray]:
    """0.02*N(0,1) per parameter in spec order from one ``default_rng(seed)``.

    Recipe of python/tests/conftest.py:47-63 and bench_kv.py:68-72.  ``only``
    keeps a subset of names, but the generator still advances through every spec,
    so the kept arrays equal those of a full draw.
    """
    rng = np.random.default_rng(seed)
    out: Dict[str, np.ndarray] = {}
    for name, shape in specs:
        arr = (0.02 * rng.standard_normal(shape)).astype(dtype)
        if only is None or only(name):
            out[name] = arr
    return out


# --------------------------------------------------------------------------- #
# precision emulation
# --------------------------------------------------------------------------- #


class Prec:
    """Where the reference keeps the model dtype and where it forces float32."""

    def __init__(self, mode: str):
        if mode not in ("f64", "f32", "f16"):
            raise ValueError(mode)
        self.mode = mode
        self.dt = {"f64": np.float64, "f32": np.float32, "f16": np.float16}[mode]
        self.hi = np.float64 if mode == "f64" else np.float32  # the reference's "float32" points
        self.acc = self.hi

    def cast(self, a) -> np.ndarray:
        return np.asarray(a).astype(self.dt)

    def up(self, a) -> np.ndarray:
        return np.asarray(a).astype(self.acc, copy=False)

    def mm(self, a, b) -> np.ndarray:
        """Matmul in the model dtype: operands upcast, accumulate, round once."""
        return self.cast(np.matmul(self.up(a), self.up(b)))


def get_weight(params: Dict[str, np.ndarray], base: str) -> np.ndarray:
    """Linear weight [out,in]; dequantizes q4f16_1 params (quant.py:301-325)."""
    w = params.get(base + ".weight")
    if w is not None:
        return w
    from .q4_oracle import dequantize

    return dequantize(params[base + ".q_weight"], params[base + ".q_scale"])


def linear(x, params, base: str, P: Prec, bias: bool = False) -> np.ndarray:
    """nn.Linear in the model dtype: dt(x @ W^T), then dt(. + b) (quant.py:322-324)."""
    w = get_weight(params, base)
    y = P.mm(x, w.T)
    if bias:
        y = P.cast(P.up(y) + P.up(params[base + ".bias"]))
    return y


# --------------------------------------------------------------------------- #
# host helpers (sample.py, openpi_ref.py)
# --------------------------------------------------------------------------- #


def sinusoidal_time_emb(timestep: float, dim: int, min_period: float = 4e-3,
                        max_period: float = 4.0) -> np.ndarray:
    """[1, dim] f32: [sin(2*pi*t/period), cos(...)], period = min*(max/min)^linspace(0,1,dim/2).

    openpi_ref.py:49-58 (computed in float64, cast to float32).
    """
    if dim % 2 != 0:
        raise ValueError("dim must be even")
    frac = np.linspace(0.0, 1.0, dim // 2, dtype=np.float64)
    period = min_period * (max_period / min_period) ** frac
    arg = (1.0 / period * 2 * math.pi) * float(timestep)
    return np.concatenate([np.sin(arg), np.cos(arg)])[None, :].astype(np.float32)


def make_time_embs(num_steps: int, width: int) -> List[np.ndarray]:
    """Per-step time embeddings for t = 1, 1+dt, ... with Python-float t (sample.py:27-35)."""
    dt = -1.0 / num_steps
    t = 1.0
    out = []
    for _ in range(num_steps):
        out.append(sinusoidal_time_emb(t, width))
        t += dt
    return out


def embed_language(table: np.ndarray, input_ids: np.ndarray) -> np.ndarray:
    """Pi0Model.embed_language (pi0_model.py:101-104): ``embed_tokens(ids) * sqrt(width)``.
    The table is fp16 and the Python float becomes a constant of the tensor's dtype, so the
    result is the fp16 product of two fp16 values (numpy float16 arithmetic rounds it once)."""
    width = table.shape[1]
    scale = np.float16(math.sqrt(width))
    with np.errstate(over="ignore"):  # products past the fp16 range round to inf, as on the GPU
        return (table[np.asarray(input_ids)].astype(np.float16) * scale).astype(np.float16)


def make_rope_np(num_positions: int, head_dim: int, theta: float,
                 offset: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """cos/sin [1, L, 1, hd/2] f32 with radians = pos / theta^((2/hd)*i) in f64 (sample.py:38-47)."""
    half = head_dim // 2
    pos = np.arange(offset, offset + num_positions, dtype=np.float64)
    inv = theta ** ((2.0 / head_dim) * np.arange(half, dtype=np.float64))
    rad = pos[:, None] / inv[None, :]
    shape = (1, num_positions, 1, half)
    return np.cos(rad).reshape(shape).astype(np.float32), np.sin(rad).reshape(shape).astype(np.float32)


def make_prefix_mask_np(prefix_len: int, num_valid: Optional[int] = None,
                        pad_mask=None, neg: float = -1e9) -> np.ndarray:
    """[1,1,1,P] f32 additive mask: 0 valid, ``neg`` padded; pad_mask wins (sample.py:50-64)."""
    if pad_mask is not None:
        valid = np.asarray(pad_mask, dtype=np.float32).reshape(-1)[:prefix_len]
    elif num_valid is not None:
        valid = (np.arange(prefix_len) < int(num_valid)).astype(np.float32)
    else:
        valid = np.ones(prefix_len, np.float32)
    return np.where(valid > 0, np.float32(0.0), np.float32(neg)).astype(np.float32).reshape(1, 1, 1, prefix_len)


def euler_loop(step_fn, x0: np.ndarray, num_steps: int, dtype=np.float32) -> np.ndarray:
    """x <- x + (-1/N) * v in float32, N times (sample.py:67-74).

    ``dtype`` is float32 in the reference; the fp64 truth mode passes float64.
    """
    dt = -1.0 / num_steps
    x = x0.astype(dtype)
    for i in range(num_steps):
        v = step_fn(x, i).astype(dtype)
        x = x + dtype(dt) * v
    return x


def build_additive_mask(prefix_len: int, suffix_len: int, neg_inf: float, dtype) -> np.ndarray:
    """M0 joint mask [1,1,T,T]: prefix block sees prefix; suffix sees everything (pi0_model.py:29-41)."""
    total = prefix_len + suffix_len
    block = (np.arange(total) >= prefix_len).astype(np.int64)  # block id: 0 prefix, 1 suffix
    allow = block[None, :] <= block[:, None]
    with np.errstate(over="ignore"):  # neg_inf -> -inf in float16, as in the reference
        return np.where(allow, 0.0, neg_inf).astype(dtype).reshape(1, 1, total, total)


# --------------------------------------------------------------------------- #
# model pieces (gemma_dual.py)
# --------------------------------------------------------------------------- #


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, P: Prec) -> np.ndarray:
    """x [L, heads, hd]; cos/sin [L, hd/2]: half-split rotation in f32 (gemma_dual.py:47-57)."""
    xf = x.astype(P.hi)
    half = xf.shape[-1] // 2
    x1, x2 = xf[..., :half], xf[..., half:]
    c = cos.astype(P.hi)[:, None, :]
    s = sin.astype(P.hi)[:, None, :]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def _rms_normed(x: np.ndarray, eps: float, P: Prec) -> np.ndarray:
    xf = x.astype(P.hi)
    var = np.sum(xf * xf, axis=-1, keepdims=True) / P.hi(xf.shape[-1])
    return xf / np.sqrt(var + P.hi(eps))


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float, P: Prec) -> np.ndarray:
    """Plain Gemma RMSNorm: normed * (1 + w) cast to the model dtype (gemma_dual.py:75-82)."""
    return P.cast(_rms_normed(x, eps, P) * (1.0 + weight.astype(P.hi)))


def modulation(params, base: str, cond: np.ndarray, P: Prec) -> np.ndarray:
    """adaRMS modulation = cond @ W^T + b in the model dtype, [1, 3W] (gemma_dual.py:84-85)."""
    return linear(cond, params, base + ".modulation", P, bias=True)


def ada_rms_norm(x: np.ndarray, mod: np.ndarray, eps: float, P: Prec) -> Tuple[np.ndarray, np.ndarray]:
    """normed*(1+f32 scale)+f32 shift -> dt; returns (out, gate) (gemma_dual.py:83-88)."""
    w = x.shape[-1]
    scale, shift, gate = mod[..., :w], mod[..., w:2 * w], mod[..., 2 * w:]
    out = _rms_normed(x, eps, P) * (1.0 + scale.astype(P.hi)) + shift.astype(P.hi)
    return P.cast(out), gate


def gated_residual(x: np.ndarray, y: np.ndarray, gate: Optional[np.ndarray], P: Prec) -> np.ndarray:
    """x + y*gate with model-dtype rounding after each op (gemma_dual.py:91-94)."""
    if gate is None:
        return P.cast(P.up(x) + P.up(y))
    return P.cast(P.up(x) + P.up(P.cast(P.up(y) * P.up(gate))))


def softmax(z: np.ndarray) -> np.ndarray:
    m = np.max(z, axis=-1, keepdims=True)
    e = np.exp(z - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def sdpa(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: Optional[np.ndarray], P: Prec,
         logits_dtype: str = "float32") -> np.ndarray:
    """softmax(q k^T + mask) v for kv heads broadcast to q heads (gemma_dual.py:97-122).

    q [Tq, n, hd] (already roped and scaled, f32); k [Ts, kv, hd] f32; v [Ts, kv, hd] dt;
    ``mask`` broadcastable to [n, Tq, Ts].  kv must be 1 or n (``op.broadcast_to``).
    Logits in f32 (inputs cast to ``logits_dtype`` first); probs cast to v's dtype;
    probs @ v in v's dtype.  Returns [Tq, n*hd] in v's dtype.
    """
    tq, n, hd = q.shape
    kv = k.shape[1]
    if kv not in (1, n):
        raise ValueError("kv heads must broadcast to q heads")
    g = n // kv  # head h reads kv head h // g (broadcast_to semantics for kv in {1, n})
    ldt = P.hi if logits_dtype == "float32" or P.mode == "f64" else np.float16
    qh = q.astype(ldt).astype(P.acc).transpose(1, 0, 2)             # [n, Tq, hd]
    enc = np.empty((n, tq, hd), v.dtype)
    for j in range(kv):
        hs = slice(j * g, (j + 1) * g)
        kj = np.ascontiguousarray(k[:, j, :].astype(ldt).astype(P.acc))  # [Ts, hd]
        logits = np.matmul(qh[hs], kj.T).astype(P.hi)                 # [g, Tq, Ts] f32
        if mask is not None:
            logits = logits + mask.astype(P.hi)
        probs = softmax(logits).astype(v.dtype)
        vj = np.ascontiguousarray(v[:, j, :]).astype(P.acc)            # [Ts, hd]
        enc[hs] = np.matmul(probs.astype(P.acc), vj).astype(v.dtype)
    return enc.transpose(1, 0, 2).reshape(tq, n * hd)


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) (op.gelu approximate="tanh")."""
    c = math.sqrt(2.0 / math.pi)
    return 0.5 * x * (1.0 + np.tanh(c * (x + 0.044715 * x * x * x)))


def mlp(x: np.ndarray, params, base: str, P: Prec) -> np.ndarray:
    """down(gelu_tanh(gate) * up) with [gate; up] = gate_up(x) (gemma_dual.py:125-135)."""
    gu = linear(x, params, base + ".gate_up_proj", P)
    m = gu.shape[-1] // 2
    g = P.cast(gelu_tanh(gu[..., :m].astype(P.hi)))
    h = P.cast(P.up(g) * P.up(gu[..., m:]))
    return linear(h, params, base + ".down_proj", P)


def silu(x: np.ndarray, P: Prec) -> np.ndarray:
    xf = x.astype(P.hi)
    return P.cast(xf / (1.0 + np.exp(-xf)))


def time_cond(params, time_emb: np.ndarray, P: Prec) -> np.ndarray:
    """silu(time_mlp_out(silu(time_mlp_in(te)))) in the model dtype (pi0_model.py:106-109)."""
    h = silu(linear(P.cast(time_emb), params, "time_mlp_in", P, bias=True), P)
    return silu(linear(h, params, "time_mlp_out", P, bias=True), P)


# --------------------------------------------------------------------------- #
# M1 exported functions (pi0_model.py)
# --------------------------------------------------------------------------- #


def _heads(x: np.ndarray, heads: int, hd: int) -> np.ndarray:
    return x.reshape(x.shape[0], heads, hd)


def prefill(params, d: Dims, prefix_embs: np.ndarray, prefix_mask: np.ndarray,
            P: Prec) -> Tuple[np.ndarray, np.ndarray]:
    """Expert-0 over the prefix; per-layer post-RoPE K (f32) and V (dt).

    pi0_model.py:128-140 -> gemma_dual.py:398-415 (layers: prefill_e0 :334-341,
    attn_prefill_e0 :236-253).  Positions 0..P-1; ``prefix_mask`` masks padded key
    columns.  Returns keys [depth,1,kv,P,hd] (f32) and values [depth,1,kv,P,hd] (dt).
    The last layer's attention/MLP do not feed any output; they are still computed
    here exactly as the reference does.
    """
    n, kv, hd, plen = d.num_heads, d.num_kv_heads, d.head_dim, d.prefix_len
    x = P.cast(np.asarray(prefix_embs).reshape(plen, d.vlm_width))
    cos, sin = make_rope_np(plen, hd, d.theta, 0)
    cos, sin = cos.reshape(plen, hd // 2), sin.reshape(plen, hd // 2)
    mask = np.asarray(prefix_mask, np.float32).reshape(-1)
    keys = np.zeros((d.depth, 1, kv, plen, hd), P.hi)
    values = np.zeros((d.depth, 1, kv, plen, hd), P.dt)
    scale = P.hi(hd ** -0.5)
    for L in range(d.depth):
        p = f"backbone.layers.{L}."
        a = p + "self_attn.experts.0."
        xn = rms_norm(x, params[p + "input_layernorm.0.weight"], d.eps, P)
        q = apply_rope(_heads(linear(xn, params, a + "q_proj", P), n, hd), cos, sin, P) * scale
        k = apply_rope(_heads(linear(xn, params, a + "k_proj", P), kv, hd), cos, sin, P)
        v = _heads(linear(xn, params, a + "v_proj", P), kv, hd)
        keys[L, 0] = k.transpose(1, 0, 2)
        values[L, 0] = v.transpose(1, 0, 2)
        enc = sdpa(q, k, v, mask, P, d.logits_dtype)
        x = gated_residual(x, linear(enc, params, a + "o_proj", P), None, P)
        xn2 = rms_norm(x, params[p + "post_attention_layernorm.0.weight"], d.eps, P)
        x = gated_residual(x, mlp(xn2, params, p + "mlp.0", P), None, P)
    return keys, values


def all_modulations(params, d: Dims, cond: np.ndarray, P: Prec) -> List[np.ndarray]:
    """The 2*depth+1 adaRMS modulation vectors [1,3W] of one step (they only depend on cond)."""
    mods = []
    for L in range(d.depth):
        p = f"backbone.layers.{L}."
        mods.append(modulation(params, p + "input_layernorm.1", cond, P))
        mods.append(modulation(params, p + "post_attention_layernorm.1", cond, P))
    mods.append(modulation(params, "backbone.final_norm.1", cond, P))
    return mods


def decode_suffix(params, d: Dims, x: np.ndarray, keys: np.ndarray, values: np.ndarray,
                  cos: np.ndarray, sin: np.ndarray, cond: np.ndarray, full_mask: np.ndarray,
                  P: Prec, layer_hook=None) -> np.ndarray:
    """Expert-1 over the suffix against cached prefix K/V (gemma_dual.py:417-433, :343-351, :255-275)."""
    n, kv, hd, t = d.num_heads, d.num_kv_heads, d.head_dim, d.suffix_len
    scale = P.hi(hd ** -0.5)
    mods = all_modulations(params, d, cond, P)
    for L in range(d.depth):
        p = f"backbone.layers.{L}."
        a = p + "self_attn.experts.1."
        xn, gate = ada_rms_norm(x, mods[2 * L], d.eps, P)
        q = apply_rope(_heads(linear(xn, params, a + "q_proj", P), n, hd), cos, sin, P) * scale
        k = apply_rope(_heads(linear(xn, params, a + "k_proj", P), kv, hd), cos, sin, P)
        v = _heads(linear(xn, params, a + "v_proj", P), kv, hd)
        kfull = np.concatenate([np.asarray(keys[L, 0]).transpose(1, 0, 2).astype(P.hi), k], axis=0)
        vfull = np.concatenate([np.asarray(values[L, 0]).transpose(1, 0, 2).astype(P.dt), v], axis=0)
        enc = sdpa(q, kfull, vfull, full_mask, P, d.logits_dtype)
        x = gated_residual(x, linear(enc, params, a + "o_proj", P), gate, P)
        xn2, gate2 = ada_rms_norm(x, mods[2 * L + 1], d.eps, P)
        x = gated_residual(x, mlp(xn2, params, p + "mlp.1", P), gate2, P)
        if layer_hook is not None:
            layer_hook(L, x)
    out, _ = ada_rms_norm(x, mods[-1], d.eps, P)
    return out


def _full_mask(d: Dims, prefix_mask: np.ndarray) -> np.ndarray:
    """prefix pad mask || zeros(T) (pi0_model.py:157-158)."""
    return np.concatenate([np.asarray(prefix_mask, np.float32).reshape(-1),
                           np.zeros(d.suffix_len, np.float32)])


def denoise_step_kv(params, d: Dims, keys, values, x_t, time_emb, suffix_cos, suffix_sin,
                    prefix_mask, P: Prec, layer_hook=None) -> np.ndarray:
    """One suffix-only velocity evaluation; returns v [1,T,A] f32 (pi0_model.py:142-163)."""
    t, hd = d.suffix_len, d.head_dim
    x = linear(P.cast(np.asarray(x_t).reshape(t, d.action_dim)), params, "action_in_proj", P, bias=True)
    cond = time_cond(params, np.asarray(time_emb).reshape(1, d.ae_width), P)
    cos = np.asarray(suffix_cos).reshape(t, hd // 2)
    sin = np.asarray(suffix_sin).reshape(t, hd // 2)
    out = decode_suffix(params, d, x, keys, values, cos, sin, cond, _full_mask(d, prefix_mask), P,
                        layer_hook)
    v = linear(out, params, "action_out_proj", P, bias=True)
    return v.astype(P.hi).reshape(1, t, d.action_dim)


def denoise_loop_kv(params, d: Dims, keys, values, x0, time_embs, suffix_cos, suffix_sin,
                    prefix_mask, P: Prec) -> np.ndarray:
    """N in-graph Euler steps x <- x + (-1/N) f32(v), x fed as dt(x) (pi0_model.py:165-194)."""
    n = d.num_steps
    dt = P.hi(-1.0 / n)
    te = np.asarray(time_embs).reshape(n, d.ae_width)
    x = np.asarray(x0).astype(P.hi).reshape(1, d.suffix_len, d.action_dim)
    for i in range(n):
        v = denoise_step_kv(params, d, keys, values, P.cast(x), te[i:i + 1], suffix_cos,
                            suffix_sin, prefix_mask, P)
        x = x + dt * v
    return x


def sample(params, d: Dims, prefix_embs, noise, P: Prec, num_steps: Optional[int] = None,
           prefix_pad=None, graph: bool = False) -> np.ndarray:
    """PiZeroRunner.sample / sample_graph on the oracle (sample.py:107-187)."""
    n = d.num_steps if num_steps is None or graph else num_steps
    if prefix_pad is None:
        num_valid = d.prefix_len
        pmask = make_prefix_mask_np(d.prefix_len)
    else:
        num_valid = int(np.asarray(prefix_pad).reshape(-1).sum())
        pmask = make_prefix_mask_np(d.prefix_len, pad_mask=prefix_pad)
    cos, sin = make_rope_np(d.suffix_len, d.head_dim, d.theta, offset=num_valid)
    keys, values = prefill(params, d, P.cast(prefix_embs), pmask, P)
    tes = make_time_embs(n, d.ae_width)
    if graph:
        dd = dataclasses.replace(d, num_steps=n)
        return denoise_loop_kv(params, dd, keys, values, noise.astype(np.float32),
                               P.cast(np.concatenate(tes, 0)), cos, sin, pmask, P)

    def step(x_np, i):
        return denoise_step_kv(params, d, keys, values, P.cast(x_np), P.cast(tes[i]), cos, sin,
                               pmask, P)

    return euler_loop(step, noise.astype(np.float32), n, P.hi)
