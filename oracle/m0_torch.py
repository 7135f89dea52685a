"""Independent torch-fp64 restatement of the M0 joint forward (oracle; test infrastructure only).

Second, differently-written restatement of the dual-expert joint step, used to pin
the numpy M1 oracle (``pi0_oracle``) through the reference's own core gate
M1 == M0 (python/mlc_vla/compare_kv.py:39-116).  It follows the structure of the
reference's self-contained torch reference (python/mlc_vla/openpi_ref.py:92-214):
HF-style rotate_half RoPE over full-width cos/sin tables, rsqrt RMSNorm via
``torch.nn.functional.rms_norm``, logits scaled after the QK^T product, kv heads
repeated with ``repeat_interleave``, and the joint block mask built from
(query, key) block ids.  Everything runs in float64.

Reference: Pi0Model.denoise_step (model/pi0/pi0_model.py:111-125),
DualExpertAttention.forward (gemma_dual.py:162-233), DualExpertBlock.forward
(:293-331), DualExpertGemma.forward (:373-390).
"""

from __future__ import annotations

from typing import Dict

import numpy as np
import torch
import torch.nn.functional as F  # noqa: N812

from .pi0_oracle import Dims

_F64 = torch.float64


def _t(a) -> torch.Tensor:
    return torch.as_tensor(np.asarray(a, dtype=np.float64), dtype=_F64)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _rope_full(total: int, hd: int, theta: float):
    inv_freq = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=_F64) / hd))
    freqs = torch.outer(torch.arange(total, dtype=_F64), inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)  # [total, hd]
    return emb.cos(), emb.sin()


def _norm(x: torch.Tensor, eps: float) -> torch.Tensor:
    return F.rms_norm(x, (x.shape[-1],), weight=None, eps=eps)


def denoise_step_m0(params: Dict[str, np.ndarray], d: Dims, prefix_embs, x_t, time_emb) -> np.ndarray:
    """Joint prefix+suffix velocity, float64, returns [1, T, A] (pi0_model.py:111-125)."""
    W = {k: _t(v) for k, v in params.items()}
    n, kv, hd = d.num_heads, d.num_kv_heads, d.head_dim
    P, T = d.prefix_len, d.suffix_len
    total = P + T
    prefix = _t(prefix_embs).reshape(P, d.vlm_width)
    suffix = F.linear(_t(x_t).reshape(T, d.action_dim), W["action_in_proj.weight"], W["action_in_proj.bias"])
    tc = F.silu(F.linear(_t(time_emb).reshape(1, -1), W["time_mlp_in.weight"], W["time_mlp_in.bias"]))
    cond = F.silu(F.linear(tc, W["time_mlp_out.weight"], W["time_mlp_out.bias"]))  # [1, W1]

    cos, sin = _rope_full(total, hd, d.theta)
    blk = (torch.arange(total) >= P).long()
    allowed = blk[None, :] <= blk[:, None]          # query i may see key j
    mask = torch.where(allowed, 0.0, d.neg_inf).to(_F64)

    def norm(x, name, e):
        if e == 0:
            return _norm(x, d.eps) * (1.0 + W[name + ".0.weight"]), None
        mod = F.linear(cond, W[name + ".1.modulation.weight"], W[name + ".1.modulation.bias"])
        scale, shift, gate = torch.chunk(mod, 3, dim=-1)
        return _norm(x, d.eps) * (1.0 + scale) + shift, gate

    hs = [prefix, suffix]
    for L in range(d.depth):
        p = f"backbone.layers.{L}."
        qs, ks, vs, gates = [], [], [], []
        for e in range(2):
            xn, g = norm(hs[e], p + "input_layernorm", e)
            gates.append(g)
            a = f"{p}self_attn.experts.{e}."
            t = xn.shape[0]
            qs.append(F.linear(xn, W[a + "q_proj.weight"]).view(t, n, hd).transpose(0, 1))
            ks.append(F.linear(xn, W[a + "k_proj.weight"]).view(t, kv, hd).transpose(0, 1))
            vs.append(F.linear(xn, W[a + "v_proj.weight"]).view(t, kv, hd).transpose(0, 1))
        q = torch.cat(qs, dim=1)
        k = torch.cat(ks, dim=1)
        v = torch.cat(vs, dim=1)
        q = q * cos + _rotate_half(q) * sin
        k = k * cos + _rotate_half(k) * sin
        if kv != n:
            k = k.repeat_interleave(n // kv, dim=0)
            v = v.repeat_interleave(n // kv, dim=0)
        logits = torch.matmul(q, k.transpose(1, 2)) * (hd ** -0.5) + mask
        ctx = torch.matmul(torch.softmax(logits, dim=-1), v)          # [n, total, hd]
        ctx = ctx.transpose(0, 1).reshape(total, n * hd)
        new_hs = []
        start = 0
        for e in range(2):
            t = hs[e].shape[0]
            seg = ctx[start:start + t]
            start += t
            a = f"{p}self_attn.experts.{e}."
            o = F.linear(seg, W[a + "o_proj.weight"])
            x1 = hs[e] + (o if gates[e] is None else o * gates[e])
            xn2, g2 = norm(x1, p + "post_attention_layernorm", e)
            gu = F.linear(xn2, W[f"{p}mlp.{e}.gate_up_proj.weight"])
            gate, up = torch.chunk(gu, 2, dim=-1)
            m = F.linear(F.gelu(gate, approximate="tanh") * up, W[f"{p}mlp.{e}.down_proj.weight"])
            new_hs.append(x1 + (m if g2 is None else m * g2))
        hs = new_hs
    out, _ = norm(hs[1], "backbone.final_norm", 1)
    vel = F.linear(out, W["action_out_proj.weight"], W["action_out_proj.bias"])
    return vel.reshape(1, T, d.action_dim).numpy()
