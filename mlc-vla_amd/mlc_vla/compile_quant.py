"""Quantized build + fp -> q parameter conversion (drop-in for mlc_vla.compile_quant).

Mirrors python/mlc_vla/compile_quant.py:24-103: every Linear weight of the
backbone, the action head and the time MLP becomes ``q_weight`` / ``q_scale``;
biases and RMSNorm weights are cast to the model dtype.  The quantizer itself runs
on the GPU (the reference JIT-compiles it for the CPU).
"""

from __future__ import annotations

import numpy as np

from .compile import _target_kind, check_config
from .model.pi0.pi0_model import BACKBONE_FUNCS, KV_FUNCS, named_params, quantized_named_params
from .quant import QuantizeMapping, get_quant
from .runtime import Executable


def fp_named_params(config, functions):
    """named_params of the unquantized model (compile_quant.py:24-31)."""
    return named_params(config, functions)


def compile_model_quant(config, target: str, functions, quant_name: str, cuda_graph: bool = False, cublas=None,
                        hoist_modulation: bool = True):
    """Return ``(executable, q_named_params, quant_map, quant)`` (compile_quant.py:46-68)."""
    _target_kind(target)
    check_config(config, functions, quant_name)
    quant = get_quant(quant_name)
    if not quant.supported:
        raise NotImplementedError(f"preset {quant_name}: only q4f16_1 is built on gfx950")
    if quant.model_dtype != config.dtype:
        raise ValueError("config.dtype must equal the preset's model dtype")
    funcs = tuple(functions) if functions is not None else KV_FUNCS
    unknown = [f for f in funcs if f not in BACKBONE_FUNCS]
    if unknown:
        raise NotImplementedError(f"functions {unknown}: the q4f16_1 build covers {BACKBONE_FUNCS}")
    qnp = quantized_named_params(config, quant.group_size, quant.num_elem_per_storage, funcs)
    qmap = QuantizeMapping({}, {})
    for name, p in named_params(config, funcs):
        if name.endswith(".weight") and len(p.shape) == 2:
            base = name[: -len(".weight")]
            qmap.param_map[name] = [base + ".q_weight", base + ".q_scale"]
            qmap.map_func[name] = quant.quantize_weight
    return Executable(config, funcs, qnp, quant.name, cuda_graph, hoist_modulation), qnp, qmap, quant


def quantize_params(quant, src_fp: dict, q_named_params, quant_map: QuantizeMapping, device=None) -> dict:
    """fp weights keyed by fp name -> numpy params keyed by quantized name (compile_quant.py:71-103)."""
    rev = {}
    for base, qnames in quant_map.param_map.items():
        for i, qn in enumerate(qnames):
            rev[qn] = (base, i)
    cache = {}
    out = {}
    for name, p in q_named_params:
        if name in rev:
            base, idx = rev[name]
            if base not in cache:
                res = quant_map.map_func[base](np.asarray(src_fp[base]).astype(quant.model_dtype))
                cache[base] = [r.numpy() for r in res]
            out[name] = cache[base][idx]
        else:
            if name not in src_fp:
                raise KeyError(f"non-quantized parameter {name!r} missing from the fp source weights")
            out[name] = np.asarray(src_fp[name]).astype(p.dtype)
    return out
