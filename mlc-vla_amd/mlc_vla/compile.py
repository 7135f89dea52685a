"""Build entry (drop-in for mlc_vla.compile).

In the reference, ``compile_model`` lowers the TVM graph and JIT-compiles the
kernels (python/mlc_vla/compile.py:99-133).  Here the kernels are prebuilt for
gfx950 (``libmlcvla_hip.so``); ``compile_model`` validates the configuration and
returns the executable description plus the ``named_params`` list.
"""

from __future__ import annotations

import warnings

from .model.pi0.pi0_model import BUILT_FUNCS, KV_FUNCS, named_params
from .runtime import Device, Executable, device

GPU_TARGETS = ("rocm", "hip", "cuda", "gfx950")


def _target_kind(target: str) -> str:
    kind = str(target).split()[0].split("-")[0].lower()
    if kind in GPU_TARGETS:
        return "rocm"
    raise NotImplementedError(
        f"target {target!r}: this build runs on MI355X (gfx950) only; there is no CPU backend")


def cublas_available() -> bool:
    """The cuBLAS BYOC path of the reference does not exist on ROCm."""
    return False


def resolve_cublas(cublas, target_kind: str) -> bool:
    """Tri-state cuBLAS switch of the reference (compile.py:55-76); always False here."""
    if cublas:
        warnings.warn("cublas=True has no effect: GEMMs run in the gfx950 HIP kernels", RuntimeWarning,
                      stacklevel=2)
    return False


def check_config(config, functions=None, quant=None) -> None:
    """float16 models run every function; float32 models (the reference's default dtype,
    pi0_config.py:97) run the M1 functions on generic float32 kernels, unquantized."""
    if config.dtype not in ("float16", "float32"):
        raise NotImplementedError(f"dtype {config.dtype!r}: float16 or float32")
    if config.dtype == "float32":
        if quant is not None:
            raise NotImplementedError("q4f16_1 quantizes the float16 model (construct Pi0Config(dtype='float16'))")
        extra = [f for f in (functions if functions is not None else KV_FUNCS) if f not in KV_FUNCS]
        if extra:
            raise NotImplementedError(f"functions {extra} are built for float16 models only (float32: {KV_FUNCS})")
    if config.attn_logits_dtype != "float32":
        raise NotImplementedError("attn_logits_dtype must be 'float32' in this build")


def compile_model(config, target: str = "rocm", functions=None, cuda_graph: bool = False, cublas=None,
                  hoist_modulation: bool = True):
    """Return ``(executable, named_params)`` (compile.py:99-133).  ``functions`` may name
    embed_language, denoise_step, prefill, denoise_step_kv and denoise_loop_kv; the default is
    the M1 functions (prefill, denoise_step_kv, denoise_loop_kv)."""
    _target_kind(target)
    check_config(config, functions)
    resolve_cublas(cublas, "rocm")
    funcs = tuple(functions) if functions is not None else KV_FUNCS
    unknown = [f for f in funcs if f not in BUILT_FUNCS]
    if unknown:
        raise NotImplementedError(f"functions {unknown} are not built on gfx950 (available: {BUILT_FUNCS})")
    npar = named_params(config, funcs)
    return Executable(config, funcs, npar, None, cuda_graph, hoist_modulation), npar


def _device_for(target: str) -> Device:
    _target_kind(target)
    return device("rocm", 0)
