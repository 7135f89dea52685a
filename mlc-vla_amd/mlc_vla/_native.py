"""ctypes binding of ``libmlcvla_hip.so`` (C ABI declared in include/mlcvla.h).

The library is the only compute path: if it is missing or no HIP device is
present, every entry point raises -- there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading

# MLCV_LIB names another build of the library (the phase-stamp build for profiling)
LIB_PATH = os.environ.get("MLCV_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmlcvla_hip.so")

MLCV_DTYPE_F16 = 1
MLCV_DTYPE_F32 = 2
MLCV_QUANT_NONE = 0
MLCV_QUANT_Q4F16_1 = 1
MLCV_OPT_USE_GRAPH = 1
MLCV_OPT_HOIST_MODULATION = 2
MLCV_OPT_PERSIST = 3
MLCV_OPT_PERSIST_SPIN = 4
MLCV_OPT_MEET_POLLS = 5
MLCV_OPT_XTP = 6
MLCV_OPT_XTP_KEEP = 7
MLCV_OPT_SYNC_WORDS = 8
MLCV_OPT_MASK_SKIP = 9
MLCV_OPT_STEP_GRAPH = 10
PROBES = {"x": 0, "q": 1, "k": 2, "v": 3, "attn": 4, "x_mid": 5, "h": 6, "mod": 7, "vout": 8, "xcd_x": 9}

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32


class MlcvError(RuntimeError):
    """A failing C ABI call (message from mlcv_last_error)."""


class Config(ctypes.Structure):
    _fields_ = [
        ("vlm_width", _i32), ("vlm_mlp", _i32), ("ae_width", _i32), ("ae_mlp", _i32),
        ("depth", _i32), ("num_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("prefix_len", _i32), ("suffix_len", _i32), ("action_dim", _i32), ("num_steps", _i32),
        ("rms_norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float),
        ("dtype", _i32), ("quant", _i32),
    ]


class VisionConfig(ctypes.Structure):
    """mlcv_vision_config (include/mlcvla.h)."""
    _fields_ = [(n, _i32) for n in ("image_size", "patch_size", "num_channels", "hidden_size", "intermediate_size",
                                     "num_hidden_layers", "num_attention_heads", "projection_dim")] + \
               [("layer_norm_eps", ctypes.c_float)]


# name -> (restype, argtypes): every symbol include/mlcvla.h declares
SIGNATURES = {
    "mlcv_last_error": (ctypes.c_char_p, []),
    "mlcv_param_count": (ctypes.c_int, [ctypes.POINTER(Config), ctypes.POINTER(_i32)]),
    "mlcv_create": (ctypes.c_int, [ctypes.POINTER(Config), ctypes.POINTER(_vp)]),
    "mlcv_destroy": (ctypes.c_int, [_vp]),
    "mlcv_bind_params": (ctypes.c_int, [_vp, ctypes.POINTER(_vp), _i32, _vp]),
    "mlcv_set_option": (ctypes.c_int, [_vp, _i32, ctypes.c_int64]),
    "mlcv_sync": (ctypes.c_int, [_vp, _vp]),
    "mlcv_step_probe": (ctypes.c_int, [_vp, _i32, _i32, _vp, ctypes.c_size_t, _vp]),
    "mlcv_prefill": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "mlcv_denoise_step": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "mlcv_embed_language": (ctypes.c_int, [_vp, _i32, _vp, _i32, _i32, _vp, _vp]),
    "mlcv_vision_param_count": (ctypes.c_int, [ctypes.POINTER(VisionConfig), ctypes.POINTER(_i32)]),
    "mlcv_embed_image_workspace": (ctypes.c_int, [ctypes.POINTER(VisionConfig), ctypes.POINTER(ctypes.c_size_t)]),
    "mlcv_embed_image": (ctypes.c_int, [ctypes.POINTER(VisionConfig), ctypes.POINTER(_vp), _i32, _vp, _vp, _vp,
                                        ctypes.c_size_t, _vp]),
    "mlcv_denoise_step_kv": (ctypes.c_int, [_vp] * 10),
    "mlcv_denoise_loop_kv": (ctypes.c_int, [_vp] * 10),
    "mlcv_chunk": (ctypes.c_int, [_vp] * 9),
    "mlcv_joint_attention": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp,
                                            _i32, _vp, _vp]),
    "mlcv_prefill_attention": (ctypes.c_int, [_vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                              _vp]),
    "mlcv_q4_quantize": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _vp]),
    "mlcv_q4_dequantize": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _vp]),
    "mlcv_linear": (ctypes.c_int, [_vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp]),
    "mlcv_linear_noalloc": (ctypes.c_int, [_vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp]),
    "mlcv_tile_linear": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i32, _vp, _i32, _i32, _i32, _vp]),
    "mlcv_bench_op": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp, _vp, _vp]),
}

OPS = {"time_mod": 0, "modulation": 1, "qkv": 2, "attention": 3, "o_proj": 4, "gate_up": 5, "down": 6, "head": 7,
       "attention_only": 8, "action_in": 9, "xt_attn": 10, "xt_mlp": 11}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library (raises if it was not built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise MlcvError(
                    f"{LIB_PATH} is missing: build it with `python mlc-vla_amd/build.py` "
                    "(the gfx950 HIP library is the only compute path)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().mlcv_last_error()
        raise MlcvError(msg.decode() if msg else f"mlcv error {rc}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
