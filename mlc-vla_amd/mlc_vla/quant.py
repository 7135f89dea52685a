"""Group weight quantization presets and the q4f16_1 quantizer (drop-in for mlc_vla.quant).

Preset fields and derived sizes follow the reference's GroupQuantize
(python/mlc_vla/quant.py:116-149, :370-392).  Quantizing and dequantizing run in
the gfx950 kernels (``mlcv_q4_quantize`` / ``mlcv_q4_dequantize``), which
implement quant.py:217-266 (+ pack_weight :65-86) and quant.py:176-193:

    per (row n, group of 32 along K):  s = fp16(max|w| / 7)
    q = clamp(round_half_even(fp16(fp16(w / s) + 7)), 0, 14)
    word[n, j] = sum_r q[n, 8j + r] << 4r
    dequant:  W[n, k] = fp16(fp16(q - 7) * s)

Only q4f16_1 is built on gfx950; the other presets are listed for completeness.
"""

from __future__ import annotations

import ctypes
import dataclasses
from typing import Callable, Dict, List

import numpy as np
import torch

from . import _native as N
from . import runtime

_BITS = {"int3": 3, "int4": 4, "int8": 8}


@dataclasses.dataclass
class QuantizeMapping:
    """fp weight name -> quantized names + the function producing them (quant.py:35-40)."""

    param_map: Dict[str, List[str]]
    map_func: Dict[str, Callable]


@dataclasses.dataclass
class GroupQuantize:
    name: str
    kind: str
    group_size: int
    quantize_dtype: str
    storage_dtype: str
    model_dtype: str
    linear_weight_layout: str
    quantize_embedding: bool = True
    quantize_final_fc: bool = True
    num_elem_per_storage: int = 0
    num_storage_per_group: int = 0
    max_int_value: int = 0

    def __post_init__(self):
        if self.kind != "group-quant":
            raise ValueError(f"GroupQuantize covers kind 'group-quant', got {self.kind!r}")
        bits = _BITS[self.quantize_dtype]
        word_bits = 32 if self.storage_dtype == "uint32" else int(self.storage_dtype[4:])
        per_word = word_bits // bits
        if per_word == 0:
            raise ValueError(f"a {bits}-bit {self.quantize_dtype} value does not fit in one {self.storage_dtype}")
        if self.group_size % per_word:
            raise ValueError(f"group_size {self.group_size} is not a whole number of {self.storage_dtype} words "
                             f"({per_word} values each)")
        # derived sizes: values per storage word, words per group, and the offset that maps a
        # signed code in [-offset, offset + 1] to the unsigned value stored
        self.num_elem_per_storage = per_word
        self.num_storage_per_group = self.group_size // per_word
        self.max_int_value = (1 << (bits - 1)) - 1
        self.linear_quant_axis = 0 if self.linear_weight_layout == "KN" else 1

    @property
    def supported(self) -> bool:
        return (self.quantize_dtype, self.storage_dtype, self.model_dtype, self.group_size,
                self.linear_weight_layout) == ("int4", "uint32", "float16", 32, "NK")

    def _require(self):
        if not self.supported:
            raise NotImplementedError(f"preset {self.name}: only q4f16_1 is built on gfx950")

    def quantize_weight(self, weight, axis: int = -1, output_transpose: bool = False):
        """[N, K] weight -> [q_weight [N, K/8] uint32, q_scale [N, K/32] fp16] as device tensors."""
        self._require()
        if output_transpose or axis not in (-1, 1):
            raise NotImplementedError("only the NK layout (quantization along K) is built")
        w = runtime.as_tensor(weight) if not isinstance(weight, np.ndarray) else runtime.tensor(
            np.asarray(weight, dtype=np.float16))
        if w.dtype != "float16":
            w = runtime.Tensor(w.torch.to(torch.float16), "float16")
        n, k = w.shape
        if k % self.group_size:
            raise NotImplementedError("K must be a multiple of the group size")
        qw = runtime.empty((n, k // self.num_elem_per_storage), "uint32")
        qs = runtime.empty((n, k // self.group_size), "float16")
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        N.call("mlcv_q4_quantize", runtime._ptr(w), runtime._ptr(qw), runtime._ptr(qs), n, k, stream)
        return [qw, qs]

    def dequantize_weight(self, q_weight, q_scale):
        """[q_weight, q_scale] -> fp16 [N, K] device tensor (quant.py:176-193)."""
        self._require()
        qw, qs = runtime.as_tensor(q_weight), runtime.as_tensor(q_scale)
        n, kw = qw.shape
        k = kw * self.num_elem_per_storage
        out = runtime.empty((n, k), "float16")
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        N.call("mlcv_q4_dequantize", runtime._ptr(qw), runtime._ptr(qs), runtime._ptr(out), n, k, stream)
        return out


PRESETS: Dict[str, GroupQuantize] = {
    "q4bf16_1": GroupQuantize(name="q4bf16_1", kind="group-quant", group_size=32, quantize_dtype="int4",
                              storage_dtype="uint32", model_dtype="bfloat16", linear_weight_layout="NK",
                              quantize_embedding=False, quantize_final_fc=True),
    "q4f16_1": GroupQuantize(name="q4f16_1", kind="group-quant", group_size=32, quantize_dtype="int4",
                             storage_dtype="uint32", model_dtype="float16", linear_weight_layout="NK",
                             quantize_embedding=False, quantize_final_fc=True),
    "q3f16_1": GroupQuantize(name="q3f16_1", kind="group-quant", group_size=40, quantize_dtype="int3",
                             storage_dtype="uint32", model_dtype="float16", linear_weight_layout="NK",
                             quantize_embedding=False, quantize_final_fc=True),
}


def get_quant(name: str) -> GroupQuantize:
    if name not in PRESETS:
        raise KeyError(f"unknown quantization preset {name!r}; available: {list(PRESETS)}")
    return PRESETS[name]
