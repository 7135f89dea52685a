"""q4f16_1 group quantization restated in numpy (oracle; test infrastructure only).

Preset q4f16_1 (python/mlc_vla/quant.py:376-380): int4 stored as uint32 (8 nibbles
per word), group size 32 along K (the input dim), zero point 7 (max_int =
2^(4-1)-1, quant.py:147), fp16 scales, "NK" layout: q_weight [N, ceil(K/32)*4]
uint32, q_scale [N, ceil(K/32)] fp16.

==================  ==========================================  ======================================
oracle function     reference                                   pinned by (tests/test_oracle_q4.py)
==================  ==========================================  ======================================
quantize            quant.py:217-266 (_quantize),               hand-computed known answers, q in [0,14],
                    quant.py:65-86 (pack_weight)                max|w| -> 0 or 14, |w-deq| <= s/2 + ulp,
                                                                brute-force per-element restatement
unpack_nibbles      quant.py:46-62 (convert_uint_to_float)      bit-by-bit pack/unpack round trip
dequantize          quant.py:176-193 (_dequantize)              exact (q-7)*s product check in fp64
linear_q4           quant.py:301-325 (GroupQuantizeLinear)      equals linear on the dequantized matrix
quantize_params     compile_quant.py:71-103                     name/shape/dtype contract
==================  ==========================================  ======================================

Arithmetic: the quantizer runs in the model dtype (fp16).  Each fp16 operation is
emulated as the float32 operation followed by one rounding to fp16, which is how
LLVM lowers half arithmetic on a CPU without native fp16 (the reference JIT-compiles
the quantizer for llvm, compile_quant.py:77-96).  ``tirx.round`` is taken as
round-half-to-even (LLVM ``nearbyint``); ties are "parity unpinned" since TVM is not
importable here.  A group whose max |w| is 0 has scale 0 and the reference divides
0/0; its code is not pinned, and this restatement (like the HIP quantizer) writes 7
so that the group dequantizes to +0.
"""

from __future__ import annotations

from typing import Dict, List, Sequence, Tuple

import numpy as np

GROUP = 32
BITS = 4
PER_WORD = 8
MAX_INT = 7


def quantize(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """fp16 [N, K] -> (q_weight uint32 [N, ceil(K/32)*4], q_scale fp16 [N, ceil(K/32)])."""
    w16 = np.asarray(w).astype(np.float16)
    n, k = w16.shape
    ng = -(-k // GROUP)
    kp = ng * GROUP
    wp = np.zeros((n, kp), np.float16)
    wp[:, :k] = w16
    valid = np.zeros((n, kp), bool)
    valid[:, :k] = True
    absw = np.where(valid, np.abs(wp), np.float16(0.0)).reshape(n, ng, GROUP)
    max_abs = absw.max(axis=-1)                                            # fp16, exact
    scale = (max_abs.astype(np.float32) / np.float32(MAX_INT)).astype(np.float16)
    sb = np.repeat(scale, GROUP, axis=1)
    with np.errstate(divide="ignore", invalid="ignore"):
        scaled = (wp.astype(np.float32) / sb.astype(np.float32)).astype(np.float16)
    scaled = (scaled.astype(np.float32) + np.float32(MAX_INT)).astype(np.float16)
    r = np.rint(scaled.astype(np.float32))                                 # ties to even
    r = np.where(sb == 0, np.float32(MAX_INT), r)
    q = np.clip(r, 0, 2 * MAX_INT).astype(np.uint32)
    q = np.where(valid, q, np.uint32(0)).astype(np.uint32)
    q_weight = pack(q)
    return q_weight, scale


def pack(q: np.ndarray) -> np.ndarray:
    """word[n, j] = sum_r q[n, 8j+r] << 4r (quant.py:65-86)."""
    n, k = q.shape
    nw = -(-k // PER_WORD)
    qp = np.zeros((n, nw * PER_WORD), np.uint64)
    qp[:, :k] = q
    qp = qp.reshape(n, nw, PER_WORD)
    shifts = (np.arange(PER_WORD, dtype=np.uint64) * BITS)[None, None, :]
    return np.bitwise_or.reduce(qp << shifts, axis=-1).astype(np.uint32)


def unpack_nibbles(q_weight: np.ndarray, k: int) -> np.ndarray:
    """nibble[n, k] = (word[n, k//8] >> 4*(k%8)) & 0xF (quant.py:46-62)."""
    qw = np.asarray(q_weight, np.uint32)
    idx = np.arange(k)
    words = qw[:, idx // PER_WORD]
    return ((words >> (BITS * (idx % PER_WORD)).astype(np.uint32)) & np.uint32(0xF)).astype(np.uint8)


def dequantize(q_weight: np.ndarray, q_scale: np.ndarray, k: int = None) -> np.ndarray:
    """W[n,k] = fp16(fp16(nibble) - 7) * scale[n, k//32], one fp16 rounding (quant.py:176-193)."""
    qs = np.asarray(q_scale, np.float16)
    if k is None:
        k = qs.shape[1] * GROUP
    nib = unpack_nibbles(q_weight, k).astype(np.float32) - np.float32(MAX_INT)
    s = qs.astype(np.float32)[:, np.arange(k) // GROUP]
    return (nib * s).astype(np.float16)


def linear_q4(x: np.ndarray, q_weight, q_scale, bias=None) -> np.ndarray:
    """fp16(x @ dequant(W)^T) (+ fp16 bias add) (quant.py:301-325)."""
    w = dequantize(q_weight, q_scale).astype(np.float32)
    y = (np.asarray(x, np.float16).astype(np.float32) @ w.T).astype(np.float16)
    if bias is not None:
        y = (y.astype(np.float32) + np.asarray(bias, np.float16).astype(np.float32)).astype(np.float16)
    return y


def quantized_specs(specs: Sequence[Tuple[str, Tuple[int, ...]]]) -> List[Tuple[str, Tuple[int, ...], str]]:
    """(name, shape, dtype) after GroupQuantize.quantize_model (quant.py:151-174, :269-288).

    Every 2-D ``X.weight`` (an nn.Linear) becomes ``X.q_weight`` (uint32) and
    ``X.q_scale`` (fp16); every other parameter keeps its name as fp16.
    """
    out: List[Tuple[str, Tuple[int, ...], str]] = []
    for name, shape in specs:
        if name.endswith(".weight") and len(shape) == 2:
            base = name[: -len(".weight")]
            n, k = shape
            ng = -(-k // GROUP)
            out.append((base + ".q_weight", (n, ng * GROUP // PER_WORD), "uint32"))
            out.append((base + ".q_scale", (n, ng), "float16"))
        else:
            out.append((name, tuple(shape), "float16"))
    return out


def quantize_params(src_fp: Dict[str, np.ndarray],
                    specs: Sequence[Tuple[str, Tuple[int, ...]]]) -> Dict[str, np.ndarray]:
    """fp params -> q params keyed by quantized names (compile_quant.py:71-103)."""
    out: Dict[str, np.ndarray] = {}
    for name, shape in specs:
        if name.endswith(".weight") and len(shape) == 2:
            base = name[: -len(".weight")]
            qw, qs = quantize(src_fp[name].astype(np.float16))
            out[base + ".q_weight"] = qw
            out[base + ".q_scale"] = qs
        else:
            out[name] = src_fp[name].astype(np.float16)
    return out
