"""mlcv_linear_noalloc -- mlcv_linear with its split-K scratch in a static device array (no
allocation) -- against mlcv_linear through the C ABI: two calls in a row, the second with a
smaller input, fp16 and q4f16_1 weights, each bit-identical to mlcv_linear's output (same
kernels, same split plan, same summation order); and a size beyond its scratch is refused
before anything runs."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from mlc_vla import _native as N
from oracle import q4_oracle as Q

pytestmark = pytest.mark.gpu


def _st():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def _case(m, k, n, q4, seed):
    rng = np.random.default_rng(seed)
    x = _dev(rng.standard_normal((m, k)).astype(np.float16))
    w = (0.02 * rng.standard_normal((n, k))).astype(np.float16)
    b = _dev((0.02 * rng.standard_normal(n)).astype(np.float16))
    if q4:
        qw, qs = Q.quantize(w)
        return x, None, _dev(qw), _dev(qs), b
    return x, _dev(w), None, None, b


@pytest.mark.parametrize("q4", [False, True], ids=["f16", "q4"])
def test_noalloc_linear_matches_linear_twice(q4):
    # the first call: an 8192-wide projection over 50 rows (gate_up of the step, split-K);
    # the second, smaller: 16 rows, 512 -> 1024 (other tiles, another split count)
    for m, k, n in ((50, 1024, 8192), (16, 512, 1024)):
        print(f"noalloc linear M={m} K={k} N={n} q4={q4}", flush=True)
        x, w, qw, qs, b = _case(m, k, n, q4, seed=m + k + n)
        y_ref = torch.empty((m, n), dtype=torch.float16, device="cuda")
        y = torch.full((m, n), float("nan"), dtype=torch.float16, device="cuda")
        N.call("mlcv_linear", _p(x), m, k, _p(w), _p(qw), _p(qs), _p(b), _p(y_ref), n, _st())
        N.call("mlcv_linear_noalloc", _p(x), m, k, _p(w), _p(qw), _p(qs), _p(b), _p(y), n, _st())
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), (y.float() - y_ref.float()).abs().max().item()


def test_noalloc_linear_refuses_sizes_beyond_its_scratch():
    m, k, n = 1, 32, 64 * 70000  # 70000 output tiles: more arrival counters than the scratch holds
    x = torch.zeros((m, k), dtype=torch.float16, device="cuda")
    w = torch.zeros((1, k), dtype=torch.float16, device="cuda")  # never read: refused first
    y = torch.zeros((m, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(N.MlcvError, match="output tiles"):
        N.call("mlcv_linear_noalloc", _p(x), m, k, _p(w), None, None, None, _p(y), n, _st())
