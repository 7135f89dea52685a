"""Bounded device-side waits that give up are reported as failed calls, forced from the host
so that every kernel still exits normally (a poll limit of zero: the waiting workgroups give
up at once and the last arrival still resets the meeting), and the library computes correctly
again afterwards.

- The tile GEMM's split-K meeting (csrc/gemm_tile.hip): through mlcv_tile_linear, which
  returns -4, and through the prefill of a context (MLCV_OPT_MEET_POLLS), reported by
  mlcv_sync when the keys are read.

Also: a failed mlcv_bind_params leaves the context unbound, so a caller that still believes
the old binding stands gets "parameters not bound" instead of a step over freed copies.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import TINY_KWARGS
from mlc_vla import _native as N
from mlc_vla import runtime
from mlc_vla.model.pi0 import Pi0Config
from mlc_vla.sample import PiZeroRunner, make_prefix_mask_np
from oracle import pi0_oracle as O

pytestmark = pytest.mark.gpu


def _st():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr())


def test_tile_linear_meeting_give_up_is_an_error():
    # 968 x 2048 -> 1024 (the o_proj of the prefill at P=968): 32 tiles over 8 K slices
    m, k, n = 968, 2048, 1024
    print(f"tile linear meeting give-up M={m} K={k} N={n}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn((m, k), generator=g, device="cuda").half()
    w = (torch.randn((n, k), generator=g, device="cuda") / k ** 0.5).half()
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    with pytest.raises(N.MlcvError, match="gave up"):
        N.call("mlcv_tile_linear", _p(x), m, k, _p(w), n, _p(y), 0, 0, 0, _st())
    assert torch.isnan(y.float()).any().item()  # the workgroups that gave up wrote NaN
    N.call("mlcv_tile_linear", _p(x), m, k, _p(w), n, _p(y), 0, 0, -1, _st())
    torch.cuda.synchronize()
    ref = (x.float() @ w.float().T)
    assert torch.isfinite(y.float()).all().item()
    assert (y.float() - ref).abs().max().item() < 2e-2


def test_prefill_meeting_give_up_is_reported_by_sync():
    cfg = Pi0Config(**TINY_KWARGS)
    d = O.dims_from_config(cfg)
    runner = PiZeroRunner(cfg, "rocm")
    p16 = O.make_params(O.param_specs(d), 0, "float16")
    params = runner.to_params([p16[n] for n, _ in runner.named_params])
    prefix = np.random.default_rng(3).standard_normal((1, cfg.prefix_len, cfg.vlm.width)).astype(np.float16)
    dv = lambda a: runtime.tensor(a, runner.dev)  # noqa: E731
    pm = dv(make_prefix_mask_np(cfg.prefix_len))
    vm = runner.vm
    good_k, good_v = (t.numpy() for t in vm["prefill"](dv(prefix), pm, params))
    vm.set_meet_polls(0)
    try:
        keys, _ = vm["prefill"](dv(prefix), pm, params)
        with pytest.raises(N.MlcvError, match="split-K meeting"):
            keys.numpy()
    finally:
        vm.set_meet_polls(1 << 22)
    k2, v2 = (t.numpy() for t in vm["prefill"](dv(prefix), pm, params))
    np.testing.assert_array_equal(k2, good_k)
    np.testing.assert_array_equal(v2, good_v)


def test_failed_bind_leaves_the_context_unbound():
    from stepcheck import Step

    print("bind failure: tiny model", flush=True)
    s = Step(TINY_KWARGS, form="chain")
    vm = s.runner.vm
    good = s.run()
    ptrs = list(vm._bound)  # the device pointers of the current binding
    ptrs[len(ptrs) // 2] = None
    arr = (ctypes.c_void_p * len(ptrs))(*[ctypes.c_void_p(p) if p else None for p in ptrs])
    with pytest.raises(N.MlcvError, match="null parameter pointer"):
        N.call("mlcv_bind_params", vm._ctx, arr, len(ptrs), _st())
    # the VM still believes in its old binding; the context refuses instead of stepping
    with pytest.raises(N.MlcvError, match="parameters not bound"):
        s.run()
    vm._bound = None  # a caller that binds again gets the same results as before
    np.testing.assert_array_equal(s.run(), good)
