"""The launch chain -- denoise_step_kv's default path -- checked kernel by kernel.

After a step on the chain, its operations run again one at a time with the same kernels and
arguments (stepcheck.ChainReplay, through mlcv_bench_op): the replay must reproduce the step's
velocity bit for bit, and each operation's output is checked against the oracle fed the GPU's
own inputs, then along the whole chain (stepcheck.per_op_checks / chain_checks).  These are
the instantiations the step runs: the adaRMS-by-prescale q/k/v GEMM with RoPE and the hi/lo q
fragments, the step attention (fragment-order q, fp32 suffix keys) with its split combine,
o_proj and down with the gated residual and the next norm's pre-scaled input, gate_up with
GeGLU, and the head.  Tiny size and the full pi0.5 shape (968 prefix keys, 50 suffix rows,
8 heads of 256).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import TINY_KWARGS
from stepcheck import ChainReplay, Step, chain_checks, per_op_checks

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("which", ["tiny", "full"])
def test_chain_ops_vs_oracle(which):
    kw = TINY_KWARGS if which == "tiny" else dict(dtype="float16", action_horizon=50)
    print(f"launch chain op by op: {which}", flush=True)
    s = Step(kw, form="chain")
    v = s.run()
    r = ChainReplay(s)
    np.testing.assert_array_equal(r.probe("vout", 0).reshape(v.shape), v)
    per_op_checks(r, v)
    chain_checks(r, v)
