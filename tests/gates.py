"""Parity gates shared by the GPU tests and by the ablation tests that show the gates can
fail (a planted mistake in the oracle, on the CPU, must be rejected by the same gate a GPU
result has to pass).

Each gate returns ``(ok, stats)`` so that a test can assert either outcome and print the
margins.  The tolerances are the ones the GPU tests use:

- ``action_gate``: actions / velocities against the float32 oracle, max_abs <= 1e-2 and
  cosine >= 0.999 (the target tolerance of the fp16 path);
- ``rel_gate``: an intermediate tensor (prefix K / V of one layer, the residual stream after
  one layer, one attention output) against the float32 oracle, max_abs <= rel * max|ref| and
  cosine >= cos; the defaults are the per-layer gate of the full-size tests;
- ``kv_gate``: one layer's prefix K or V against the float32 oracle, max_abs <= 1e-2 max|ref|
  and cosine >= 0.99999 (the 1.1-scaled prefill attention moves the next layer's K / V to a
  cosine of 0.999985, while fp16 rounding alone stays above 0.9999995 in three layers);
- ``kernel_gate``: one kernel against a float64 reference, max_abs <= 2e-3 max|ref| + 2e-4 and
  cosine > 0.99999.
"""

from __future__ import annotations

import numpy as np


def _stats(got, ref):
    g = np.asarray(got, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    finite = bool(np.all(np.isfinite(g)))
    err = float(np.max(np.abs(g - r))) if finite else float("inf")
    cos = float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r) + 1e-300)) if finite else -1.0
    return finite, err, cos, float(np.max(np.abs(r)))


def action_gate(got, ref, atol=1e-2, cos=0.999):
    finite, err, c, scale = _stats(got, ref)
    return finite and err <= atol and c >= cos, dict(max_abs=err, cos=c, scale=scale)


def rel_gate(got, ref, rel=1e-2, cos=0.9999):
    finite, err, c, scale = _stats(got, ref)
    return finite and err <= rel * scale and c >= cos, dict(max_abs=err, rel=err / max(scale, 1e-300), cos=c,
                                                            scale=scale)


def kv_gate(got, ref):
    return rel_gate(got, ref, rel=1e-2, cos=0.99999)


def kernel_gate(got, ref):
    finite, err, c, scale = _stats(got, ref)
    return finite and err <= 2e-3 * scale + 2e-4 and c > 0.99999, dict(max_abs=err, cos=c, scale=scale)
