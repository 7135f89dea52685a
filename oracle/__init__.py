"""CPU oracle for the pi0.5 M1 denoise path (test infrastructure only).

This package restates, in numpy (plus a torch-fp64 second restatement of the
joint M0 forward), the arithmetic of mlc-vla's ``prefill`` / ``denoise_step_kv``
/ ``denoise_loop_kv`` and of its q4f16_1 group quantizer.  It exists to CHECK the
HIP implementation; nothing in the product imports it.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker / the timed CPU baseline.

Modules
-------
pi0_oracle   model math (M1 prefill/decode/loop, host helpers), numpy
m0_torch     independent torch-fp64 restatement of the M0 joint forward
q4_oracle    q4f16_1 quantize / pack / unpack / dequant / linear, numpy

Parity pinning (which check pins which function) is listed in each module's
docstring.  Functions without an independent check are marked
"parity unpinned" there.
"""
