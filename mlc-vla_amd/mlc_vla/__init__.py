"""MI355X (gfx950) implementation of mlc-vla's M1 denoise path.

Drop-in host API: ``mlc_vla.sample.PiZeroRunner`` (sample / sample_graph), the VM-style
functions ``prefill`` / ``denoise_step_kv`` / ``denoise_loop_kv`` from
``mlc_vla.compile.compile_model`` + ``mlc_vla.runtime.VirtualMachine``, the q4f16_1
quantizer in ``mlc_vla.quant`` / ``mlc_vla.compile_quant``.  All arithmetic of those
functions runs in hand-written HIP kernels (``libmlcvla_hip.so``, C ABI in
``include/mlcvla.h``).
"""

__version__ = "0.1.0"
