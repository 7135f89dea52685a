"""Build the gfx950 HIP library ``mlc_vla/libmlcvla_hip.so`` in-tree.

    python mlc-vla_amd/build.py          # compiles every csrc/*.hip and links
    python mlc-vla_amd/build.py --trace  # also libmlcvla_hip_trace.so (XCD step phase stamps)

Each translation unit is compiled for ``--offload-arch=gfx950`` only, in
parallel, into ``mlc-vla_amd/_build/``; the shared library is written next to
the Python package so that it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "mlc_vla", "libmlcvla_hip.so")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # no packed-fp32 VALU instructions on this target: some of their forms gave wrong results
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the gfx950 library)")


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in r.stdout.splitlines() if "packed-fp32-ops" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False) -> str:
    hipcc = _hipcc()
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = [os.path.join(BUILD, s[:-4] + ".o") for s in srcs]
    jobs = [[hipcc, *FLAGS, "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(srcs, objs)]
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for out in ex.map(_run, jobs):
            if verbose and out.strip():
                print(out)
    tmp = LIB + ".tmp"
    # --no-undefined: a kernel whose host launch stub went missing fails here, not at load
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


TRACE_LIB = os.path.join(HERE, "mlc_vla", "libmlcvla_hip_trace.so")


def build_trace(verbose: bool = False) -> str:
    """The library with the XCD step's phase stamps (step_xtp.hip with MLCV_XT_TRACE: every
    workgroup of the last step's launches writes s_memrealtime at each phase boundary), for
    ``bench.py --xt-timeline`` with ``MLCV_LIB`` naming it.  The other objects are the normal
    build's."""
    hipcc = _hipcc()
    build(verbose=False)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = [os.path.join(BUILD, s[:-4] + ".o") for s in srcs if s != "step_xtp.hip"]
    tobj = os.path.join(BUILD, "step_xtp_trace.o")
    _run([hipcc, *FLAGS, "-DMLCV_XT_TRACE", "-c", os.path.join(CSRC, "step_xtp.hip"), "-o", tobj])
    tmp = TRACE_LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", *objs, tobj, "-o", tmp])
    os.replace(tmp, TRACE_LIB)
    if verbose:
        print(f"built {TRACE_LIB}")
    return TRACE_LIB


if __name__ == "__main__":
    if "--trace" in sys.argv:
        build_trace(verbose="-q" not in sys.argv)
    else:
        build(verbose="-q" not in sys.argv)
