"""The launch planners (mlc-vla_amd/csrc/plan.h) on the CPU: tests/plan_check.cpp sweeps the
attention, skinny-GEMM and tile-GEMM plans and checks their invariants (every key / K range
covered with no empty slice, partials inside their workspace, a split-K tile grid resident at
once), built with g++ under AddressSanitizer and UndefinedBehaviorSanitizer."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_planners_under_sanitizers(tmp_path):
    exe = str(tmp_path / "plan_check")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-Wall", "-Werror", os.path.join(HERE, "plan_check.cpp"), "-o", exe], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    assert "failures: 0" in r.stdout
