"""CPU check of the launch planner: tests/native/plan_check.cpp includes the
kernel source, runs make_plan / bind / the workspace queries over ~2500 shapes
(single, grouped, SwiGLU pair, unaligned) and asserts the properties the
kernels rely on (K-split coverage, split-major workgroup order, LDS bound,
disjoint workspace regions clear of the status word, size query >= plan)."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None, reason="needs hipcc")
def test_planner_invariants(tmp_path):
    from w4a16 import build

    exe = tmp_path / "plan_check"
    src = os.path.join(ROOT, "tests", "native", "plan_check.cpp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O1", "-std=c++17", *build.DEVICE_FLAGS, src, "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0 and run.stdout.strip().endswith("ok"), run.stdout + run.stderr


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None, reason="needs hipcc")
def test_planner_invariants_under_address_and_ub_sanitizers(tmp_path):
    """The same sweep with the host side built with AddressSanitizer and
    UndefinedBehaviorSanitizer (host code only; the device code is not run)."""
    from w4a16 import build

    exe = tmp_path / "plan_check_asan"
    src = os.path.join(ROOT, "tests", "native", "plan_check.cpp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", *build.DEVICE_FLAGS,
           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=undefined", src, "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0 and run.stdout.strip().endswith("ok"), run.stdout + run.stderr

