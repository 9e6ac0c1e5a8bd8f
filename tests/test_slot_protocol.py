"""CPU check of the decode kernels' split-K slot protocol: the encoding in
inf-engine_amd/csrc/slot_protocol.h driven by a threaded host emulation
(tests/native/slot_protocol_emu.cpp): publish / poll / in-order sum /
re-zeroing, and the bounded give-up that sets the workspace status word."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_slot_protocol_host_emulation(tmp_path):
    exe = tmp_path / "slot_emu"
    src = os.path.join(ROOT, "tests", "native", "slot_protocol_emu.cpp")
    inc = os.path.join(ROOT, "inf-engine_amd", "csrc")
    subprocess.run(["g++", "-O2", "-std=c++17", "-pthread", "-I", inc, src, "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), res.stdout + res.stderr


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_slot_protocol_host_emulation_under_thread_sanitizer(tmp_path):
    """The threaded emulation built with ThreadSanitizer: publishers, finisher and
    late publishers touch the slots only through atomics."""
    exe = tmp_path / "slot_emu_tsan"
    src = os.path.join(ROOT, "tests", "native", "slot_protocol_emu.cpp")
    inc = os.path.join(ROOT, "inf-engine_amd", "csrc")
    subprocess.run(["g++", "-O1", "-g", "-std=c++17", "-pthread", "-fsanitize=thread", "-I", inc, src, "-o", str(exe)],
                   check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), res.stdout + res.stderr
    assert "WARNING: ThreadSanitizer" not in res.stderr, res.stderr


def test_status_offset_and_spin_limit_api(native_lib):
    from w4a16 import _native as nat
    import ctypes

    off = ctypes.c_size_t(0)
    assert native_lib.w4a16_status_offset(1 << 20, ctypes.byref(off)) == nat.W4A16_OK
    assert off.value == (1 << 20) - 4
    assert native_lib.w4a16_status_offset(1001, ctypes.byref(off)) == nat.W4A16_OK and off.value == 996
    assert native_lib.w4a16_status_offset(100, ctypes.byref(off)) == nat.W4A16_ERR_WORKSPACE
    assert native_lib.w4a16_status_offset(1 << 20, None) == nat.W4A16_ERR_NULL
    old = nat.set_spin_limit(5)
    assert old == 1 << 20
    assert nat.set_spin_limit(old) == 5
