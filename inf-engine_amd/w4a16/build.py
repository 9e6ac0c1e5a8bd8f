"""Build ``libw4a16.so`` (gfx950) in-tree with hipcc.

    python -m w4a16.build          # from inf-engine_amd/
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [os.path.join(ROOT, "csrc", "w4a16_kernels.hip")]
# Files the library is compiled from (sources and the headers they include).
DEPENDENCIES = SOURCES + [
    os.path.join(ROOT, "csrc", "w4a16_device.h"),
    os.path.join(ROOT, "csrc", "slot_protocol.h"),
    os.path.join(os.path.dirname(ROOT), "include", "w4a16.h"),
]
OUTPUT = os.path.join(HERE, "libw4a16.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Code-generation flags every compile of the kernel source uses.
DEVICE_FLAGS = [
    # Keep the compiler from forming packed-fp32 VALU ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: the kernels rescale their
    # accumulators with VALU ops every 128-row group, which on AGPRs costs a
    # read and a write per element.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", *DEVICE_FLAGS]


def is_stale() -> bool:
    """True when the library is missing or older than a file it is built from."""
    if not os.path.exists(OUTPUT):
        return True
    built = os.path.getmtime(OUTPUT)
    return any(os.path.exists(p) and os.path.getmtime(p) > built for p in DEPENDENCIES)


def build(verbose: bool = False) -> str:
    """Compile every HIP source into OUTPUT; returns the library path."""
    tmp = OUTPUT + ".tmp"
    cmd = [HIPCC, *FLAGS, *SOURCES, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}")
    if verbose:
        sys.stdout.write(res.stdout)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))
