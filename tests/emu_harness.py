"""Harness of the emulated-kernel tests: build the gfx950 kernel source as host
C++ with the wave emulator of tests/native/emu, and drive its C ABI from
Python with guarded host buffers standing in for device memory.

TEST INFRASTRUCTURE ONLY (tests/test_emulated_kernels.py and the scripts it
starts); nothing in the product imports it.
"""

from __future__ import annotations

import ctypes
import glob
import os
import shutil
import subprocess
import sys

import numpy as np

from oracle import int4_oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EMU = os.path.join(ROOT, "tests", "native", "emu")
KERNELS = os.path.join(ROOT, "inf-engine_amd", "csrc", "w4a16_kernels.hip")


def clang() -> str | None:
    for c in ("/opt/rocm/llvm/bin/clang++", shutil.which("clang++")):
        if c and os.path.exists(c):
            return c
    return None


def ubsan_runtime() -> str | None:
    libs = glob.glob(os.path.join(os.path.dirname(os.path.dirname(clang() or "")), "lib", "clang", "*", "lib",
                                  "linux", "libclang_rt.ubsan_standalone-x86_64.so"))
    return libs[0] if libs else None


def build_emulator(out_dir: str, source: str = KERNELS, ubsan: bool = False) -> str:
    """Compile `source` with the wave emulator into out_dir/libw4a16_emu.so
    (with `ubsan`, the kernel code under UndefinedBehaviorSanitizer, aborting
    at the first finding: misaligned vector accesses, signed overflow, bad shifts)."""
    sys.path.insert(0, EMU)
    try:
        import prepare
    finally:
        sys.path.remove(EMU)
    tu = os.path.join(out_dir, "w4a16_host.cpp")
    with open(source) as f:
        text = prepare.transform(f.read())
    with open(tu, "w") as f:
        f.write(text)
    lib = os.path.join(out_dir, "libw4a16_emu.so")
    rt = os.path.join(out_dir, "emu_runtime.o")
    inc = [f"-I{EMU}", f"-I{os.path.join(ROOT, 'inf-engine_amd', 'csrc')}", f"-I{os.path.join(ROOT, 'include')}"]
    # The emulator (MFMA arithmetic, fiber switches) optimized; the kernel TU at
    # -O0: it builds in seconds instead of a minute and runs about 1.5x slower.
    san = []
    if ubsan:
        rt_lib = ubsan_runtime()
        san = ["-fsanitize=undefined", "-fno-sanitize-recover=undefined", "-shared-libsan",
               f"-Wl,-rpath,{os.path.dirname(rt_lib)}"]
    for cmd in ([clang(), "-O2", "-std=c++17", "-fPIC", "-c", *inc, os.path.join(EMU, "emu_runtime.cpp"), "-o", rt],
                [clang(), "-O0", "-g", "-std=c++17", "-shared", "-fPIC", *san, *inc, tu, rt, "-o", lib]):
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, res.stdout + res.stderr
    return lib


class Emu:
    """ctypes view of the emulated library plus guarded host 'device' buffers."""

    def __init__(self, path: str):
        self.lib = lib = ctypes.CDLL(path)
        vp, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
        lib.emu_alloc.restype = vp
        lib.emu_alloc.argtypes = [sz]
        lib.w4a16_linear.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, vp, sz, vp]
        lib.w4a16_linear_noalloc.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, vp]
        lib.w4a16_workspace_size.argtypes = [i32, i32, i32, i32, ctypes.POINTER(sz)]
        lib.w4a16_swiglu.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, vp, i64,
                                     i32, i32, i32, i32, vp, sz, vp]
        lib.w4a16_workspace_size_swiglu.argtypes = [i32, i32, i32, i32, ctypes.POINTER(sz)]
        lib.w4a16_bf16_gemv.argtypes = [vp, i64, vp, i64, vp, i64, i32, i32, i32, vp]
        lib.w4a16_dequant.argtypes = [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, vp]
        lib.w4a16_status_offset.argtypes = [sz, ctypes.POINTER(sz)]
        lib.w4a16_noalloc_status.argtypes = [vp, ctypes.POINTER(ctypes.c_uint32)]
        lib.emu_set_capturing.argtypes = [i32]
        lib.emu_load_count.restype = ctypes.c_uint64
        sys.path.insert(0, os.path.join(ROOT, "inf-engine_amd"))
        from w4a16 import _native
        self.Problem = _native.Problem
        lib.w4a16_linear_grouped.argtypes = [ctypes.POINTER(_native.Problem), i32, i32, vp, sz, vp]
        lib.w4a16_workspace_size_grouped.argtypes = [ctypes.POINTER(_native.Problem), i32, i32, ctypes.POINTER(sz)]

    def _aligned(self, nbytes: int) -> int:
        """A 16-byte aligned buffer of nbytes whose end is within 15 bytes of the
        trailing guard page (buffers end at a page boundary, so the start is
        -size mod 16 without the pad)."""
        p = self.lib.emu_alloc(nbytes + (-nbytes) % 16)
        assert p % 16 == 0
        return p

    def put(self, arr: np.ndarray) -> int:
        """Copy arr into a 16-byte aligned guarded buffer (as a device allocation is)."""
        a = np.ascontiguousarray(arr)
        p = self._aligned(a.nbytes)
        ctypes.memmove(p, a.ctypes.data, a.nbytes)
        return p

    def zeros(self, nbytes: int) -> int:
        p = self._aligned(nbytes)
        ctypes.memset(p, 0, nbytes)
        return p

    def get(self, p: int, shape, dtype) -> np.ndarray:
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return np.frombuffer(ctypes.string_at(p, n), dtype=dtype).reshape(shape).copy()

    def workspace(self, nbytes: int) -> tuple[int | None, int]:
        return (self.zeros(nbytes), nbytes) if nbytes else (None, 0)

    def slots_clear(self, ws: int | None, nbytes: int) -> bool:
        """Lower (slot) half zero and status word clear."""
        if not ws:
            return True
        half = (nbytes // 2) & ~255
        off = ctypes.c_size_t(0)
        assert self.lib.w4a16_status_offset(nbytes, ctypes.byref(off)) == 0
        low = self.get(ws, (half,), np.uint8)
        status = self.get(ws + off.value, (1,), np.uint32)[0]
        return not low.any() and status == 0


def bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_value(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def problem(m, k, n, seed, pad_x=0, pad_w=0, quantized=False):
    """x (bf16 bits, [m, k + pad_x]), packed [k/2, n + pad_w], scale [k/128, n + pad_w]."""
    rng = np.random.default_rng(seed)
    if quantized:
        w = (rng.standard_normal((k, n + pad_w)) * 0.02).astype(np.float32)
        packed, scale = orc.quantize(w)
    else:
        packed = rng.integers(-128, 128, size=(k // 2, n + pad_w), dtype=np.int8)
        scale = (rng.random((k // 128, n + pad_w), dtype=np.float32) * 0.01 + 0.001).astype(np.float32)
    xb = bf16_bits(rng.standard_normal((m, k + pad_x)).astype(np.float32))
    return xb, packed, scale


def run_linear(emu, xb, packed, scale, m, k, n, misalign_x=False, check_ws=True):
    lib = emu.lib
    ldx, ldp, lds = xb.shape[1], packed.shape[1], scale.shape[1]
    ws_bytes = ctypes.c_size_t(0)
    assert lib.w4a16_workspace_size(m, n, k, 128, ctypes.byref(ws_bytes)) == 0
    # Round the workspace to what _native would pass (it only grows), with slack.
    nb = ws_bytes.value + (4096 if ws_bytes.value else 0)
    ws, nb = emu.workspace(nb)
    if misalign_x:
        # One element off 16-byte alignment: the generic-load path (and, for M > 32,
        # the decode kernel in 32-row chunks).
        xp = place(emu, xb, 2, front=False)
    else:
        xp = emu.put(xb)
    y = emu.zeros(m * n * 2)
    rc = lib.w4a16_linear(xp, ldx, emu.put(packed), ldp, emu.put(scale), lds, y, n, m, n, k, 128, ws, nb, None)
    assert rc == 0, rc
    if check_ws:
        assert emu.slots_clear(ws, nb), "workspace slot half or status word not clear after the call"
    return emu.get(y, (m, n), np.uint16)


def reference(xb, packed, scale, m, k, n):
    return orc.fused_reference(bf16_value(xb[:, :k]), packed[:, :n], scale[:, :n])


def place(emu, arr, misalign: int, front: bool) -> int:
    """Copy arr to a guarded buffer so that its first byte sits `misalign` bytes
    past a 16-byte boundary.  front=False: the data ends within 16 bytes of the
    trailing guard page (exactly at it when the sizes allow); front=True: the
    buffer starts right after the leading guard page."""
    a = np.ascontiguousarray(arr)
    if front:
        emu.lib.emu_alloc_front.restype = ctypes.c_void_p
        emu.lib.emu_alloc_front.argtypes = [ctypes.c_size_t]
        p = emu.lib.emu_alloc_front(a.nbytes + misalign) + misalign
    else:
        # The buffer ends at a page boundary, so its start is -size (mod 16):
        # pad the size until the start lands `misalign` past a 16-byte boundary.
        pad = (-a.nbytes - misalign) % 16
        p = emu.lib.emu_alloc(a.nbytes + pad)
    assert p % 16 == misalign % 16
    ctypes.memmove(p, a.ctypes.data, a.nbytes)
    return p


def rows_with_stride(rows, cols, ld, dtype, fill):
    """A [rows, ld] buffer cut right after the last row's `cols` elements."""
    full = np.zeros((rows, ld), dtype=dtype)
    full[:, :cols] = fill
    return full.reshape(-1)[: (rows - 1) * ld + cols]


def set_schedule(emu, mode, seed=0):
    emu.lib.emu_set_schedule.argtypes = [ctypes.c_int, ctypes.c_uint64]
    emu.lib.emu_set_schedule(mode, seed)


def set_concurrency(emu, slots, reverse=False):
    emu.lib.emu_set_concurrency.argtypes = [ctypes.c_int, ctypes.c_int]
    emu.lib.emu_set_concurrency(slots, 1 if reverse else 0)
