"""The gfx950 kernels run on the CPU under the wave emulator (tests/native/emu).

inf-engine_amd/csrc/w4a16_kernels.hip is compiled as host C++ (three mechanical
rewrites, tests/native/emu/prepare.py) and linked with a fiber-per-thread wave
emulator; every entry point of the C ABI then runs the real kernel code on the
CPU.  These tests check, with no GPU:

* parity of every kernel family against the float64 oracle, at the bar of the
  GPU tests (oracle/tolerance.py), on shapes across every planner branch and
  the seeded random sweep of the GPU suite;
* memory safety: every buffer handed to a kernel ends at (or, for some cases,
  starts right after) an inaccessible page, so a kernel that reads or writes
  outside a buffer stops the run; operands off their natural alignment, row
  strides past the row and buffers cut right after the last row are included,
  and a negative control shows that the detection works;
* the workspace contract: the decode slot half is zero again after every call
  and the status word stays clear;
* determinism (two calls, identical bits);
* LDS: static arrays are per workgroup, poisoned and guarded like the dynamic
  LDS, and the two together must fit 160 KB (negative control);
* the GEMM's copy pipeline: direct-to-LDS copies land only at a wait that covers
  them, so a wait one operation short reads stale tiles (negative control);
* races inside a workgroup: results must not depend on the order in which the
  emulator runs the threads between meeting points (a decode kernel with its
  reduction barrier removed is the negative control);
* the raw-buffer range check read both ways (scalar offset counted or not) and
  cross-workgroup data read only through agent-coherent accesses (negative
  controls for both);
* the decode split-K protocol with every workgroup resident and interleaved,
  dispatched first-to-last and last-to-first (finishers then poll while their
  publishers run): identical bits, empty slots; and its give-up path, forced
  with a zero poll budget and finishers dispatched before their publishers;
* the kernel code under UndefinedBehaviorSanitizer (alignment of every vector
  access, signed overflow, shifts);
* the Python wrappers' operand marshalling, driven with CPU tensors.

What the emulator does not model (timing, caches and the store-to-load
ordering they allow between workgroups, the matrix cores' rounding order) is
covered by the GPU suite only.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

from oracle import int4_oracle as orc
from oracle.tolerance import assert_parity

from emu_harness import (KERNELS, ROOT, Emu, bf16_bits, bf16_value, build_emulator, clang, place, problem, reference,
                         rows_with_stride, run_linear, set_concurrency, set_schedule, ubsan_runtime)


@pytest.fixture(scope="module")
def emu(tmp_path_factory):
    if clang() is None:
        pytest.skip("clang++ not available")
    return Emu(build_emulator(str(tmp_path_factory.mktemp("emu"))))


@pytest.fixture(autouse=True)
def _release_buffers(request):
    """Unmap the guarded buffers a test allocated (the library stays loaded)."""
    yield
    if "emu" in request.fixturenames:
        request.getfixturevalue("emu").lib.emu_free_all()


# Shapes across the planner's branches: batch-1 decode, split / unsplit K,
# 4 and 8 waves, 64- and 128-column strips, M subtiles (<= 16, <= 32, <= 64),
# the GEMM (256- and 128-column tiles, two K halves, split K + reduce), odd N.
SHAPES = [
    (1, 128, 128), (1, 1024, 3072), (1, 4096, 1024), (1, 12288, 512), (2, 2048, 640), (4, 4096, 768),
    (8, 1024, 256), (13, 512, 200), (16, 4096, 1024), (17, 1024, 512), (24, 2048, 384), (32, 4096, 2048),
    (33, 512, 320), (48, 1024, 1000), (64, 2048, 512), (65, 512, 256), (100, 1024, 768),
    (128, 4096, 1024), (200, 512, 2048), (256, 1024, 4096), (300, 1536, 333),
]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_linear_matches_oracle(emu, m, k, n):
    xb, packed, scale = problem(m, k, n, seed=m * 7 + k + n, quantized=(m % 2 == 0))
    y = run_linear(emu, xb, packed, scale, m, k, n)
    assert_parity(bf16_value(y).astype(np.float64), reference(xb, packed, scale, m, k, n), f"emu M={m} K={k} N={n}")


@pytest.mark.parametrize("m", [1, 5, 24, 40, 130])
def test_linear_strided_unaligned_and_sliced(emu, m):
    """Row strides past K, activations off 16-byte alignment, column slices of
    wider weight and scale tensors (the generic-load paths)."""
    k, n = 1024, 300
    xb, packed, scale = problem(m, k, n, seed=90 + m, pad_x=24, pad_w=100)
    ref = reference(xb, packed, scale, m, k, n)
    for misalign in (False, True):
        # Slices: pass the wide tensors with the narrow n (row strides stay wide).
        y = run_linear(emu, xb if not misalign else xb[:, :k], packed, scale, m, k, n, misalign_x=misalign)
        assert_parity(bf16_value(y).astype(np.float64), ref, f"emu sliced M={m} misaligned={misalign}")


@pytest.mark.parametrize("m,k,n", [(1, 4096, 12288), (32, 12288, 1024), (2048, 512, 1024)])
def test_linear_full_size_shapes(emu, m, k, n):
    """Qwen3-8B gate at M = 1 (768 workgroups, 8-way split K), down's K at M = 32 (24 splits
    in 8-wave workgroups), and a prefill-sized GEMM (16 row tiles)."""
    xb, packed, scale = problem(m, k, n, seed=k + n, quantized=True)
    y = run_linear(emu, xb, packed, scale, m, k, n)
    assert_parity(bf16_value(y).astype(np.float64), reference(xb, packed, scale, m, k, n), f"emu M={m} K={k} N={n}")


SWEEP_SEED = 20261202


@pytest.mark.parametrize("case", range(32))
def test_random_shape_sweep(emu, case):
    """The GPU suite's seeded sweep (same shapes), on the emulator."""
    rng = np.random.default_rng(SWEEP_SEED + case)
    m = int(rng.choice([1, 2, 3, 5, 8, 13, 16, 17, 24, 31, 32, 33, 48, 64, 65, 96, 127, 128, 129, 200, 300]))
    k = 128 * int(rng.integers(1, 17))
    n = int(rng.integers(1, 2049))
    pad_x = int(rng.choice([0, 0, 8, 24]))
    pad_w = int(rng.choice([0, 0, 4, 100]))
    xb, packed, scale = problem(m, k, n, seed=SWEEP_SEED + case, pad_x=pad_x, pad_w=pad_w)
    y = run_linear(emu, xb, packed, scale, m, k, n)
    assert_parity(bf16_value(y).astype(np.float64), reference(xb, packed, scale, m, k, n),
                  f"emu sweep {case}: M={m} K={k} N={n} pad_x={pad_x} pad_w={pad_w}")


def test_deterministic(emu):
    xb, packed, scale = problem(4, 4096, 1024, seed=3)
    a = run_linear(emu, xb, packed, scale, 4, 4096, 1024)
    b = run_linear(emu, xb, packed, scale, 4, 4096, 1024)
    assert np.array_equal(a, b)


def test_grouped_matches_oracle(emu):
    """q/k/v-like problems sharing x, plus experts with their own M, decode and GEMM sized."""
    lib = emu.lib
    specs = [(3, 1024, 512, 0), (3, 1024, 128, 0), (3, 1024, 128, 0), (7, 512, 384, 1), (96, 512, 256, 2)]
    xs = {}
    table = (emu.Problem * len(specs))()
    outs, refs = [], []
    for i, (m, k, n, xid) in enumerate(specs):
        if xid not in xs:
            xb, _, _ = problem(m, k, n, seed=500 + xid)
            xs[xid] = (xb, emu.put(xb))
        xb, xp = xs[xid]
        _, packed, scale = problem(m, k, n, seed=600 + i, quantized=True)
        y = emu.zeros(m * n * 2)
        table[i] = emu.Problem(xp, k, emu.put(packed), n, emu.put(scale), n, y, n, m, n, k)
        outs.append((y, m, n))
        refs.append(reference(xb, packed, scale, m, k, n))
    nb = ctypes.c_size_t(0)
    assert lib.w4a16_workspace_size_grouped(table, len(specs), 128, ctypes.byref(nb)) == 0
    ws, size = emu.workspace(nb.value)
    assert lib.w4a16_linear_grouped(table, len(specs), 128, ws, size, None) == 0
    assert emu.slots_clear(ws, size)
    for (y, m, n), ref in zip(outs, refs):
        assert_parity(bf16_value(emu.get(y, (m, n), np.uint16)).astype(np.float64), ref, f"emu grouped M={m} N={n}")


@pytest.mark.parametrize("m,k,n", [(1, 1024, 1024), (5, 512, 384), (24, 1024, 256), (2048, 128, 2048), (256, 512, 1024), (130, 512, 200)])
def test_swiglu_matches_oracle(emu, m, k, n):
    """Decode pair kernel, the GEMM-sized pair kernel (256 tiles of 128 x 128: M=2048,
    N=2048) and the grouped-GEMM + elementwise fallback (too few tiles, or odd N)."""
    lib = emu.lib
    xb, gp, gs = problem(m, k, n, seed=800 + m, quantized=True)
    _, up, us = problem(m, k, n, seed=900 + m, quantized=True)
    nb = ctypes.c_size_t(0)
    assert lib.w4a16_workspace_size_swiglu(m, n, k, 128, ctypes.byref(nb)) == 0
    ws, size = emu.workspace(nb.value)
    h = emu.zeros(m * n * 2)
    rc = lib.w4a16_swiglu(emu.put(xb), k, emu.put(gp), n, emu.put(gs), n, emu.put(up), n, emu.put(us), n,
                          h, n, m, n, k, 128, ws, size, None)
    assert rc == 0
    xf = bf16_value(xb)
    ref = orc.swiglu_reference(xf, (gp, gs), (up, us))
    fallback = m > 64 and not (n % 128 == 0 and -(-m // 128) * (n // 128) >= 256)
    assert_parity(bf16_value(emu.get(h, (m, n), np.uint16)).astype(np.float64), ref, f"emu swiglu M={m} N={n}",
                  roundings=6 if fallback else 1)


@pytest.mark.parametrize("m,n,k", [(1, 1000, 4096), (3, 520, 1024), (4, 64, 640), (9, 200, 512), (16, 100, 1024)])
def test_bf16_gemv_matches_oracle(emu, m, n, k):
    rng = np.random.default_rng(m + n + k)
    xb = bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    wb = bf16_bits((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    y = emu.zeros(m * n * 2)
    assert emu.lib.w4a16_bf16_gemv(emu.put(xb), k, emu.put(wb), k, y, n, m, n, k, None) == 0
    ref = bf16_value(xb).astype(np.float64) @ bf16_value(wb).astype(np.float64).T
    assert_parity(bf16_value(emu.get(y, (m, n), np.uint16)).astype(np.float64), ref, f"emu gemv M={m} N={n} K={k}")


def test_dequant_bit_exact(emu):
    k, n = 512, 136
    rng = np.random.default_rng(11)
    packed = rng.integers(-128, 128, size=(k // 2, n), dtype=np.int8)
    scale = np.ldexp(np.float32(1.0), rng.integers(-6, 6, size=(k // 128, n))).astype(np.float32)
    pp, sp = emu.put(packed), emu.put(scale)
    out = emu.zeros(k * n * 4)
    assert emu.lib.w4a16_dequant(pp, n, sp, n, out, n, 0, k, n, 128, None) == 0
    assert np.array_equal(emu.get(out, (k, n), np.float32), orc.dequantize(packed, scale))
    out16 = emu.zeros(k * n * 2)
    assert emu.lib.w4a16_dequant(pp, n, sp, n, out16, n, 1, k, n, 128, None) == 0
    assert np.array_equal(emu.get(out16, (k, n), np.uint16), bf16_bits(orc.dequantize_bf16(packed, scale)))


def test_noalloc_matches_linear(emu):
    """The allocation-free entry point (its scratch is the emulated static array): calls in a
    row, smaller after larger and decode after GEMM, against w4a16_linear."""
    # A decode call after the GEMM: the GEMM's scratch (upper half) must leave the
    # decode slots (lower half) empty.
    for m, k, n in ((4, 4096, 2048), (2, 1024, 512), (96, 512, 256), (3, 4096, 1024)):
        xb, packed, scale = problem(m, k, n, seed=m + 1)
        ref = run_linear(emu, xb, packed, scale, m, k, n)
        y = emu.zeros(m * n * 2)
        rc = emu.lib.w4a16_linear_noalloc(emu.put(xb), k, emu.put(packed), n, emu.put(scale), n, y, n, m, n, k, 128, None)
        assert rc == 0
        assert np.array_equal(emu.get(y, (m, n), np.uint16), ref)


def test_guard_pages_catch_an_out_of_bounds_kernel(tmp_path, emu):
    """Negative control: an output buffer one row short makes the decode kernel's
    last row store land on the guard page, and the emulator reports it."""
    lib_path = emu.lib._name
    script = textwrap.dedent(f"""
        import ctypes, sys
        sys.path[:0] = [{ROOT!r}, {os.path.join(ROOT, 'tests')!r}]
        from emu_harness import Emu, problem
        emu = Emu({lib_path!r})
        m, k, n = 3, 512, 256
        xb, packed, scale = problem(m, k, n, seed=1)
        y = emu.zeros((m - 1) * n * 2)
        nb = ctypes.c_size_t(0)
        emu.lib.w4a16_workspace_size(m, n, k, 128, ctypes.byref(nb))
        ws, size = emu.workspace(nb.value)
        emu.lib.w4a16_linear(emu.put(xb), k, emu.put(packed), n, emu.put(scale), n, y, n, m, n, k, 128, ws, size, None)
        print("no fault")
    """)
    res = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=120)
    assert res.returncode == 97, (res.returncode, res.stdout, res.stderr)
    assert "memory access outside every buffer" in res.stderr and "gemv_kernel" in res.stderr, res.stderr


def test_late_lds_copies_are_modelled(tmp_path):
    """Negative control for the direct-to-LDS model: a GEMM whose copy wait leaves one
    operation too many outstanding (vmcnt(18) instead of 17) reads activation tiles
    before they land, and the emulated result is wrong."""
    if clang() is None:
        pytest.skip("clang++ not available")
    with open(KERNELS) as f:
        src = f.read()
    assert src.count("constexpr int kLoadsAfterA = 1 + 16;") == 1
    bad = tmp_path / "w4a16_short_wait.hip"
    bad.write_text(src.replace("constexpr int kLoadsAfterA = 1 + 16;", "constexpr int kLoadsAfterA = 1 + 17;"))
    emu = Emu(build_emulator(str(tmp_path), str(bad)))
    m, k, n = 256, 1024, 1024
    xb, packed, scale = problem(m, k, n, seed=5)
    y = run_linear(emu, xb, packed, scale, m, k, n)
    with pytest.raises(AssertionError):
        assert_parity(bf16_value(y).astype(np.float64), reference(xb, packed, scale, m, k, n), "short wait")


def test_range_check_reading_is_pinned(tmp_path):
    """Negative control for the range-check audit: a GEMM whose exhausted weight
    loads go past the buffer through the scalar offset (group G) rather than the
    per-lane offset reads zero if the hardware counts the scalar offset in its
    range check, and memory past the weights if it does not.  The emulator stops
    such an access, so the shipped kernels (which pass every test above) do not
    depend on that detail of the check."""
    if clang() is None:
        pytest.skip("clang++ not available")
    with open(KERNELS) as f:
        src = f.read()
    shipped = ("    const int g_next = has_next ? g + KW : g;\n"
               "    const uint32_t wv_next = (has_next || !w_small) ? wvoff : 0x80000000u;\n")
    assert src.count(shipped) == 1
    bad = tmp_path / "w4a16_soffset_oob.hip"
    bad.write_text(src.replace(shipped, "    const int g_next = has_next ? g + KW : G;\n"
                                        "    const uint32_t wv_next = wvoff;\n"))
    lib_path = build_emulator(str(tmp_path), str(bad))
    script = textwrap.dedent(f"""
        import sys
        sys.path[:0] = [{ROOT!r}, {os.path.join(ROOT, 'tests')!r}]
        from emu_harness import Emu, problem, run_linear
        emu = Emu({lib_path!r})
        m, k, n = 256, 512, 512
        xb, packed, scale = problem(m, k, n, seed=3)
        run_linear(emu, xb, packed, scale, m, k, n)
        print("no fault")
    """)
    res = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=300)
    assert res.returncode == 97, (res.returncode, res.stdout, res.stderr[-2000:])
    assert "soffset counted or not" in res.stderr and "gemm_kernel" in res.stderr, res.stderr[-2000:]


def test_cross_workgroup_reads_must_be_coherent(tmp_path):
    """Negative control for the coherence audit: a decode kernel whose split-K
    finisher polls the published slots with ordinary loads (no agent-coherence
    bit) could read a stale line of its own cache on the chip; the emulator,
    where every store is visible at once, stops it.  The shipped kernels pass
    the whole suite with the audit on."""
    if clang() is None:
        pytest.skip("clang++ not available")
    with open(KERNELS) as f:
        src = f.read()
    poll = "raw_buffer_load_b32(rs, off[j] + (uint32_t)(sp0 + i) * stride, 0, kAgentCoherent)"
    assert src.count(poll) == 2
    bad = tmp_path / "w4a16_plain_polls.hip"
    bad.write_text(src.replace(poll, poll.replace("kAgentCoherent", "0")))
    lib_path = build_emulator(str(tmp_path), str(bad))
    script = textwrap.dedent(f"""
        import sys
        sys.path[:0] = [{ROOT!r}, {os.path.join(ROOT, 'tests')!r}]
        from emu_harness import Emu, problem, run_linear
        emu = Emu({lib_path!r})
        m, k, n = 1, 4096, 512
        xb, packed, scale = problem(m, k, n, seed=3)
        run_linear(emu, xb, packed, scale, m, k, n)
        print("no fault")
    """)
    res = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=300)
    assert res.returncode == 97, (res.returncode, res.stdout, res.stderr[-2000:])
    assert "without agent-coherent accesses" in res.stderr and "gemv_kernel" in res.stderr, res.stderr[-2000:]


def test_lds_over_160_kb_is_caught(tmp_path):
    """Negative control for the LDS budget check: static LDS arrays are emulated per
    workgroup and counted with the dynamic LDS against the 160 KB a gfx950
    workgroup can hold.  Activation buffers grown by half fit the 4-wave GEMM
    (97 KB) but not the 8-wave two-K-half GEMM (194 KB), and the emulator stops it."""
    if clang() is None:
        pytest.skip("clang++ not available")
    with open(KERNELS) as f:
        src = f.read()
    decl = "__shared__ u32x4_t As0[KW * kATile], As1[KW * kATile];"
    assert src.count(decl) == 1
    bad = tmp_path / "w4a16_big_lds.hip"
    bad.write_text(src.replace(decl, "__shared__ u32x4_t As0[KW * kATile * 3 / 2], As1[KW * kATile * 3 / 2];"))
    lib_path = build_emulator(str(tmp_path), str(bad))
    script = textwrap.dedent(f"""
        import sys
        import numpy as np
        sys.path[:0] = [{ROOT!r}, {os.path.join(ROOT, 'tests')!r}]
        from emu_harness import Emu, problem, reference, run_linear, bf16_value
        from oracle.tolerance import assert_parity
        emu = Emu({lib_path!r})
        m, k, n = 256, 256, 1024      # 4-wave GEMM: fits
        xb, packed, scale = problem(m, k, n, seed=3)
        y = run_linear(emu, xb, packed, scale, m, k, n)
        assert_parity(bf16_value(y).astype(np.float64), reference(xb, packed, scale, m, k, n), "fits")
        print("4-wave ok", flush=True)
        m, k, n = 128, 128, 192 * 256  # 192 tiles of 128 x 256: the 8-wave GEMM
        xb, packed, scale = problem(m, k, n, seed=4)
        run_linear(emu, xb, packed, scale, m, k, n)
        print("no fault")
    """)
    res = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=300)
    assert res.returncode == 97 and "4-wave ok" in res.stdout, (res.returncode, res.stdout, res.stderr[-2000:])
    assert "exceeds 160 KB" in res.stderr and "gemm_kernel" in res.stderr, res.stderr[-2000:]


SCHEDULE_SHAPES = [(1, 1024, 512), (3, 4096, 1024), (16, 2048, 512), (24, 1024, 640), (40, 512, 320),
                   (130, 512, 256), (256, 1024, 512), (200, 512, 333)]


def test_results_do_not_depend_on_thread_schedule(emu):
    """Race check inside workgroups: the emulator runs each workgroup's threads in
    ascending, descending and two pseudo-random orders between meeting points.  A
    read of LDS written by another thread without a barrier in between would see
    different data under some order; every kernel must give identical bits."""
    try:
        for m, k, n in SCHEDULE_SHAPES:
            xb, packed, scale = problem(m, k, n, seed=m)
            outs = []
            for i, mode in enumerate((0, 1, 2, 2)):
                set_schedule(emu, mode, 7 + i)
                outs.append(run_linear(emu, xb, packed, scale, m, k, n))
            for o in outs[1:]:
                assert np.array_equal(outs[0], o), f"schedule-dependent result at M={m} K={k} N={n}"
    finally:
        set_schedule(emu, 0)


def test_schedule_check_finds_a_missing_barrier(tmp_path):
    """Negative control: without the barrier between the decode kernel's LDS
    stores of wave totals and their sum, the result depends on the schedule."""
    if clang() is None:
        pytest.skip("clang++ not available")
    with open(KERNELS) as f:
        src = f.read()
    barrier = "      }\n    }\n  __syncthreads();\n  const int elems = M * WCOLS;"
    assert src.count(barrier) == 1
    bad = tmp_path / "w4a16_no_barrier.hip"
    bad.write_text(src.replace(barrier, "      }\n    }\n  const int elems = M * WCOLS;"))
    emu = Emu(build_emulator(str(tmp_path), str(bad)))
    m, k, n = 3, 4096, 1024
    xb, packed, scale = problem(m, k, n, seed=m)
    set_schedule(emu, 0)
    a = run_linear(emu, xb, packed, scale, m, k, n)
    set_schedule(emu, 1)
    b = run_linear(emu, xb, packed, scale, m, k, n)
    assert not np.array_equal(a, b)


@pytest.mark.parametrize("case", range(24))
def test_guarded_misaligned_operands(emu, case):
    """Random shapes with operands off their natural alignment, row strides past the
    row, buffers cut right after the last row, and the guard page before or after
    every buffer: no kernel may touch a byte outside its operands."""
    rng = np.random.default_rng(1000 + case)
    m = int(rng.choice([1, 2, 3, 4, 7, 8, 12, 16, 17, 23, 32, 33, 40, 63, 64, 65, 100, 128, 129, 200, 257]))
    k = 128 * int(rng.integers(1, 25))
    n = int(rng.integers(1, 2200))
    front = bool(rng.integers(0, 2))
    ldx = k + int(rng.choice([0, 0, 1, 8, 13]))
    ldp = n + int(rng.choice([0, 0, 1, 16, 33]))
    lds = n + int(rng.choice([0, 0, 1, 4, 7]))
    ldy = n + int(rng.choice([0, 0, 1, 4]))
    mx, mp, ms, my = (int(rng.choice(c)) for c in ([0, 0, 2, 6, 8], [0, 0, 1, 4, 8, 12], [0, 0, 4, 8, 12], [0, 0, 2, 4, 6]))
    packed = rng.integers(-128, 128, size=(k // 2, n), dtype=np.int8)
    scale = (rng.random((k // 128, n), dtype=np.float32) * 0.01 + 0.001).astype(np.float32)
    xb = bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    xp = place(emu, rows_with_stride(m, k, ldx, np.uint16, xb), mx, front)
    pp = place(emu, rows_with_stride(k // 2, n, ldp, np.int8, packed), mp, front)
    sp = place(emu, rows_with_stride(k // 128, n, lds, np.float32, scale), ms, front)
    ylen = (m - 1) * ldy + n
    yp = place(emu, np.zeros(ylen, np.uint16), my, front)
    nb = ctypes.c_size_t(0)
    assert emu.lib.w4a16_workspace_size(m, n, k, 128, ctypes.byref(nb)) == 0
    ws, size = emu.workspace(nb.value)
    desc = f"M={m} K={k} N={n} ld={ldx},{ldp},{lds},{ldy} misalign={mx},{mp},{ms},{my} front={front}"
    assert emu.lib.w4a16_linear(xp, ldx, pp, ldp, sp, lds, yp, ldy, m, n, k, 128, ws, size, None) == 0, desc
    flat = np.frombuffer(ctypes.string_at(yp, ylen * 2), np.uint16)
    y = np.stack([flat[r * ldy: r * ldy + n] for r in range(m)])
    assert_parity(bf16_value(y).astype(np.float64), orc.fused_reference(bf16_value(xb), packed, scale), desc)
    assert emu.slots_clear(ws, size), desc


# Decode launches with split K: (M, K, N) -> workgroups (strips x splits).
SPLIT_K_SHAPES = [(1, 4096, 512), (1, 12288, 256), (4, 4096, 384), (16, 2048, 512), (24, 2048, 640), (40, 1024, 256)]


@pytest.mark.parametrize("reverse", [False, True])
def test_gemm_with_resident_workgroups(emu, reverse):
    """The GEMM path (row sums, GEMM with and without K split, the split-K reduce)
    with every workgroup resident and interleaved: the same bits as one at a time."""
    try:
        for m, k, n in ((130, 512, 256), (256, 1024, 512), (200, 512, 333)):
            xb, packed, scale = problem(m, k, n, seed=m + n, quantized=True)
            set_concurrency(emu, 1)
            seq = run_linear(emu, xb, packed, scale, m, k, n)
            set_concurrency(emu, 4096, reverse)
            assert np.array_equal(seq, run_linear(emu, xb, packed, scale, m, k, n)), (m, k, n, reverse)
    finally:
        set_concurrency(emu, 1)


@pytest.mark.parametrize("reverse", [False, True])
def test_split_k_with_resident_workgroups(emu, reverse):
    """Every workgroup of a decode launch resident at once and interleaved at each
    meeting point, dispatched first-to-last or last-to-first: split-K finishers
    poll while their publishers still run.  Results must equal the one-at-a-time
    run bit for bit (partials are summed in split order, not arrival order), and
    the slots must be empty again."""
    try:
        for m, k, n in SPLIT_K_SHAPES:
            xb, packed, scale = problem(m, k, n, seed=m + k + n, quantized=True)
            set_concurrency(emu, 1)
            seq = run_linear(emu, xb, packed, scale, m, k, n)
            set_concurrency(emu, 4096, reverse)
            conc = run_linear(emu, xb, packed, scale, m, k, n)
            assert np.array_equal(seq, conc), f"M={m} K={k} N={n} reverse={reverse}"
        # The SwiGLU pair: every gate workgroup publishes, up's finishers sum both.
        m, k, n = 3, 2048, 512
        xb, gp, gs = problem(m, k, n, seed=71, quantized=True)
        _, up, us = problem(m, k, n, seed=72, quantized=True)
        nb = ctypes.c_size_t(0)
        assert emu.lib.w4a16_workspace_size_swiglu(m, n, k, 128, ctypes.byref(nb)) == 0
        outs = []
        for slots in (1, 4096):
            set_concurrency(emu, slots, reverse and slots > 1)
            ws, size = emu.workspace(nb.value)
            h = emu.zeros(m * n * 2)
            assert emu.lib.w4a16_swiglu(emu.put(xb), k, emu.put(gp), n, emu.put(gs), n, emu.put(up), n,
                                        emu.put(us), n, h, n, m, n, k, 128, ws, size, None) == 0
            assert emu.slots_clear(ws, size)
            outs.append(emu.get(h, (m, n), np.uint16))
        assert np.array_equal(outs[0], outs[1])
    finally:
        set_concurrency(emu, 1)


def test_split_k_give_up_path(emu):
    """The finisher's bounded poll, forced: finishers dispatched before their
    publishers (last-first, one at a time) with a zero poll budget give up.  Their
    outputs are NaN, the status word says so, the late publishers leave their
    slots set (the workspace must be zeroed before reuse), and every kernel ends.
    A zeroed workspace then gives exact results again."""
    lib = emu.lib
    lib.w4a16_debug_set_spin_limit.argtypes = [ctypes.c_uint32]
    lib.w4a16_debug_set_spin_limit.restype = ctypes.c_uint32
    m, k, n = 1, 4096, 512
    xb, packed, scale = problem(m, k, n, seed=5, quantized=True)
    ref = run_linear(emu, xb, packed, scale, m, k, n)
    nb = ctypes.c_size_t(0)
    assert lib.w4a16_workspace_size(m, n, k, 128, ctypes.byref(nb)) == 0
    ws, size = emu.workspace(nb.value)
    xp, pp, sp = emu.put(xb), emu.put(packed), emu.put(scale)
    old = lib.w4a16_debug_set_spin_limit(0)
    try:
        set_concurrency(emu, 1, reverse=True)
        y = emu.zeros(m * n * 2)
        assert lib.w4a16_linear(xp, k, pp, n, sp, n, y, n, m, n, k, 128, ws, size, None) == 0
    finally:
        lib.w4a16_debug_set_spin_limit(old)
        set_concurrency(emu, 1)
    out = emu.get(y, (m, n), np.uint16)
    assert (out == 0x7FC0).all()  # every strip's finisher ran before its publishers
    off = ctypes.c_size_t(0)
    assert lib.w4a16_status_offset(size, ctypes.byref(off)) == 0
    assert emu.get(ws + off.value, (1,), np.uint32)[0] & 1  # W4A16_STATUS_SPLITK_TIMEOUT
    assert not emu.slots_clear(ws, size)
    ctypes.memset(ws, 0, size)
    y2 = emu.zeros(m * n * 2)
    assert lib.w4a16_linear(xp, k, pp, n, sp, n, y2, n, m, n, k, 128, ws, size, None) == 0
    assert np.array_equal(emu.get(y2, (m, n), np.uint16), ref)
    assert emu.slots_clear(ws, size)


def test_noalloc_give_up_is_reported_and_cleared(emu):
    """A forced give-up inside w4a16_linear_noalloc leaves NaN outputs, a set status
    word and late partials in the shared scratch; w4a16_noalloc_status reports the
    bit once, zeroes the scratch, and the next call is exact again."""
    lib = emu.lib
    lib.w4a16_debug_set_spin_limit.argtypes = [ctypes.c_uint32]
    lib.w4a16_debug_set_spin_limit.restype = ctypes.c_uint32
    m, k, n = 2, 4096, 512
    xb, packed, scale = problem(m, k, n, seed=9, quantized=True)
    ref = run_linear(emu, xb, packed, scale, m, k, n)
    xp, pp, sp = emu.put(xb), emu.put(packed), emu.put(scale)
    st = ctypes.c_uint32(7)
    assert lib.w4a16_noalloc_status(None, ctypes.byref(st)) == 0 and st.value == 0
    old = lib.w4a16_debug_set_spin_limit(0)
    try:
        set_concurrency(emu, 1, reverse=True)
        y = emu.zeros(m * n * 2)
        assert lib.w4a16_linear_noalloc(xp, k, pp, n, sp, n, y, n, m, n, k, 128, None) == 0
    finally:
        lib.w4a16_debug_set_spin_limit(old)
        set_concurrency(emu, 1)
    assert (emu.get(y, (m, n), np.uint16) == 0x7FC0).all()
    # Without the reset the late partials would be summed into the next call.
    assert lib.w4a16_noalloc_status(None, ctypes.byref(st)) == 0 and st.value == 1
    assert lib.w4a16_noalloc_status(None, ctypes.byref(st)) == 0 and st.value == 0
    for _ in range(2):
        y2 = emu.zeros(m * n * 2)
        assert lib.w4a16_linear_noalloc(xp, k, pp, n, sp, n, y2, n, m, n, k, 128, None) == 0
        assert np.array_equal(emu.get(y2, (m, n), np.uint16), ref)
    assert lib.w4a16_noalloc_status(None, ctypes.byref(st)) == 0 and st.value == 0


def test_noalloc_first_call_under_capture_is_refused(tmp_path, emu):
    """In a fresh process, a first no-alloc call made while the stream captures a
    graph returns W4A16_ERR_CAPTURING and launches nothing (its zero fill would
    become a 96 MiB node of the graph); after one eager call, calls under capture
    go through.  The status reader is refused under capture too."""
    lib_path = emu.lib._name
    script = textwrap.dedent(f"""
        import ctypes, sys
        import numpy as np
        sys.path[:0] = [{ROOT!r}, {os.path.join(ROOT, 'tests')!r}]
        from emu_harness import Emu, problem, run_linear
        emu = Emu({lib_path!r})
        lib = emu.lib
        m, k, n = 1, 4096, 512
        xb, packed, scale = problem(m, k, n, seed=4, quantized=True)
        ref = run_linear(emu, xb, packed, scale, m, k, n)
        args = lambda y: (emu.put(xb), k, emu.put(packed), n, emu.put(scale), n, y, n, m, n, k, 128, None)
        st = ctypes.c_uint32(0)
        lib.emu_set_capturing(1)
        y = emu.zeros(m * n * 2)
        assert lib.w4a16_linear_noalloc(*args(y)) == 9
        assert not emu.get(y, (m, n), np.uint16).any()
        assert lib.w4a16_noalloc_status(None, ctypes.byref(st)) == 9
        lib.emu_set_capturing(0)
        assert lib.w4a16_linear_noalloc(*args(y)) == 0
        assert np.array_equal(emu.get(y, (m, n), np.uint16), ref)
        lib.emu_set_capturing(1)
        y = emu.zeros(m * n * 2)
        assert lib.w4a16_linear_noalloc(*args(y)) == 0
        assert np.array_equal(emu.get(y, (m, n), np.uint16), ref)
        lib.emu_set_capturing(0)
        assert lib.w4a16_noalloc_status(None, ctypes.byref(st)) == 0 and st.value == 0
        print("capture rule ok")
    """)
    res = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and "capture rule ok" in res.stdout, res.stdout[-2000:] + res.stderr[-3000:]


def test_give_up_costs_one_poll_budget(emu):
    """A finisher that gives up waits one poll budget in all, not one per chunk of
    slots: with every finisher dispatched before its publishers, the buffer loads
    added by raising the budget are the same for 8 published slots (one chunk) as
    for 17 or 23 (three chunks).  Counted over the whole launch; the slope is
    4 strips x 64 lanes x 8 polls per round."""
    lib = emu.lib
    lib.w4a16_debug_set_spin_limit.argtypes = [ctypes.c_uint32]
    lib.w4a16_debug_set_spin_limit.restype = ctypes.c_uint32
    m, n = 1, 256
    slopes = []
    old = lib.w4a16_debug_set_spin_limit(0)
    try:
        set_concurrency(emu, 1, reverse=True)
        for k in (4608, 9216, 12288):  # 9, 18 and 24 K splits
            xb, packed, scale = problem(m, k, n, seed=1, quantized=True)
            nb = ctypes.c_size_t(0)
            assert lib.w4a16_workspace_size(m, n, k, 128, ctypes.byref(nb)) == 0
            loads = []
            for budget in (0, 100):
                ws, size = emu.workspace(nb.value)
                lib.w4a16_debug_set_spin_limit(budget)
                y = emu.zeros(m * n * 2)
                lib.emu_reset_load_count()
                assert lib.w4a16_linear(emu.put(xb), k, emu.put(packed), n, emu.put(scale), n, y, n, m, n, k, 128,
                                        ws, size, None) == 0
                loads.append(lib.emu_load_count())
                assert (emu.get(y, (m, n), np.uint16) == 0x7FC0).all()
            slopes.append(loads[1] - loads[0])
    finally:
        lib.w4a16_debug_set_spin_limit(old)
        set_concurrency(emu, 1)
    assert slopes == [4 * 64 * 8 * 100] * 3, slopes


def test_kernels_under_undefined_behavior_sanitizer(tmp_path):
    """The kernel code built with UndefinedBehaviorSanitizer (alignment of every
    vector access, signed overflow, shifts) on planner-branch shapes, the
    misaligned-operand cases and every other entry point, in a child process
    so that a finding (which aborts) fails this test with its report."""
    if clang() is None or ubsan_runtime() is None:
        pytest.skip("clang++ with the UBSan runtime not available")
    lib = build_emulator(str(tmp_path), ubsan=True)
    script = textwrap.dedent(f"""
        import sys
        sys.path[:0] = [{ROOT!r}, {os.path.join(ROOT, 'tests')!r}]
        import test_emulated_kernels as T
        emu = T.Emu({lib!r})
        for m, k, n in T.SHAPES[::2]:
            T.test_linear_matches_oracle(emu, m, k, n)
        for m in (5, 40):
            T.test_linear_strided_unaligned_and_sliced(emu, m)
        for case in range(24):
            T.test_guarded_misaligned_operands(emu, case)
        T.test_grouped_matches_oracle(emu)
        for a in [(5, 512, 384), (256, 512, 1024), (130, 512, 200)]:
            T.test_swiglu_matches_oracle(emu, *a)
        for a in [(1, 1000, 4096), (9, 200, 512)]:
            T.test_bf16_gemv_matches_oracle(emu, *a)
        T.test_dequant_bit_exact(emu)
        T.test_noalloc_matches_linear(emu)
        print("ubsan clean")
    """)
    res = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=900)
    assert res.returncode == 0 and "ubsan clean" in res.stdout, res.stdout[-2000:] + res.stderr[-4000:]


@pytest.fixture
def wrappers_on_emulator(emu, monkeypatch):
    """w4a16._native bound to the emulated library, driven with CPU tensors: the
    wrappers' view handling (row strides, overlapping rows, column slices,
    unaligned rows, grouped tables, SwiGLU operand order) runs unchanged and the
    kernels read host memory."""
    from types import SimpleNamespace

    import torch

    from w4a16 import _native

    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "LIB_PATH", emu.lib._name)
    monkeypatch.setattr(_native, "_workspaces", {})
    monkeypatch.setattr(_native, "_retired", [])
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: SimpleNamespace(cuda_stream=0))
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    yield _native
    _native._lib = None  # the next load_library() loads the real library again


def _torch_problem(m, k, n, seed):
    import torch

    g = torch.Generator().manual_seed(seed)
    packed = torch.randint(-128, 128, (k // 2, n), generator=g, dtype=torch.int8)
    scale = torch.rand(k // 128, n, generator=g) * 0.01 + 0.001
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    return x, packed, scale


def _ref(x, packed, scale):
    return orc.fused_reference(x.float().numpy(), packed.numpy(), scale.numpy())


def test_wrappers_handle_views(wrappers_on_emulator):
    import torch

    nat = wrappers_on_emulator
    k, n = 1024, 384
    for m in (1, 5, 40, 130):
        x, packed, scale = _torch_problem(m, k, n, seed=m)
        ref = _ref(x, packed, scale)
        views = {
            "contiguous": x,
            "row stride K+8": torch.nn.functional.pad(x, (0, 8))[:, :k],
            "row stride K+3": torch.nn.functional.pad(x, (0, 3))[:, :k],
            "pointer off alignment": torch.cat([torch.zeros(1, dtype=x.dtype), x.reshape(-1)])[1:].view(m, k),
            "transposed": x.t().contiguous().t(),
        }
        for name, v in views.items():
            y = nat.linear(v, packed, scale, 128)
            assert_parity(y.float().numpy().astype(np.float64), ref, f"linear M={m} {name}")
        wide_p = torch.nn.functional.pad(packed, (0, 16))
        wide_s = torch.nn.functional.pad(scale, (0, 4))
        y = nat.linear(x, wide_p[:, :n], wide_s[:, :n], 128)
        assert_parity(y.float().numpy().astype(np.float64), ref, f"linear M={m} column-sliced weights")
    x1, packed, scale = _torch_problem(1, k, n, seed=99)
    y = nat.linear(x1[0].expand(6, k), packed, scale, 128)  # overlapping rows (row stride 0)
    assert_parity(y.float().numpy().astype(np.float64), np.repeat(_ref(x1, packed, scale), 6, axis=0), "expand")


def test_wrappers_grouped_swiglu_and_gemv(wrappers_on_emulator):
    import torch

    nat = wrappers_on_emulator
    k = 512
    x, p0, s0 = _torch_problem(36, k, 256, seed=1)
    _, p1, s1 = _torch_problem(36, k, 128, seed=2)
    xo = torch.cat([torch.zeros(1, dtype=x.dtype), x.reshape(-1)])[1:].view(36, k)  # shared, unaligned
    outs = nat.linear_grouped([xo, xo], [(p0, s0), (p1, s1)], 128)
    for y, (p, s) in zip(outs, [(p0, s0), (p1, s1)]):
        assert_parity(y.float().numpy().astype(np.float64), _ref(x, p, s), "grouped shared unaligned x")
    for m in (3, 130):
        xs, gp, gs = _torch_problem(m, k, 256, seed=10 + m)
        _, up, us = _torch_problem(m, k, 256, seed=20 + m)
        h = nat.swiglu(xs, (gp, gs), (up, us), 128)
        ref = orc.swiglu_reference(xs.float().numpy(), (gp.numpy(), gs.numpy()), (up.numpy(), us.numpy()))
        assert_parity(h.float().numpy().astype(np.float64), ref, f"swiglu M={m}", roundings=1 if m <= 64 else 6)
    g = torch.Generator().manual_seed(5)
    xg = torch.randn(3, 1024, generator=g).to(torch.bfloat16)
    w = (torch.randn(200, 1024, generator=g) * 0.02).to(torch.bfloat16)
    xg_off = torch.cat([torch.zeros(1, dtype=xg.dtype), xg.reshape(-1)])[1:].view(3, 1024)
    y = nat.bf16_gemv(xg_off, w)  # unaligned rows are copied for the GEMV
    ref = xg.double().numpy() @ w.double().numpy().T
    assert_parity(y.float().numpy().astype(np.float64), ref, "bf16_gemv unaligned x")


def test_integration_ctypes_stub_runs_on_the_emulator(emu, monkeypatch):
    """The Option B ctypes stub of INTEGRATION.md, executed as written against the
    emulated library with CPU tensors: outputs match the oracle, and its workspace
    bookkeeping follows the capture rule (a buffer born in one capture gets a fill
    recorded by each other capture that uses it, once; an eager call zeroes it)."""
    import re
    from types import SimpleNamespace

    import torch

    with open(os.path.join(ROOT, "INTEGRATION.md")) as f:
        text = f.read()
    stub = next(b for b in re.findall(r"```python\n(.*?)```", text, re.S) if "def int4_matmul_device" in b)
    assert stub.count('"/path/to/libw4a16.so"') == 1
    stub = stub.replace('"/path/to/libw4a16.so"', repr(emu.lib._name))
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: SimpleNamespace(cuda_stream=0))
    ns: dict = {}
    exec(compile(stub, "INTEGRATION.md", "exec"), ns)
    for m, k, n in ((1, 4096, 512), (3, 1024, 384), (40, 512, 256)):
        x, packed, scale = _torch_problem(m, k, n, seed=m)
        y = ns["int4_matmul_device"](x, packed, scale)
        assert_parity(y.float().numpy().astype(np.float64), _ref(x, packed, scale), f"stub M={m} K={k} N={n}")
    # Capture bookkeeping (on the CPU a recorded fill runs at once, which makes it visible).
    x, packed, scale = _torch_problem(1, 4096, 512, seed=7)
    ref = _ref(x, packed, scale)
    ns["_ws"].clear()
    try:
        emu.lib.emu_set_capturing(5)
        ns["int4_matmul_device"](x, packed, scale)
        entry = ns["_ws"][(None, 0)]
        assert entry[1] is False and entry[2] == {5}
        entry[0].fill_(0x55)
        emu.lib.emu_set_capturing(6)  # another capture reuses the buffer: its own fill first
        y = ns["int4_matmul_device"](x, packed, scale)
        assert entry[2] == {5, 6}
        assert_parity(y.float().numpy().astype(np.float64), ref, "stub, second capture")
    finally:
        emu.lib.emu_set_capturing(0)
    entry[0].fill_(0x55)
    y = ns["int4_matmul_device"](x, packed, scale)  # eager: zeroed first
    assert entry[1] is True
    assert_parity(y.float().numpy().astype(np.float64), ref, "stub, eager after captures")
