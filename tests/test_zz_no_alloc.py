"""w4a16_linear_noalloc (the allocation-free variant of w4a16_linear, scratch
in a fixed per-GPU array of the library) against w4a16_linear on the same
inputs, through the C ABI: bit-equal, on consecutive calls whose second one is
smaller, on the decode and the GEMM path (run with -m gpu)."""

from __future__ import annotations

import ctypes
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _case(m, k, n, seed):
    from w4a16 import synth

    packed, scale = synth.make_weight(k, n, seed=seed, device=DEV)
    x = synth.make_activations(m, k, seed=seed + 1, device=DEV)
    return x, packed, scale


def _noalloc(x, packed, scale):
    from w4a16 import _native

    y = torch.full((x.shape[0], packed.shape[1]), float("nan"), dtype=torch.bfloat16, device=DEV)
    _native.linear_noalloc(x, packed, scale, y)
    return y


# (first call, second smaller call): decode split-K, batched decode, GEMM with
# split K and row sums, GEMM without split.
SEQUENCES = [
    ((1, 12288, 4096), (1, 4096, 1024)),
    ((32, 4096, 12288), (4, 4096, 4096)),
    ((512, 4096, 1024), (96, 1024, 512)),
    ((2048, 4096, 4096), (256, 4096, 4096)),
]


@pytest.mark.parametrize("first,second", SEQUENCES)
def test_noalloc_matches_linear_on_consecutive_calls(native_lib, first, second):
    from w4a16 import _native

    say(f"noalloc {first} then {second}")
    for rep, (m, k, n) in enumerate((first, second)):
        x, packed, scale = _case(m, k, n, seed=m + k + n)
        ref = _native.linear(x, packed, scale, 128)
        got = _noalloc(x, packed, scale)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (m, k, n, rep)
    # and once more in the other order: the smaller call leaves clean scratch for a larger one
    x, packed, scale = _case(*first, seed=sum(first))
    assert torch.equal(_noalloc(x, packed, scale), _native.linear(x, packed, scale, 128))


def test_noalloc_rejects_too_large_and_bad_args(native_lib):
    from w4a16 import _native as nat

    lib = native_lib
    big = 1 << 40  # never dereferenced: rejected before any launch
    # Decode M=32 over N=131072: split-K slots need ~100 MiB of scratch.
    assert lib.w4a16_linear_noalloc(big, 4096, big, 131072, big, 131072, big, 131072,
                                    32, 131072, 4096, 128, None) == nat.W4A16_ERR_TOO_LARGE
    assert lib.w4a16_linear_noalloc(big, 4096, big, 4096, big, 4096, big, 4096, 1, 4096, 4096, 64,
                                    None) == nat.W4A16_ERR_GROUP_SIZE
    assert lib.w4a16_linear_noalloc(None, 4096, big, 4096, big, 4096, big, 4096, 1, 4096, 4096, 128,
                                    None) == nat.W4A16_ERR_NULL
    assert lib.w4a16_linear_noalloc(None, 0, None, 0, None, 0, None, 0, 0, 16, 128, 128, None) == nat.W4A16_OK


def test_noalloc_captured_in_a_graph(native_lib):
    """The allocation-free call inside a HIP graph capture, replayed: equals eager."""
    from w4a16 import _native

    x, packed, scale = _case(1, 4096, 12288, seed=5)
    ref = _native.linear(x, packed, scale, 128)
    _noalloc(x, packed, scale)  # scratch set up eagerly on this device
    y = torch.empty(1, 12288, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _native.linear_noalloc(x, packed, scale, y)
    for _ in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref)


def test_noalloc_status_reports_and_clears_a_give_up(native_lib):
    """Host-forced give-ups (zero poll budget) inside w4a16_linear_noalloc: columns
    of a strip that gave up are NaN and noalloc_status() reports the bit; after it
    has cleared the scratch, calls are exact again and the status reads zero."""
    from w4a16 import _native

    x, packed, scale = _case(1, 12288, 4096, seed=61)  # down_proj shape: 24 splits at M=1
    ref = _native.linear(x, packed, scale, 128)
    torch.cuda.synchronize()
    assert _native.noalloc_status() == 0
    old = _native.set_spin_limit(0)
    gave_up = 0
    try:
        for _ in range(5):
            y = _noalloc(x, packed, scale)
            torch.cuda.synchronize()
            status = _native.noalloc_status()
            nan = torch.isnan(y.float())
            assert torch.equal(y[~nan], ref[~nan])
            if nan.any():
                assert status & _native.W4A16_STATUS_SPLITK_TIMEOUT
                gave_up += 1
            else:
                assert status == 0
    finally:
        _native.set_spin_limit(old)
    say(f"noalloc give-ups in 5 calls with a zero poll budget: {gave_up}")
    for _ in range(3):
        assert torch.equal(_noalloc(x, packed, scale), ref)
    assert _native.noalloc_status() == 0


def test_noalloc_wrapper_validates_y():
    from w4a16 import _native

    x, packed, scale = _case(2, 1024, 512, seed=3)
    for y in (torch.empty(2, 512, dtype=torch.float32, device=DEV),
              torch.empty(2, 256, dtype=torch.bfloat16, device=DEV),
              torch.empty(512, 2, dtype=torch.bfloat16, device=DEV).t()):
        with pytest.raises(ValueError):
            _native.linear_noalloc(x, packed, scale, y)
