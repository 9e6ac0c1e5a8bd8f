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
