"""GPU checks of the drop-in contract around the kernels (run with -m gpu):

* the reference's own HIP-graph capture pattern (engine/llama_paged_engine.py:
  315-347: warm up on a fresh side stream, then ``torch.cuda.graph(g)`` with no
  stream argument), several buckets kept alive, then larger eager calls that
  grow the workspaces, then replays that must match eager bit for bit;
* device-side quantization bit-exact against the oracle (the reference
  quantizes on the GPU for models up to 8B, main.py:474-478);
* the split-K finisher's bounded poll: forced from the host with a zero poll
  budget, a give-up writes NaN and sets the workspace status word, and the
  wrapper restores a clean workspace.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import int4_oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu(native_lib):
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    yield


def _int4_weight(k, n, seed):
    from w4a16 import _Int4Weight, synth

    packed, scale = synth.make_weight(k, n, seed=seed, device=DEV)
    return _Int4Weight(packed, scale, 128, (n, k))


def test_reference_graph_capture_pattern_with_growing_workspaces():
    from w4a16 import _native, linear, synth

    # Buckets of rising M: decode (split-K slots), batched decode, GEMM with
    # split K (k/v shape at M=128) -- each needs a larger workspace than the last.
    wq = _int4_weight(4096, 4096, seed=1)
    wk = _int4_weight(4096, 1024, seed=2)
    wg = _int4_weight(4096, 12288, seed=3)
    buckets = [1, 4, 16, 32, 128]
    xs = {m: synth.make_activations(m, 4096, seed=10 + m, device=DEV).reshape(1, m, 4096) for m in buckets}

    def forward(x):
        return [linear(x, wq), linear(x, wk), linear(x, wg)]

    eager = {m: forward(xs[m]) for m in buckets}
    torch.cuda.synchronize()
    graphs = {}
    for m in buckets:
        say(f"capture bucket M={m}")
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                forward(xs[m])
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):  # torch's default capture stream, as the reference
            outs = forward(xs[m])
        graphs[m] = (graph, outs)
    # Eager calls larger than every bucket, on the current stream and on the
    # capture stream itself: both workspaces grow past what the graphs hold.
    big = synth.make_activations(1024, 4096, seed=99, device=DEV)
    big_ref = forward(big)
    cap = torch.cuda.graphs.graph.default_capture_stream
    if cap is not None:
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap):
            big_cap = forward(big)
        torch.cuda.current_stream().wait_stream(cap)
        torch.cuda.synchronize()
        for a, b in zip(big_cap, big_ref):
            assert torch.equal(a, b)
    torch.cuda.synchronize()
    assert _native.workspace_status() == 0
    for rep in range(3):
        # Allocate and scribble over freed memory between replays.
        junk = [torch.full((1 << 22,), 7, dtype=torch.int32, device=DEV) for _ in range(8)]
        for m in reversed(buckets):
            graph, outs = graphs[m]
            for o in outs:
                o.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for i, (o, e) in enumerate(zip(outs, eager[m])):
                assert torch.equal(o, e), f"replay {rep} bucket M={m} projection {i}"
        del junk
    assert _native.workspace_status() == 0


def test_capture_first_use_of_a_stream_and_eager_after():
    """A stream whose first call is inside a capture gets its workspace from
    the capture; eager calls on it afterwards (before any replay) still work."""
    from w4a16 import int4_matmul, synth

    packed, scale = synth.make_weight(4096, 12288, seed=21, device=DEV)
    x = synth.make_activations(1, 4096, seed=22, device=DEV)
    ref = int4_matmul(x, packed, scale)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = int4_matmul(x, packed, scale)
    with torch.cuda.stream(s):
        y = int4_matmul(x, packed, scale)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


def test_device_scalar_division_rule():
    """What oracle.quantize(device_division=True) assumes of torch on the GPU:
    tensor / 7 is tensor * float32(1/7), and tensor / tensor is a true
    (correctly rounded) division."""
    t = torch.rand(1 << 20, generator=torch.Generator().manual_seed(3)) * 0.2
    d = torch.rand(1 << 20, generator=torch.Generator().manual_seed(4)) + 0.01
    got = (t.to(DEV) / 7).cpu().numpy()
    tn = t.numpy()
    np.testing.assert_array_equal(got, (tn * (np.float32(1.0) / np.float32(7.0))).astype(np.float32))
    assert (got != (tn / np.float32(7.0))).any()  # the rule is visible on this sample
    np.testing.assert_array_equal((t.to(DEV) / d.to(DEV)).cpu().numpy(), (tn / d.numpy()).astype(np.float32))


@pytest.mark.parametrize("k,n,seed", [(4096, 12288, 0), (12288, 4096, 1), (1024, 3072, 2)])
def test_device_quantize_bit_exact_vs_oracle(k, n, seed):
    """quantize_weight_int4 on cuda tensors: the oracle's bytes and scales
    under torch's device division rule."""
    from w4a16 import quantize_weight_int4

    say(f"device quantize K={k} N={n}")
    gen = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16).T.contiguous().float()
    p, s = quantize_weight_int4(w.to(DEV), 128)
    po, so = orc.quantize(w.numpy(), 128, device_division=True)
    np.testing.assert_array_equal(p.cpu().numpy(), po)
    np.testing.assert_array_equal(s.cpu().numpy(), so)


def test_device_quantize_ties_and_amax():
    from w4a16 import quantize_weight_int4

    col = np.zeros(128, dtype=np.float32)
    col[:8] = [7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]
    w = np.random.default_rng(3).standard_normal((256, 16)).astype(np.float32)
    w[5, 3] = -50.0
    for arr in (col.reshape(128, 1), w):
        p, s = quantize_weight_int4(torch.from_numpy(arr).to(DEV), 128)
        po, so = orc.quantize(arr, 128, device_division=True)
        np.testing.assert_array_equal(p.cpu().numpy(), po)
        np.testing.assert_array_equal(s.cpu().numpy(), so)
    p, _ = quantize_weight_int4(torch.from_numpy(col.reshape(128, 1)).to(DEV), 128)
    assert orc.codes(p.cpu().numpy())[:8, 0].tolist() == [7, 0, 2, 2, 0, -2, -2, 4]


def test_capture_born_workspace_replays_in_any_order():
    """Two decode buckets captured one after the other on a fresh stream, so the
    stream's workspace is born inside the first capture and reused by the second.
    The buffer is then poisoned and the second graph replayed before the first has
    ever run: its own recorded fill must give outputs bit-equal to eager."""
    from w4a16 import _native, int4_matmul, synth

    packed, scale = synth.make_weight(4096, 12288, seed=41, device=DEV)
    xs = {m: synth.make_activations(m, 4096, seed=42 + m, device=DEV) for m in (1, 4)}
    eager = {m: int4_matmul(xs[m], packed, scale) for m in xs}
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    graphs = {}
    for m in (4, 1):  # the larger need first, so the second capture reuses the buffer
        say(f"capture-born workspace: capture M={m}")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = int4_matmul(xs[m], packed, scale)
        graphs[m] = (g, out)
    ws = _native._workspaces[(torch.device(DEV).index or 0, s.cuda_stream)]
    assert ws.captured and not ws.defined and len(ws.filled_in) == 2
    for order in ((1, 4), (4, 1)):
        ws.tensor.fill_(0x55)  # what a pool buffer may hold before any fill ran
        torch.cuda.synchronize()
        for m in order:
            g, out = graphs[m]
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager[m]), f"replay order {order}, M={m}"
    assert _native.workspace_status() == 0


def test_splitk_give_up_sets_status_and_workspace_recovers():
    """Zero poll budget (host-forced): each finisher either sees every slot on
    its first poll or gives up at once.  Every kernel ends normally.  Columns of
    a strip that gave up are NaN and the status word says so; after
    workspace_status() has cleaned the workspace, calls are exact again."""
    from w4a16 import _native, int4_matmul, synth

    packed, scale = synth.make_weight(12288, 4096, seed=31, device=DEV)  # down_proj: 24 splits at M=1
    x = synth.make_activations(1, 12288, seed=32, device=DEV)
    ref = int4_matmul(x, packed, scale)
    torch.cuda.synchronize()
    assert _native.workspace_status() == 0
    old = _native.set_spin_limit(0)
    gave_up = 0
    try:
        for _ in range(5):
            y = int4_matmul(x, packed, scale)
            torch.cuda.synchronize()
            status = _native.workspace_status()
            nan = torch.isnan(y.float())
            ok = ~nan
            assert torch.equal(y[ok], ref[ok])
            if nan.any():
                assert status & _native.W4A16_STATUS_SPLITK_TIMEOUT
                gave_up += 1
            else:
                assert status == 0
    finally:
        _native.set_spin_limit(old)
    say(f"give-ups in 5 calls with a zero poll budget: {gave_up}")
    for _ in range(3):
        y = int4_matmul(x, packed, scale)
        torch.cuda.synchronize()
        assert torch.equal(y, ref)
    assert _native.workspace_status() == 0
