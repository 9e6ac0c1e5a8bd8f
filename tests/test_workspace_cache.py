"""CPU tests of the split-K workspace cache of w4a16._native.

The cache decides which buffer a call's kernels write their split-K slots
into, and whether a buffer that a captured HIP graph holds may ever be freed.
Its rules are host logic, so they are checked here on CPU tensors with the
capture state of the current stream stubbed (the GPU suite runs the same
rules under real captures: tests/test_gpu_contract.py):

* one buffer per (device, stream), zeroed when allocated, at least the size
  asked for, reused while large enough;
* outgrowing a buffer that no capture used drops it; outgrowing one that a
  capture used keeps it alive for the rest of the process;
* a buffer first allocated inside a capture is not known to be zero until a
  replay ran, so the next eager call on that stream zeroes it first;
* every other capture that uses such a buffer records a zero fill of its own,
  once per capture, so no graph's replays depend on another graph having
  replayed first.

On CPU tensors a "recorded" fill runs at once, which is what makes it visible
here.
"""

from __future__ import annotations

import pytest
import torch

from w4a16 import _native

DEV = torch.device("cpu", 0)  # any device with an index; the cache never launches work


@pytest.fixture
def cache(monkeypatch):
    """A fresh cache with a settable 'is capturing' flag."""
    state = {"capturing": False, "id": 1}
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: state["capturing"])
    monkeypatch.setattr(_native, "capture_id", lambda handle: state["id"] if state["capturing"] else 0)
    monkeypatch.setattr(_native, "_workspaces", {})
    monkeypatch.setattr(_native, "_retired", [])
    return state


def test_allocates_zeroed_and_reuses(cache):
    a = _native.get_workspace(DEV, 11, 1000)
    assert a.numel() >= max(1000, _native._MIN_WORKSPACE) and not a.any()
    assert _native.get_workspace(DEV, 11, 10) is a
    assert _native.get_workspace(DEV, 11, a.numel()) is a
    assert _native.get_workspace(DEV, 11, 0) is None


def test_one_buffer_per_stream(cache):
    a = _native.get_workspace(DEV, 11, 1000)
    b = _native.get_workspace(DEV, 12, 1000)
    assert a.data_ptr() != b.data_ptr()
    assert _native.get_workspace(DEV, 11, 1000) is a


def test_growth_without_capture_drops_the_old_buffer(cache):
    a = _native.get_workspace(DEV, 11, 1000)
    b = _native.get_workspace(DEV, 11, 4 * a.numel())
    assert b is not a and b.numel() >= 4 * a.numel() and not b.any()
    assert _native._retired == []


def test_growth_after_capture_keeps_the_captured_buffer(cache):
    a = _native.get_workspace(DEV, 11, 1000)
    cache["capturing"] = True
    assert _native.get_workspace(DEV, 11, 1000) is a  # a graph now holds a's address
    cache["capturing"] = False
    b = _native.get_workspace(DEV, 11, 4 * a.numel())
    assert b is not a
    assert any(t is a for t in _native._retired)  # never freed: replays still write into it
    # Growth doubles at least, so repeated small growth does not retire a buffer per call.
    c = _native.get_workspace(DEV, 11, b.numel() + 1)
    assert c.numel() >= 2 * b.numel()


def test_buffer_first_used_inside_a_capture_is_zeroed_before_eager_use(cache):
    cache["capturing"] = True
    a = _native.get_workspace(DEV, 21, 1000)
    ws = _native._workspaces[(0, 21)]
    assert ws.captured and not ws.defined
    a.fill_(7)  # what the capture's own fill kernel has not yet run to clear
    cache["capturing"] = False
    b = _native.get_workspace(DEV, 21, 1000)
    assert b is a and not b.any() and ws.defined


def test_capture_of_a_grown_buffer_inside_the_capture(cache):
    """Growing inside a capture: the new buffer comes from the graph's pool and the
    captured old one is retired, never freed."""
    a = _native.get_workspace(DEV, 31, 1000)
    cache["capturing"] = True
    _native.get_workspace(DEV, 31, 1000)
    b = _native.get_workspace(DEV, 31, 4 * a.numel())
    assert b is not a and any(t is a for t in _native._retired)
    ws = _native._workspaces[(0, 31)]
    assert ws.captured and not ws.defined


def test_each_capture_that_reuses_a_capture_born_buffer_fills_it_once(cache):
    """The reference captures one graph per decode bucket on torch's capture stream
    (engine/llama_paged_engine.py:315-347).  A buffer born in the first capture is
    reused by the next ones; each records its own fill (once), so replaying the
    second graph before the first has ever run still starts from empty slots."""
    cache["capturing"], cache["id"] = True, 101
    a = _native.get_workspace(DEV, 41, 1000)
    ws = _native._workspaces[(0, 41)]
    assert ws.filled_in == {101}
    a.fill_(7)
    assert _native.get_workspace(DEV, 41, 500) is a and a.eq(7).all()  # same capture: no second fill
    cache["id"] = 102
    assert _native.get_workspace(DEV, 41, 1000) is a and not a.any()  # its own fill
    a.fill_(7)
    assert _native.get_workspace(DEV, 41, 1000) is a and a.eq(7).all()  # once per capture
    assert ws.filled_in == {101, 102} and not ws.defined
    # Once zeroed eagerly the buffer stays zero between calls: later captures record no fill.
    cache["capturing"] = False
    assert _native.get_workspace(DEV, 41, 1000) is a and not a.any() and ws.defined
    cache["capturing"], cache["id"] = True, 103
    a.fill_(7)
    assert _native.get_workspace(DEV, 41, 1000) is a and a.eq(7).all()
    assert ws.filled_in == {101, 102}


def test_unknown_capture_id_records_a_fill_on_every_use(cache, monkeypatch):
    """If the runtime cannot name the capture, every use of a capture-born buffer
    inside a capture records a fill: more fills, never a missing one."""
    monkeypatch.setattr(_native, "capture_id", lambda handle: None)
    cache["capturing"] = True
    a = _native.get_workspace(DEV, 51, 1000)
    for _ in range(2):
        a.fill_(7)
        assert _native.get_workspace(DEV, 51, 1000) is a and not a.any()
