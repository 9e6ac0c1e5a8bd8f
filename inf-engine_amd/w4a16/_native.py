"""ctypes binding of the C ABI declared in include/w4a16.h.

The shared library ``libw4a16.so`` is built in-tree (see ``w4a16.build``) and
loaded from this package directory.  There is no fallback: if the library is
missing or a HIP device is absent, every device entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libw4a16.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

W4A16_OK = 0
W4A16_ERR_NULL = 1
W4A16_ERR_SHAPE = 2
W4A16_ERR_K_GROUP = 3
W4A16_ERR_GROUP_SIZE = 4
W4A16_ERR_WORKSPACE = 5
W4A16_ERR_LAUNCH = 6
W4A16_ERR_DTYPE = 7
W4A16_ERR_TOO_LARGE = 8
W4A16_ERR_CAPTURING = 9

W4A16_STATUS_SPLITK_TIMEOUT = 1

# W4A16_ABI_VERSION of include/w4a16.h this binding is written against.
ABI_VERSION = 7

DTYPE_F32 = 0
DTYPE_BF16 = 1

MAX_PROBLEMS = 16  # W4A16_MAX_PROBLEMS

# Every symbol include/w4a16.h declares.
EXPORTED_SYMBOLS = (
    "w4a16_abi_version",
    "w4a16_error_string",
    "w4a16_workspace_size",
    "w4a16_linear",
    "w4a16_linear_grouped",
    "w4a16_workspace_size_grouped",
    "w4a16_dequant",
    "w4a16_bf16_gemv",
    "w4a16_swiglu",
    "w4a16_workspace_size_swiglu",
    "w4a16_status_offset",
    "w4a16_debug_set_spin_limit",
    "w4a16_linear_noalloc",
    "w4a16_noalloc_status",
    "w4a16_capture_id",
)


class Problem(ctypes.Structure):
    """struct w4a16_problem of include/w4a16.h."""

    _fields_ = [
        ("x", ctypes.c_void_p), ("ldx", ctypes.c_int64),
        ("packed", ctypes.c_void_p), ("ldp", ctypes.c_int64),
        ("scale", ctypes.c_void_p), ("lds", ctypes.c_int64),
        ("y", ctypes.c_void_p), ("ldy", ctypes.c_int64),
        ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int),
    ]

_lib = None
_lib_lock = threading.Lock()


class NativeLibraryMissing(RuntimeError):
    """The HIP extension has not been built (run ``__graft_entry__.build()``)."""


def load_library() -> ctypes.CDLL:
    """Load (once) and return the native library, with argtypes configured."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryMissing(
                f"{LIB_PATH} not found: the w4a16 HIP extension is not built "
                "(python -c 'import __graft_entry__ as g; g.build()')"
            )
        lib = ctypes.CDLL(LIB_PATH)
        i64, i32, vp, sz = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
        lib.w4a16_abi_version.argtypes = []
        lib.w4a16_abi_version.restype = i32
        built = lib.w4a16_abi_version()
        if built != ABI_VERSION:
            raise NativeLibraryMissing(
                f"{LIB_PATH} implements ABI version {built}, this package expects {ABI_VERSION}: "
                "the library is stale (python -c 'import __graft_entry__ as g; g.build()')"
            )
        lib.w4a16_status_offset.argtypes = [sz, ctypes.POINTER(sz)]
        lib.w4a16_status_offset.restype = i32
        lib.w4a16_debug_set_spin_limit.argtypes = [ctypes.c_uint32]
        lib.w4a16_debug_set_spin_limit.restype = ctypes.c_uint32
        lib.w4a16_error_string.argtypes = [i32]
        lib.w4a16_error_string.restype = ctypes.c_char_p
        lib.w4a16_workspace_size.argtypes = [i32, i32, i32, i32, ctypes.POINTER(sz)]
        lib.w4a16_workspace_size.restype = i32
        lib.w4a16_linear.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, vp, sz, vp]
        lib.w4a16_linear.restype = i32
        lib.w4a16_linear_noalloc.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, vp]
        lib.w4a16_linear_noalloc.restype = i32
        lib.w4a16_noalloc_status.argtypes = [vp, ctypes.POINTER(ctypes.c_uint32)]
        lib.w4a16_noalloc_status.restype = i32
        lib.w4a16_capture_id.argtypes = [vp, ctypes.POINTER(ctypes.c_ulonglong)]
        lib.w4a16_capture_id.restype = i32
        lib.w4a16_dequant.argtypes = [vp, i64, vp, i64, vp, i64, i32, i32, i32, i32, vp]
        lib.w4a16_dequant.restype = i32
        lib.w4a16_swiglu.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, vp, i64,
                                     i32, i32, i32, i32, vp, sz, vp]
        lib.w4a16_swiglu.restype = i32
        lib.w4a16_workspace_size_swiglu.argtypes = [i32, i32, i32, i32, ctypes.POINTER(sz)]
        lib.w4a16_workspace_size_swiglu.restype = i32
        lib.w4a16_bf16_gemv.argtypes = [vp, i64, vp, i64, vp, i64, i32, i32, i32, vp]
        lib.w4a16_bf16_gemv.restype = i32
        pp = ctypes.POINTER(Problem)
        lib.w4a16_linear_grouped.argtypes = [pp, i32, i32, vp, sz, vp]
        lib.w4a16_linear_grouped.restype = i32
        lib.w4a16_workspace_size_grouped.argtypes = [pp, i32, i32, ctypes.POINTER(sz)]
        lib.w4a16_workspace_size_grouped.restype = i32
        _lib = lib
        return lib


def error_string(code: int) -> str:
    return load_library().w4a16_error_string(code).decode()


def check(code: int, what: str) -> None:
    """Map a C status to the exception type the reference raises for it."""
    if code == W4A16_OK:
        return
    msg = f"{what}: {error_string(code)} (code {code})"
    if code == W4A16_ERR_GROUP_SIZE:
        # engine/kernels/quant.py:267 asserts group_size == 128.
        raise AssertionError(msg)
    if code in (W4A16_ERR_K_GROUP, W4A16_ERR_SHAPE):
        # engine/kernels/quant.py:100-103 raise ValueError for bad K.
        raise ValueError(msg)
    raise RuntimeError(msg)


def _rows(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    """``t`` as rows the C ABI can address, and its row stride in elements.

    The kernels read unit-stride rows ``ld`` elements apart.  Views whose
    columns are strided, or whose rows overlap (row stride below the row width,
    e.g. ``x.expand(M, K)``), are copied; a single row may have any row stride,
    since only that row is read.  The reference's Triton kernel honours such
    strides (engine/kernels/quant.py:275), so they are accepted here too.
    """
    rows, width = t.shape
    if t.stride(1) != 1 or (rows > 1 and t.stride(0) < width):
        t = t.contiguous()
    return t, (t.stride(0) if rows > 1 else max(t.stride(0), width))


def _activations(a: torch.Tensor, always: bool = False) -> tuple[torch.Tensor, int]:
    """``_rows`` for activations, copied to a fresh (aligned) tensor when their
    rows are not 16-byte aligned (data pointer or row stride) and M > 32, or
    whenever ``always``.  The GEMM stages x with 16-byte copies; given such rows
    the C entry points run M > 32 through the decode kernel 32 rows at a time,
    and every chunk streams all of the weights again, so one copy of x is far
    cheaper.  The lm_head GEMV takes aligned rows only (``always``)."""
    a, ld = _rows(a)
    if (always or a.shape[0] > 32) and (a.data_ptr() % 16 or ld % 8):
        a = a.clone(memory_format=torch.contiguous_format)
        ld = a.shape[1]
    return a, ld


def workspace_size(m: int, n: int, k: int, group_size: int = 128) -> int:
    out = ctypes.c_size_t(0)
    check(load_library().w4a16_workspace_size(m, n, k, group_size, ctypes.byref(out)), "w4a16_workspace_size")
    return out.value


# Split-K workspaces.
#
# One zero-initialised buffer per (device, stream): calls on one stream are
# ordered, which is what makes sharing a buffer safe (the decode kernels'
# published-partial slots are empty again when every call ends).  The full
# size is passed on every call.
#
# HIP graphs bake the workspace pointer into their kernel nodes, so a buffer
# that any capture has used is never freed: when it is outgrown it moves to
# `_retired` and stays allocated for the life of the process.  A stream that
# first needs a workspace while it is capturing (torch.cuda.graph captures on
# its own side stream after the caller warmed up on another one) gets a buffer
# allocated inside the capture, from the graph's memory pool; its zero fill is
# a fill kernel recorded into that graph.  Until such a buffer has been zeroed
# eagerly its contents are defined only inside graphs that hold a fill of it,
# so every capture that uses it records one fill of its own (once per capture,
# by capture id) and an eager call zeroes it first.  Replays then never depend
# on which graph ran first.
class _Workspace:
    __slots__ = ("tensor", "captured", "defined", "filled_in")

    def __init__(self, tensor: torch.Tensor, captured: bool, defined: bool, filled_in: set[int | None]):
        self.tensor = tensor
        self.captured = captured    # some captured graph holds this buffer's address
        self.defined = defined      # zeroed eagerly: every call leaves its slots empty from then on
        self.filled_in = filled_in  # ids of the captures that recorded a zero fill (None: unnamed)


_workspaces: dict[tuple[int, int], _Workspace] = {}
_retired: list[torch.Tensor] = []
_ws_lock = threading.Lock()
_MIN_WORKSPACE = 1 << 20


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def capture_id(stream_handle: int) -> int | None:
    """Id of the graph capture the stream is in (0 when it is not capturing),
    or None when the runtime cannot say (the caller then treats every use as a
    new capture, which is safe but records more fills)."""
    out = ctypes.c_ulonglong(0)
    if load_library().w4a16_capture_id(stream_handle, ctypes.byref(out)) != W4A16_OK:
        return None
    return int(out.value)


def get_workspace(device: torch.device, stream_handle: int, nbytes: int) -> torch.Tensor | None:
    """The workspace of (device, stream), at least ``nbytes`` long (None for 0)."""
    if nbytes == 0:
        return None
    key = (_device_index(device), stream_handle)
    capturing = torch.cuda.is_current_stream_capturing()
    cid = capture_id(stream_handle) if capturing else 0
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is not None and ws.tensor.numel() >= nbytes:
            if capturing:
                ws.captured = True
                if not ws.defined and (cid is None or cid not in ws.filled_in):
                    ws.tensor.zero_()  # recorded into this capture
                    ws.filled_in.add(cid)
            elif not ws.defined:
                ws.tensor.zero_()
                ws.defined = True
            return ws.tensor
        size = max(nbytes, _MIN_WORKSPACE)
        if ws is not None:
            size = max(size, 2 * ws.tensor.numel())
            if ws.captured:
                _retired.append(ws.tensor)
        ws = _Workspace(torch.zeros(size, dtype=torch.uint8, device=device), captured=capturing,
                        defined=not capturing, filled_in={cid} if capturing else set())
        _workspaces[key] = ws
        return ws.tensor


def reserve_workspace(nbytes: int, device=None, stream=None) -> None:
    """Pre-size the workspace of ``stream`` (default: the current stream) to
    ``nbytes``, e.g. with ``workspace_size`` of the largest call a graph will
    capture.  Optional: without it the workspace grows on demand, in graph
    captures too."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    s = torch.cuda.current_stream(dev) if stream is None else stream
    with torch.cuda.device(dev), torch.cuda.stream(s):
        get_workspace(dev, s.cuda_stream, nbytes)


def workspace_status(device=None) -> int:
    """OR of the status words of every workspace (of ``device``, or all),
    the retired ones that captured graphs still use included.

    Synchronises the device.  A set W4A16_STATUS_SPLITK_TIMEOUT means a decode
    finisher gave up and wrote NaN; the affected workspaces are zeroed here
    (their slots may hold late partials) before the value is returned.
    """
    lib = load_library()
    want = None if device is None else _device_index(torch.device(device))
    status = 0
    with _ws_lock:
        buffers = [(w.tensor, w) for w in _workspaces.values()] + [(t, None) for t in _retired]
        for t, ws in buffers:
            if want is not None and t.device.index != want:
                continue
            off = ctypes.c_size_t(0)
            if lib.w4a16_status_offset(t.numel(), ctypes.byref(off)) != W4A16_OK:
                continue
            with torch.cuda.device(t.device):
                torch.cuda.synchronize()
                word = int(t[off.value:off.value + 4].cpu().view(torch.int32)[0])
                if word:
                    t.zero_()
                    torch.cuda.synchronize()
                    if ws is not None:
                        ws.defined = True
            status |= word
    return status


def set_spin_limit(polls: int) -> int:
    """Poll budget of the decode split-K finisher for later calls; returns the old one (tests only)."""
    return int(load_library().w4a16_debug_set_spin_limit(polls))


def linear(a: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, group_size: int) -> torch.Tensor:
    """y = a @ dequant(packed, scale) on the current HIP stream; a is [M, K] bf16."""
    lib = load_library()
    m, k = a.shape
    n = packed.shape[1]
    a, ldx = _activations(a)
    packed, ldp = _rows(packed)
    scale, lds = _rows(scale)
    y = torch.empty((m, n), device=a.device, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream(a.device).cuda_stream
    nbytes = workspace_size(m, n, k, group_size)
    ws = get_workspace(a.device, stream, nbytes)
    rc = lib.w4a16_linear(
        a.data_ptr(), ldx,
        packed.data_ptr(), ldp,
        scale.data_ptr(), lds,
        y.data_ptr(), y.stride(0),
        m, n, k, group_size,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        stream,
    )
    check(rc, "w4a16_linear")
    return y


def linear_noalloc(a: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, y: torch.Tensor,
                   group_size: int = 128) -> None:
    """y = a @ dequant(packed, scale) through w4a16_linear_noalloc, into the
    caller's y (bf16 [M, N], unit column stride, on a's device); no workspace.

    The C call allocates nothing.  Like ``linear``, activations whose rows are
    not 16-byte aligned are copied when M > 32 (the one allocation here, made
    before the call; pass aligned rows to avoid it)."""
    lib = load_library()
    m, k = a.shape
    n = packed.shape[1]
    if (y.dtype != torch.bfloat16 or tuple(y.shape) != (m, n) or (n > 1 and y.stride(1) != 1)
            or (m > 1 and y.stride(0) < n)):
        raise ValueError(f"y must be bf16 [{m}, {n}] with unit column stride and disjoint rows, got {y.dtype} "
                         f"{tuple(y.shape)} strides {tuple(y.stride())}")
    if y.device != a.device:
        raise ValueError(f"y is on {y.device}, the activations on {a.device}")
    a, ldx = _activations(a)
    packed, ldp = _rows(packed)
    scale, lds = _rows(scale)
    ldy = y.stride(0) if m > 1 else max(y.stride(0), n)
    with torch.cuda.device(a.device):
        stream = torch.cuda.current_stream(a.device).cuda_stream
        rc = lib.w4a16_linear_noalloc(a.data_ptr(), ldx, packed.data_ptr(), ldp, scale.data_ptr(), lds,
                                      y.data_ptr(), ldy, m, n, k, group_size, stream)
    check(rc, "w4a16_linear_noalloc")


def noalloc_status(device=None) -> int:
    """Status word of the no-alloc scratch of ``device`` (default: current).

    Synchronises the current stream of that device.  A set
    W4A16_STATUS_SPLITK_TIMEOUT means a decode finisher gave up and wrote NaN;
    the scratch is zeroed again before this returns, so later calls start from
    empty slots.  Sets the scratch up on first use; not allowed under capture."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    out = ctypes.c_uint32(0)
    with torch.cuda.device(dev):
        rc = load_library().w4a16_noalloc_status(torch.cuda.current_stream(dev).cuda_stream, ctypes.byref(out))
    check(rc, "w4a16_noalloc_status")
    return int(out.value)


def linear_grouped(xs, weights, group_size: int) -> list[torch.Tensor]:
    """Several projections in one call; xs[i] is [M_i, K_i] bf16, weights[i] = (packed, scale)."""
    lib = load_library()
    if not 0 < len(weights) <= MAX_PROBLEMS:
        raise ValueError(f"a grouped call takes 1..{MAX_PROBLEMS} projections, got {len(weights)}")
    table = (Problem * len(weights))()
    outs, keep = [], []
    rows = {}  # one (possibly copied) view per distinct activation tensor, so shared x stays shared
    for i, (x, (packed, scale)) in enumerate(zip(xs, weights)):
        if id(x) not in rows:
            rows[id(x)] = _activations(x)
        x, ldx = rows[id(x)]
        packed, ldp = _rows(packed)
        scale, lds = _rows(scale)
        keep += [x, packed, scale]
        m, n = x.shape[0], packed.shape[1]
        y = torch.empty((m, n), device=x.device, dtype=torch.bfloat16)
        outs.append(y)
        table[i] = Problem(x.data_ptr(), ldx, packed.data_ptr(), ldp, scale.data_ptr(), lds,
                           y.data_ptr(), y.stride(0), m, n, x.shape[1])
    dev = xs[0].device
    stream = torch.cuda.current_stream(dev).cuda_stream
    nbytes = ctypes.c_size_t(0)
    check(lib.w4a16_workspace_size_grouped(table, len(weights), group_size, ctypes.byref(nbytes)),
          "w4a16_workspace_size_grouped")
    ws = get_workspace(dev, stream, nbytes.value)
    rc = lib.w4a16_linear_grouped(table, len(weights), group_size,
                                  ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
                                  stream)
    check(rc, "w4a16_linear_grouped")
    return outs


def swiglu(a: torch.Tensor, gate, up, group_size: int) -> torch.Tensor:
    """h = silu(a @ Wg) * (a @ Wu) on the current HIP stream; gate/up are (packed, fp32 scale)."""
    lib = load_library()
    m, k = a.shape
    a, ldx = _activations(a)
    ops, lds_ = [], []
    for packed, scale in (gate, up):
        for t in (packed, scale):
            t, ld = _rows(t)
            ops.append(t)
            lds_.append(ld)
    n = ops[0].shape[1]
    h = torch.empty((m, n), device=a.device, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream(a.device).cuda_stream
    nbytes = ctypes.c_size_t(0)
    check(lib.w4a16_workspace_size_swiglu(m, n, k, group_size, ctypes.byref(nbytes)), "w4a16_workspace_size_swiglu")
    ws = get_workspace(a.device, stream, nbytes.value)
    rc = lib.w4a16_swiglu(
        a.data_ptr(), ldx,
        ops[0].data_ptr(), lds_[0], ops[1].data_ptr(), lds_[1],
        ops[2].data_ptr(), lds_[2], ops[3].data_ptr(), lds_[3],
        h.data_ptr(), h.stride(0),
        m, n, k, group_size,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        stream,
    )
    check(rc, "w4a16_swiglu")
    return h


def bf16_gemv(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """y = x @ w.T on the current HIP stream; x [M, K] bf16 (M <= 16), w [N, K] bf16."""
    lib = load_library()
    m, k = x.shape
    n = w.shape[0]
    x, ldx = _activations(x, always=True)
    w, ldw = _rows(w)
    y = torch.empty((m, n), device=x.device, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = lib.w4a16_bf16_gemv(x.data_ptr(), ldx, w.data_ptr(), ldw, y.data_ptr(), y.stride(0),
                             m, n, k, stream)
    check(rc, "w4a16_bf16_gemv")
    return y


def dequant(packed: torch.Tensor, scale: torch.Tensor, group_size: int, out_dtype: torch.dtype) -> torch.Tensor:
    """Dense [K, N] weights from packed/scale on the current HIP stream."""
    lib = load_library()
    if out_dtype == torch.float32:
        code = DTYPE_F32
    elif out_dtype == torch.bfloat16:
        code = DTYPE_BF16
    else:
        raise TypeError(f"w4a16 dequant supports float32 and bfloat16 outputs, got {out_dtype}")
    packed, ldp = _rows(packed)
    scale, lds = _rows(scale)
    k = packed.shape[0] * 2
    n = packed.shape[1]
    out = torch.empty((k, n), device=packed.device, dtype=out_dtype)
    stream = torch.cuda.current_stream(packed.device).cuda_stream
    rc = lib.w4a16_dequant(
        packed.data_ptr(), ldp, scale.data_ptr(), lds,
        out.data_ptr(), out.stride(0), code, k, n, group_size, stream,
    )
    check(rc, "w4a16_dequant")
    return out
