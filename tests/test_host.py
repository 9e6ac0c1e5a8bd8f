"""Host-side checks that need no GPU: the C ABI library, argument validation,
workspace planning and the Python surface (quantize_llama, error mapping)."""

from __future__ import annotations

import ctypes
import os
import re
import types

import numpy as np
import pytest
import torch

from oracle import int4_oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "w4a16.h")


def header_functions() -> list[str]:
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(w4a16_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol(native_lib):
    from w4a16 import _native

    names = header_functions()
    assert set(names) == set(_native.EXPORTED_SYMBOLS), names
    for name in names:
        assert hasattr(native_lib, name), name
    assert native_lib.w4a16_abi_version() == _native.ABI_VERSION == 7


def _linear(lib, *, x=1, ldx=4096, packed=1, ldp=4096, scale=1, lds=4096, y=1, ldy=4096, m=1, n=4096,
            k=4096, gs=128, ws=None, ws_bytes=0):
    return lib.w4a16_linear(x, ldx, packed, ldp, scale, lds, y, ldy, m, n, k, gs, ws, ws_bytes, None)


def test_linear_argument_validation_returns_codes(native_lib):
    from w4a16 import _native as nat

    lib = native_lib
    assert _linear(lib, gs=64) == nat.W4A16_ERR_GROUP_SIZE
    assert _linear(lib, k=200, ldx=200) == nat.W4A16_ERR_K_GROUP
    assert _linear(lib, m=-1) == nat.W4A16_ERR_SHAPE
    assert _linear(lib, ldx=100) == nat.W4A16_ERR_SHAPE
    assert _linear(lib, ldp=100) == nat.W4A16_ERR_SHAPE
    assert _linear(lib, lds=100) == nat.W4A16_ERR_SHAPE
    assert _linear(lib, ldy=100) == nat.W4A16_ERR_SHAPE
    assert _linear(lib, x=None) == nat.W4A16_ERR_NULL
    assert _linear(lib, packed=None) == nat.W4A16_ERR_NULL
    assert _linear(lib, scale=None) == nat.W4A16_ERR_NULL
    assert _linear(lib, y=None) == nat.W4A16_ERR_NULL
    # Split-K shapes need a workspace: rejected before anything is launched.
    assert _linear(lib, n=12288, ldp=12288, lds=12288, ldy=12288) == nat.W4A16_ERR_WORKSPACE
    # Empty outputs are no-ops that touch no pointer.
    assert _linear(lib, m=0, x=None, packed=None, scale=None, y=None) == nat.W4A16_OK
    assert _linear(lib, n=0, x=None, packed=None, scale=None, y=None) == nat.W4A16_OK


def test_linear_rejects_split_k_slots_past_32_bit_offsets(native_lib):
    """Decode shapes whose published split-K slots exceed 4 GB are refused before any launch
    (the finish addresses slots with 32-bit byte offsets); no pointer is dereferenced."""
    from w4a16 import _native as nat

    m, n, k = 32, 1 << 20, 128 * 1024  # 128 K splits x 32 rows x 2^20 columns of fp32 = 16 GB of slots
    need = ctypes.c_size_t(0)
    assert native_lib.w4a16_workspace_size(m, n, k, 128, ctypes.byref(need)) == nat.W4A16_OK
    assert need.value > 1 << 32
    rc = _linear(native_lib, ldx=k, ldp=n, lds=n, ldy=n, m=m, n=n, k=k, ws=4096, ws_bytes=need.value)
    assert rc == nat.W4A16_ERR_TOO_LARGE


def test_grouped_argument_validation(native_lib):
    from w4a16 import _native as nat

    lib = native_lib
    n_max = nat.MAX_PROBLEMS
    table = (nat.Problem * (n_max + 1))()
    for i in range(n_max + 1):
        table[i] = nat.Problem(1, 4096, 1, 4096, 1, 4096, 1, 4096, 1, 4096, 4096)
    size = ctypes.c_size_t(0)
    assert lib.w4a16_linear_grouped(table, n_max + 1, 128, None, 0, None) == nat.W4A16_ERR_SHAPE
    assert lib.w4a16_linear_grouped(None, 2, 128, None, 0, None) == nat.W4A16_ERR_NULL
    neg = (nat.Problem * 1)(nat.Problem(1, 4096, 1, 4096, 1, 4096, 1, 4096, -1, 4096, 4096))
    assert lib.w4a16_linear_grouped(neg, 1, 128, None, 0, None) == nat.W4A16_ERR_SHAPE
    assert lib.w4a16_linear_grouped(table, 2, 64, None, 0, None) == nat.W4A16_ERR_GROUP_SIZE
    assert lib.w4a16_linear_grouped(table, 0, 128, None, 0, None) == nat.W4A16_OK
    bad = (nat.Problem * 2)(table[0], nat.Problem(1, 4096, 1, 4096, 1, 4096, None, 4096, 1, 4096, 4096))
    assert lib.w4a16_linear_grouped(bad, 2, 128, None, 0, None) == nat.W4A16_ERR_NULL
    bad[1] = nat.Problem(1, 4096, 1, 4096, 1, 4096, 1, 4096, 1, 4096, 4000)
    assert lib.w4a16_linear_grouped(bad, 2, 128, None, 0, None) == nat.W4A16_ERR_K_GROUP
    # A problem with M = 0 is skipped before its pointers are looked at.
    empty = (nat.Problem * 1)(nat.Problem(None, 4096, None, 4096, None, 4096, None, 4096, 0, 4096, 4096))
    assert lib.w4a16_linear_grouped(empty, 1, 128, None, 0, None) == nat.W4A16_OK
    # Decode split-K of two problems needs a workspace: sized, then rejected without one.
    assert lib.w4a16_workspace_size_grouped(table, 2, 128, ctypes.byref(size)) == nat.W4A16_OK
    assert size.value >= 65536 + 2 * 8 * 4096 * 4
    assert lib.w4a16_linear_grouped(table, 2, 128, None, 0, None) == nat.W4A16_ERR_WORKSPACE
    # Mixed M: the decode and GEMM batches share one workspace, sized for the larger.
    mixed = (nat.Problem * 2)(table[0], nat.Problem(16, 4096, 16, 4096, 16, 4096, 16, 4096, 2048, 4096, 4096))
    assert lib.w4a16_workspace_size_grouped(mixed, 2, 128, ctypes.byref(size)) == nat.W4A16_OK
    decode_only, gemm_only = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert lib.w4a16_workspace_size_grouped(table, 1, 128, ctypes.byref(decode_only)) == nat.W4A16_OK
    gemm = (nat.Problem * 1)(mixed[1])
    assert lib.w4a16_workspace_size_grouped(gemm, 1, 128, ctypes.byref(gemm_only)) == nat.W4A16_OK
    assert size.value == max(decode_only.value, gemm_only.value)


def test_dequant_argument_validation(native_lib):
    from w4a16 import _native as nat

    lib = native_lib
    assert lib.w4a16_dequant(1, 8, 1, 8, 1, 8, 5, 256, 8, 128, None) == nat.W4A16_ERR_DTYPE
    assert lib.w4a16_dequant(1, 8, 1, 8, 1, 8, 0, 256, 8, 0, None) == nat.W4A16_ERR_GROUP_SIZE
    assert lib.w4a16_dequant(1, 8, 1, 8, 1, 8, 0, 250, 8, 128, None) == nat.W4A16_ERR_K_GROUP
    assert lib.w4a16_dequant(None, 8, 1, 8, 1, 8, 0, 256, 8, 128, None) == nat.W4A16_ERR_NULL
    assert lib.w4a16_dequant(1, 4, 1, 8, 1, 8, 0, 256, 8, 128, None) == nat.W4A16_ERR_SHAPE
    assert lib.w4a16_dequant(None, 8, None, 8, None, 8, 0, 0, 8, 128, None) == nat.W4A16_OK


def test_error_strings(native_lib):
    for code in range(9):
        assert native_lib.w4a16_error_string(code)
    assert b"128" in native_lib.w4a16_error_string(4)


def test_workspace_planning(native_lib):
    from w4a16 import _native

    ws = _native.workspace_size
    assert ws(0, 4096, 4096) == 0
    assert ws(1, 0, 4096) == 0
    # A workspace is two halves plus 256 B of alignment slack.
    def half(b):
        assert (b - 256) % 512 == 0
        return (b - 256) // 2

    # M=1 Qwen3-8B gate: 8 K splits, 7 published fp32 partial slots [7, 1, N] in the lower half.
    assert half(ws(1, 12288, 4096)) == 7 * 12288 * 4
    # Large M: the GEMM needs only the per-(group, row) correction sums (32 * 2048 * 4 B in the
    # upper half), but activations off 16-byte alignment run 32-row decode chunks whose 3
    # published slots of [32, N] are larger, and the size query covers both.
    assert half(ws(2048, 12288, 4096)) == max(32 * 2048 * 4, 3 * 32 * 12288 * 4)
    with pytest.raises(AssertionError):
        ws(1, 4096, 4096, 64)
    with pytest.raises(ValueError):
        ws(1, 4096, 4000)
    # Split count never gives a wave no group and never exceeds the K groups.
    for m in (1, 2, 4, 8, 16, 17, 32):
        for k in (128, 1024, 4096, 12288, 25600):
            for n in (64, 1000, 1024, 12288):
                b = ws(m, n, k)
                if b:
                    slots = half(b) // (m * n * 4)  # nsplit - 1, rounded down by the 256-B alignment
                    assert 1 <= slots + (1 if half(b) % (m * n * 4) else 0) <= (k // 128 + 3) // 4


def test_workspace_query_covers_unaligned_activations(native_lib):
    """w4a16_workspace_size sees only shapes; it must cover the plan of a call whose
    activation rows are off 16-byte alignment (M > 32 then runs the decode kernel 32
    rows at a time) as well as the aligned plan.  The grouped query, which sees the
    pointers, gives each plan's exact size."""
    from w4a16 import _native as nat

    lib = native_lib
    exact = ctypes.c_size_t(0)

    def grouped(m, n, k, x):
        q = (nat.Problem * 1)()
        q[0] = nat.Problem(x, k, 4096, n, 4096, n, 4096, n, m, n, k)
        assert lib.w4a16_workspace_size_grouped(q, 1, 128, ctypes.byref(exact)) == nat.W4A16_OK
        return exact.value

    short = 0
    for m in (1, 16, 32, 33, 40, 64, 65, 129, 300, 2048, 4096):
        for k in (128, 1024, 4096, 5120, 12288, 25600):
            for n in (64, 1000, 1024, 4096, 12288, 25600):
                size = nat.workspace_size(m, n, k)
                aligned, unaligned = grouped(m, n, k, 4096), grouped(m, n, k, 4098)
                assert size >= aligned and size >= unaligned, (m, n, k, size, aligned, unaligned)
                short += unaligned > aligned
    assert short > 0  # the unaligned plan is the larger one for some shapes (e.g. M=33, K=4096, N=25600)


def test_swiglu_workspace_and_validation(native_lib):
    from w4a16 import _native as nat

    lib = native_lib
    size = ctypes.c_size_t(0)

    def ws(m, n, k):
        assert lib.w4a16_workspace_size_swiglu(m, n, k, 128, ctypes.byref(size)) == nat.W4A16_OK
        return size.value

    assert ws(0, 12288, 4096) == 0
    assert ws(4, 12288, 0) == 0
    # M <= 16: 8-wave workgroups (the pair launches > 1000 4-wave ones), so 4 K
    # splits; gate publishes all 4, up the first 3.
    assert (ws(1, 12288, 4096) - 256) // 2 == (4 + 3) * 12288 * 4
    # Larger M: bf16 up projection at the start of the upper half, GEMM scratch after it.
    assert (ws(2048, 12288, 4096) - 256) // 2 == 2048 * 12288 * 2 + 32 * 2048 * 4
    # M <= 32 is still one decode launch: 4 + 3 slots of [32, N].
    assert (ws(32, 12288, 4096) - 256) // 2 == (4 + 3) * 32 * 12288 * 4
    assert lib.w4a16_workspace_size_swiglu(1, 4096, 4096, 64, ctypes.byref(size)) == nat.W4A16_ERR_GROUP_SIZE

    def call(m=1, n=12288, k=4096, x=1, gp=1, gs=1, up=1, us=1, h=1, ldh=12288, group=128, wsp=None, wsb=0):
        return lib.w4a16_swiglu(x, k, gp, n, gs, n, up, n, us, n, h, ldh, m, n, k, group, wsp, wsb, None)

    assert call(group=64) == nat.W4A16_ERR_GROUP_SIZE
    assert call(k=200) == nat.W4A16_ERR_K_GROUP
    assert call(m=-1) == nat.W4A16_ERR_SHAPE
    assert call(ldh=100) == nat.W4A16_ERR_SHAPE
    assert call(up=None) == nat.W4A16_ERR_NULL
    assert call(us=None) == nat.W4A16_ERR_NULL
    assert call(h=None) == nat.W4A16_ERR_NULL
    assert call() == nat.W4A16_ERR_WORKSPACE
    assert call(m=2048) == nat.W4A16_ERR_WORKSPACE
    assert call(m=0, x=None, gp=None, gs=None, up=None, us=None, h=None) == nat.W4A16_OK


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("m,k,n,gs", [(1, 256, 64, 128), (4, 1024, 96, 128), (3, 512, 40, 64)])
def test_int4_matmul_host_branch_matches_reference_cpu_path(dtype, m, k, n, gs):
    """Host tensors: dequantize with scale.to(a.dtype), then a @ w
    (engine/kernels/quant.py:264-266), bit-equal to the oracle's restatement."""
    from w4a16 import int4_matmul

    g = torch.Generator().manual_seed(m + k + n)
    packed = torch.randint(-128, 128, (k // 2, n), generator=g, dtype=torch.int8)
    scale = torch.rand(k // gs, n, generator=g) * 0.01 + 1e-3
    a = torch.randn(m, k, generator=g).to(dtype)
    out = int4_matmul(a, packed, scale, gs)
    assert out.dtype == dtype and out.shape == (m, n) and not out.is_cuda
    assert torch.equal(out, orc.cpu_path(a, packed, scale, gs))


def test_int4_matmul_host_close_to_fp():
    """The reference's own invariant (tests/test_int4_quant.py:67-82) through
    w4a16.int4_matmul on host tensors: relative error < 0.25."""
    from w4a16 import int4_matmul, quantize_weight_int4

    torch.manual_seed(2)
    w = torch.randn(256, 128)
    a = torch.randn(4, 256)
    ref = a @ w
    packed, scale = quantize_weight_int4(w, group_size=128)
    out = int4_matmul(a, packed, scale, group_size=128)
    rel_err = ((ref - out).norm() / ref.norm()).item()
    assert rel_err < 0.25
    # bf16 activations as the engine passes them
    outb = int4_matmul(a.bfloat16(), packed, scale)
    assert outb.dtype == torch.bfloat16
    assert ((ref - outb.float()).norm() / ref.norm()).item() < 0.25


def test_device_only_entry_points_reject_host_tensors():
    from w4a16 import int4_matmul_grouped, int4_swiglu

    a = torch.randn(2, 256, dtype=torch.bfloat16)
    packed = torch.zeros(128, 64, dtype=torch.int8)
    scale = torch.ones(2, 64)
    with pytest.raises(TypeError):
        int4_matmul_grouped(a, [(packed, scale)])
    with pytest.raises(TypeError):
        int4_swiglu(a, (packed, scale), (packed, scale))


def test_quantize_matches_oracle_bit_exact():
    from w4a16 import quantize_weight_int4

    torch.manual_seed(4)
    for d_in, d_out, gs in [(256, 96, 128), (1024, 40, 64), (4096, 16, 128)]:
        w = (torch.randn(d_in, d_out) * 0.02).to(torch.bfloat16).float()
        p, s = quantize_weight_int4(w, gs)
        po, so = orc.quantize(w.numpy(), gs)
        np.testing.assert_array_equal(p.numpy(), po)
        np.testing.assert_array_equal(s.numpy(), so)
    with pytest.raises(ValueError):
        quantize_weight_int4(torch.randn(100, 8), 128)
    with pytest.raises(ValueError):
        quantize_weight_int4(torch.randn(129, 8), 129)


def test_host_dequantize_matches_oracle():
    from w4a16 import dequantize_weight_int4

    g = np.load(os.path.join(ROOT, "tests", "golden", "int4_golden.npz"))
    out = dequantize_weight_int4(torch.from_numpy(g["packed"]), torch.from_numpy(g["scale"]), 128)
    np.testing.assert_array_equal(out.numpy(), g["dequant"])
    outb = dequantize_weight_int4(torch.from_numpy(g["packed"]), torch.from_numpy(g["scale"]).bfloat16(), 128)
    np.testing.assert_array_equal(outb.float().numpy(), orc.dequantize_bf16(g["packed"], g["scale"]))


class _MiniWeights:
    """Just enough of the reference's LlamaWeights (engine/llama_weights.py) for quantize_llama."""

    def __init__(self, tensors, config):
        self._t = tensors
        self.config = config

    @property
    def embed_tokens(self):
        return self._t["model.embed_tokens.weight"]

    @property
    def lm_head(self):
        return self._t["model.embed_tokens.weight"]

    @property
    def norm_weight(self):
        return self._t["model.norm.weight"]

    def layer(self, i):
        p = f"model.layers.{i}."
        return {k[len(p):]: v for k, v in self._t.items() if k.startswith(p)}


def _mini_model(d=256, f=384, layers=2, kv=128):
    torch.manual_seed(42)
    cfg = types.SimpleNamespace(n_layer=layers, is_moe=False, n_experts=0)
    t = {"model.embed_tokens.weight": torch.randn(64, d), "model.norm.weight": torch.ones(d)}
    for i in range(layers):
        p = f"model.layers.{i}."
        t.update({
            p + "input_layernorm.weight": torch.ones(d),
            p + "self_attn.q_proj.weight": torch.randn(d, d),
            p + "self_attn.k_proj.weight": torch.randn(kv, d),
            p + "self_attn.v_proj.weight": torch.randn(kv, d),
            p + "self_attn.o_proj.weight": torch.randn(d, d),
            p + "mlp.gate_proj.weight": torch.randn(f, d),
            p + "mlp.up_proj.weight": torch.randn(f, d),
            p + "mlp.down_proj.weight": torch.randn(d, f),
        })
    model = types.SimpleNamespace(config=cfg, w=_MiniWeights(t, cfg), rope_cos=torch.ones(4), rope_sin=torch.zeros(4))
    return model, {k: v.clone() for k, v in t.items()}


def test_quantize_llama_structure_and_values():
    from w4a16 import QuantizedLlamaWeights, _Int4Weight, linear, quantize_llama

    model, dense = _mini_model()
    q_model = quantize_llama(model, group_size=128)
    assert isinstance(q_model.w, QuantizedLlamaWeights)
    assert q_model.rope_cos is model.rope_cos
    for i in range(2):
        blk = q_model.w.layer(i)
        assert torch.equal(blk["input_layernorm.weight"], dense[f"model.layers.{i}.input_layernorm.weight"])
        for suffix in ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "mlp.down_proj.weight"):
            w4 = blk[suffix]
            assert isinstance(w4, _Int4Weight)
            w = dense[f"model.layers.{i}.{suffix}"]
            assert w4.shape == tuple(w.shape)
            d_out, d_in = w.shape
            assert w4.packed.shape == (d_in // 2, d_out) and w4.packed.dtype == torch.int8
            assert w4.scale.shape == (d_in // 128, d_out) and w4.scale.dtype == torch.float32
            po, so = orc.quantize(w.T.contiguous().float().numpy(), 128)
            np.testing.assert_array_equal(w4.packed.numpy(), po)
            np.testing.assert_array_equal(w4.scale.numpy(), so)
            np.testing.assert_array_equal(w4.dequantize(torch.float32).numpy(), orc.dequantize(po, so).T)
            # Dense keys were released from the original weights.
            assert f"model.layers.{i}.{suffix}" not in model.w._t
    # layers.linear duck-types: dense tensors take a plain matmul, INT4 the HIP path.
    x = torch.randn(3, 64)
    wd = torch.randn(32, 64)
    assert torch.equal(linear(x, wd), x @ wd.T)
    # On the host, INT4 weights take the reference's host branch (quant.py:264-266).
    w4 = q_model.w.layer(0)["self_attn.q_proj.weight"]
    xh = torch.randn(1, 256, dtype=torch.bfloat16)
    assert torch.equal(linear(xh, w4), orc.cpu_path(xh, w4.packed, w4.scale))


def test_quantized_to_device_requires_quantized_model():
    from w4a16 import quantized_to_device

    model, _ = _mini_model(layers=1)
    with pytest.raises(TypeError):
        quantized_to_device(model, "cpu")


# ---------------------------------------------------------------------------
# Generated-code invariant of the GEMM's streamed weight loads
# ---------------------------------------------------------------------------

def _gemm_copy_wait_paths(asm: str, func: str) -> list[str]:
    """Walk the control flow of `func` from every direct-to-LDS copy.

    The GEMM waits for its activation copies with s_waitcnt vmcnt(17): at most
    17 vector memory operations may still be in flight, which is safe only if
    at least 17 loads were issued after the copies on every path.  Returns the
    paths that reach vmcnt(17) or a barrier before any wait that the copies
    are guaranteed to satisfy (vmcnt(n) after >= n later loads).
    """
    start = asm.index(func + ":")
    body = asm[start:asm.index(".Lfunc_end", start)].splitlines()[1:]
    blocks, order, cur = {}, [], "entry"
    blocks[cur] = []
    order.append(cur)
    for line in body:
        t = line.split(";")[0].strip()
        if not t:
            continue
        if re.match(r"^\.LBB\w+:$", t):
            cur = t[:-1]
            blocks[cur] = []
            order.append(cur)
            continue
        op = t.split()[0]
        if op.startswith("buffer_load") or op.startswith("global_load"):
            blocks[cur].append(("C",) if t.endswith(" lds") else ("L",))
        elif op == "s_waitcnt" and "vmcnt(" in t:
            blocks[cur].append(("W", int(re.search(r"vmcnt\((\d+)\)", t).group(1))))
        elif op == "s_barrier":
            blocks[cur].append(("B",))
        elif op == "s_branch":
            blocks[cur].append(("J", t.split()[-1]))
        elif op.startswith("s_cbranch"):
            blocks[cur].append(("CJ", t.split()[-1]))
        elif op == "s_endpgm":
            blocks[cur].append(("E",))
    nxt = {b: (order[i + 1] if i + 1 < len(order) else None) for i, b in enumerate(order)}
    bad = []

    def walk(block, idx, count, seen):
        key = (block, idx, min(count, 17))
        if key in seen:
            return
        seen.add(key)
        ins = blocks[block]
        for j in range(idx, len(ins)):
            e = ins[j]
            if e[0] == "C":
                return  # the walk from that copy covers the rest
            if e[0] == "L":
                count += 1
            elif e[0] == "W":
                if count >= e[1]:
                    return  # the copies are complete here
                if e[1] == 17:
                    bad.append(f"{block}: vmcnt(17) after {count} loads")
                    return
            elif e[0] == "B":
                bad.append(f"{block}: barrier after {count} loads, copies not waited for")
                return
            elif e[0] == "E":
                return
            elif e[0] == "J":
                walk(e[1], 0, count, seen)
                return
            elif e[0] == "CJ":
                walk(e[1], 0, count, seen)
        if nxt[block] is not None:
            walk(nxt[block], 0, count, seen)

    for b in order:
        for i, e in enumerate(blocks[b]):
            if e[0] == "C":
                walk(b, i + 1, 0, set())
    return bad


@pytest.fixture(scope="module")
def gfx950_asm(tmp_path_factory):
    """The library's gfx950 assembly, compiled with the build's own flags."""
    import shutil
    import subprocess

    from w4a16 import build as B

    if not os.path.exists(B.HIPCC) and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "k.s"
    flags = [f for f in B.FLAGS if f not in ("-fPIC", "-shared")]
    res = subprocess.run([B.HIPCC, *flags, "--cuda-device-only", "-S", *B.SOURCES, "-o", str(out)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def _kernel_resources(asm: str) -> dict[str, dict[str, int]]:
    """name -> {vgpr, spill bytes (private segment), lds} from the code object metadata."""
    out = {}
    for m in re.finditer(r"\.name:\s+(\S+)\n((?:.*\n){0,40})", asm):
        blk = m.group(2)
        v = re.search(r"\.vgpr_count:\s+(\d+)", blk)
        p = re.search(r"\.private_segment_fixed_size:\s+(\d+)", blk)
        if v and p:
            out[m.group(1)] = {"vgpr": int(v.group(1)), "spill": int(p.group(1))}
    return out


def test_hot_kernels_keep_their_register_budget(gfx950_asm):
    """The measured speed of the hot kernels rests on their occupancy: the full-tile GEMMs
    hold two waves per SIMD (at most 256 VGPRs, no spills), the batch-1 decode kernels five
    (at most 96 VGPRs), and no full-tile decode kernel spills.  A compiler change or an edit
    that breaks this shows up here rather than as an unexplained slowdown."""
    res = _kernel_resources(gfx950_asm)
    gemm = {k: v for k, v in res.items() if re.search(r"gemm_kernelILi\dELb1E", k)}
    decode_full = {k: v for k, v in res.items() if re.search(r"gemv_kernelILi\dELi\dELb1E", k)}
    decode_m1 = {k: v for k, v in decode_full.items() if "ELi1ELb" in k}
    assert len(gemm) >= 4 and len(decode_full) >= 20 and len(decode_m1) >= 4, (len(gemm), len(decode_full))
    for name, r in gemm.items():
        assert r["vgpr"] <= 256 and r["spill"] == 0, (name, r)
    for name, r in decode_full.items():
        assert r["spill"] == 0, (name, r)
    for name, r in decode_m1.items():
        assert r["vgpr"] <= 96, (name, r)


def test_gemm_streamed_loads_cover_the_copy_wait(gfx950_asm):
    """Every full-tile GEMM instantiation issues >= 17 loads between its activation copies and
    the vmcnt(17) wait that publishes them (the source's kLoadsAfterA), on every path."""
    import sys

    asm = gfx950_asm
    funcs = sorted(set(re.findall(r"^(_Z\w*gemm_kernelILi\dELb1E\w*):", asm, re.M)))
    assert len(funcs) >= 4, funcs  # CPL 2 / 4, two K halves, the SwiGLU pair
    for f in funcs:
        assert "vmcnt(17)" in asm[asm.index(f + ":"):asm.index(".Lfunc_end", asm.index(f + ":"))], f
        bad = _gemm_copy_wait_paths(asm, f)
        assert not bad, (f, bad[:5])
        print(f, "ok", file=sys.stderr)


def test_gemm_copy_wait_walker_flags_short_paths():
    """The walker itself: 16 loads before vmcnt(17) is a race, 17 is not, through a loop."""
    def fake(nloads):
        loads = "\n".join("\tbuffer_load_dword v1, v2, s[0:3], s4 offen" for _ in range(nloads))
        return (f"fn:\n\tbuffer_load_dwordx4 v3, s[0:3], s5 offen lds\n{loads}\n.LBB0_1:\n"
                f"\ts_waitcnt vmcnt(17)\n\ts_barrier\n\tbuffer_load_dwordx4 v3, s[0:3], s5 offen lds\n{loads}\n"
                "\ts_cbranch_scc1 .LBB0_1\n\ts_endpgm\n.Lfunc_end0:\n")
    assert _gemm_copy_wait_paths(fake(17), "fn") == []
    assert _gemm_copy_wait_paths(fake(16), "fn")


def test_noalloc_entry_point_rejects_before_launch(native_lib):
    """w4a16_linear_noalloc validates and sizes its scratch need on the host:
    oversized, bad-group and null-pointer calls return codes without touching a GPU."""
    from w4a16 import _native as nat

    lib = native_lib
    big = 1 << 40  # never dereferenced
    assert lib.w4a16_linear_noalloc(big, 4096, big, 131072, big, 131072, big, 131072,
                                    32, 131072, 4096, 128, None) == nat.W4A16_ERR_TOO_LARGE
    assert lib.w4a16_linear_noalloc(big, 4096, big, 4096, big, 4096, big, 4096, 1, 4096, 4096, 64,
                                    None) == nat.W4A16_ERR_GROUP_SIZE
    assert lib.w4a16_linear_noalloc(None, 4096, big, 4096, big, 4096, big, 4096, 1, 4096, 4096, 128,
                                    None) == nat.W4A16_ERR_NULL
    assert lib.w4a16_linear_noalloc(None, 0, None, 0, None, 0, None, 0, 0, 16, 128, 128, None) == nat.W4A16_OK


def test_unaligned_activation_rows_are_copied_for_gemm_sized_m():
    """The wrappers copy activation rows that are not 16-byte aligned (pointer or row
    stride) once M > 32, instead of letting the C entry point stream the weights once per
    32-row chunk; smaller M keeps the view (the decode kernel reads any alignment), and the
    lm_head GEMV always gets aligned rows."""
    from w4a16 import _native

    base = torch.arange(70 * 256 + 8, dtype=torch.float32).to(torch.bfloat16)
    for m in (33, 64, 2048 // 32):
        view = base[1:1 + m * 256].view(m, 256)             # pointer 2 bytes off alignment
        assert view.data_ptr() % 16 == 2
        rows, ld = _native._activations(view)
        assert rows.data_ptr() % 16 == 0 and ld == 256 and torch.equal(rows, view)
    small = base[1:1 + 32 * 256].view(32, 256)
    rows, ld = _native._activations(small)
    assert rows.data_ptr() == small.data_ptr() and ld == 256
    strided = base[: 40 * 257].view(40, 257)[:, :256]         # row stride 257: not a multiple of 8
    rows, ld = _native._activations(strided)
    assert ld == 256 and rows.data_ptr() % 16 == 0 and torch.equal(rows, strided)
    one = base[1:257].view(1, 256)
    rows, ld = _native._activations(one, always=True)
    assert rows.data_ptr() % 16 == 0 and torch.equal(rows, one)
    aligned = base[:64 * 256].view(64, 256)
    assert _native._activations(aligned)[0].data_ptr() == aligned.data_ptr()
