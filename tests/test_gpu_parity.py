"""GPU parity of the HIP W4A16 path against the CPU oracle (run with -m gpu).

Bars (written out in each test):
* unpack + scale indexing: bit-exact (dequant kernel; one-hot activations
  through the fused kernels; integer problems with power-of-two scales).
* fused output: the one parity bar of oracle/tolerance.py,
  max(|y - y_ref| - r * ulp_bf16(y_ref) / 2) <= 1e-3 * RMS(y_ref), where y_ref
  is the float64 product of the same packed weights and r counts the bf16
  roundings on the reference's path (1 everywhere except the GEMM-sized SwiGLU
  fallback).
Full benchmark shapes are checked against an fp32 torch dequantize-then-matmul
of the same weights on the GPU plus a float64 oracle check on sampled columns.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from oracle import int4_oracle as orc
from oracle.tolerance import assert_parity, ulp_bf16

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "int4_golden.npz")


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu(native_lib):
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.backends.cuda.matmul.allow_tf32 = False
    yield


def check_tolerance(y: torch.Tensor, y_ref: np.ndarray, label: str) -> None:
    yv = y.float().cpu().numpy().astype(np.float64)
    rel = assert_parity(yv, y_ref, label)
    say(f"  {label}: max(excess)/rms={rel:.3e}")


def rand_problem(m, k, n, seed, dev=DEV):
    g = torch.Generator().manual_seed(seed)
    packed = torch.randint(-128, 128, (k // 2, n), generator=g, dtype=torch.int8)
    scale = (torch.rand(k // 128, n, generator=g) * 0.01 + 0.001)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    return x.to(dev), packed.to(dev), scale.to(dev)


# ---------------------------------------------------------------------------
# Bit-exact unpack and scale indexing
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("k,n,gs", [(256, 64, 128), (512, 100, 128), (1024, 3072, 128), (256, 33, 64)])
def test_dequant_bit_exact(k, n, gs):
    from w4a16 import dequantize_weight_int4

    say(f"dequant k={k} n={n} gs={gs}")
    g = torch.Generator().manual_seed(k + n)
    packed = torch.randint(-128, 128, (k // 2, n), generator=g, dtype=torch.int8)
    scale = torch.randn(k // gs, n, generator=g)
    out = dequantize_weight_int4(packed.to(DEV), scale.to(DEV), gs)
    np.testing.assert_array_equal(out.cpu().numpy(), orc.dequantize(packed.numpy(), scale.numpy(), gs))
    outb = dequantize_weight_int4(packed.to(DEV), scale.to(DEV).bfloat16(), gs)
    assert outb.dtype == torch.bfloat16
    np.testing.assert_array_equal(outb.float().cpu().numpy(), orc.dequantize_bf16(packed.numpy(), scale.numpy(), gs))


def test_dequant_golden():
    from w4a16 import dequantize_weight_int4

    g = np.load(GOLDEN)
    out = dequantize_weight_int4(torch.from_numpy(g["packed"]).to(DEV), torch.from_numpy(g["scale"]).to(DEV))
    np.testing.assert_array_equal(out.cpu().numpy(), g["dequant"])


@pytest.mark.parametrize("m,k,n", [(7, 512, 256), (32, 1024, 4096), (100, 512, 300), (256, 384, 512)])
def test_one_hot_rows_bit_exact(m, k, n):
    """x[i] = e_{k_i}: y[i, n] = bf16(fp32(q[k_i, n] * scale[k_i // 128, n])) exactly,
    through the decode (M <= 32) and the GEMM (M > 32) kernels."""
    from w4a16 import int4_matmul

    say(f"one-hot m={m} k={k} n={n}")
    g = torch.Generator().manual_seed(m * 7 + k)
    packed = torch.randint(-128, 128, (k // 2, n), generator=g, dtype=torch.int8)
    scale = torch.randn(k // 128, n, generator=g)
    rows = torch.randint(0, k, (m,), generator=g)
    x = torch.zeros(m, k)
    x[torch.arange(m), rows] = 1.0
    y = int4_matmul(x.bfloat16().to(DEV), packed.to(DEV), scale.to(DEV))
    c = orc.codes(packed.numpy())
    r = rows.numpy()
    expect = orc.bf16_round(c[r].astype(np.float32) * scale.numpy()[r // 128])
    np.testing.assert_array_equal(y.float().cpu().numpy(), expect)


@pytest.mark.parametrize("m,k,n", [(1, 4096, 1024), (5, 1024, 512), (33, 1024, 512), (128, 768, 1024)])
def test_integer_problem_exact(m, k, n):
    """Integer activations, power-of-two scales: every partial is exact in fp32,
    so the result must be the bf16 rounding of the exact product."""
    from w4a16 import int4_matmul

    say(f"integer m={m} k={k} n={n}")
    rng = np.random.default_rng(m + k + n)
    packed = rng.integers(0, 256, size=(k // 2, n), dtype=np.uint8).view(np.int8)
    scale = np.ldexp(np.float32(1.0), rng.integers(-4, 3, size=(k // 128, n))).astype(np.float32)
    x = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
    y = int4_matmul(torch.from_numpy(x).bfloat16().to(DEV), torch.from_numpy(packed).to(DEV),
                    torch.from_numpy(scale).to(DEV))
    exact = orc.fused_reference(x, packed, scale)
    np.testing.assert_array_equal(y.float().cpu().numpy(), orc.bf16_round(exact.astype(np.float32)))


def test_golden_product():
    from w4a16 import int4_matmul

    g = np.load(GOLDEN)
    y = int4_matmul(torch.from_numpy(g["x"]).bfloat16().to(DEV), torch.from_numpy(g["packed"]).to(DEV),
                    torch.from_numpy(g["scale"]).to(DEV))
    np.testing.assert_array_equal(y.float().cpu().numpy(), orc.bf16_round(g["y"].astype(np.float32)))


# ---------------------------------------------------------------------------
# Tolerance against the float64 oracle at oracle-sized shapes
# ---------------------------------------------------------------------------

SHAPES = [
    # (M, K, N): Qwen3-0.6B gate (config 1), ragged N, M on both sides of 32
    (1, 1024, 3072), (2, 1024, 3072), (3, 512, 1000), (4, 4096, 1024), (8, 1024, 4096),
    (16, 2048, 1536), (17, 1024, 2048), (31, 512, 768), (32, 4096, 1024),
    (33, 1024, 1024), (64, 1024, 1280), (100, 768, 1000), (129, 512, 640), (256, 2048, 1024),
]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_tolerance_vs_oracle(m, k, n):
    from w4a16 import int4_matmul, synth

    say(f"tolerance m={m} k={k} n={n}")
    packed, scale = synth.make_weight(k, n, seed=1000 + n)
    x = synth.make_activations(m, k, seed=2000 + m)
    y = int4_matmul(x.to(DEV), packed.to(DEV), scale.to(DEV))
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    y_ref = orc.fused_reference(x.float().numpy(), packed.numpy(), scale.numpy())
    check_tolerance(y, y_ref, f"M={m} K={k} N={n}")


# Seeded random shapes across every planner branch: M on both sides of the
# decode / GEMM boundaries (16, 32, 64), K from one to sixteen groups, N
# anywhere in 1..2048 (odd, not a multiple of any strip or tile width), with
# uniform random bytes (nibble -8 included) and, for some cases, strided
# activation rows and column slices of wider weight / scale tensors.
SWEEP_SEED = 20261202
SWEEP_CASES = 32


def _sweep_case(i: int):
    rng = np.random.default_rng(SWEEP_SEED + i)
    m = int(rng.choice([1, 2, 3, 5, 8, 13, 16, 17, 24, 31, 32, 33, 48, 64, 65, 96, 127, 128, 129, 200, 300]))
    k = 128 * int(rng.integers(1, 17))
    n = int(rng.integers(1, 2049))
    pad_x = int(rng.choice([0, 0, 8, 24]))      # extra activation columns (row stride K + pad)
    pad_w = int(rng.choice([0, 0, 4, 100]))     # extra weight / scale columns (column slice)
    return m, k, n, pad_x, pad_w


@pytest.mark.parametrize("case", range(SWEEP_CASES))
def test_random_shape_sweep_vs_oracle(case):
    from w4a16 import int4_matmul

    m, k, n, pad_x, pad_w = _sweep_case(case)
    say(f"sweep case={case} m={m} k={k} n={n} pad_x={pad_x} pad_w={pad_w}")
    g = torch.Generator().manual_seed(SWEEP_SEED + case)
    packed_full = torch.randint(-128, 128, (k // 2, n + pad_w), generator=g, dtype=torch.int8)
    scale_full = torch.rand(k // 128, n + pad_w, generator=g) * 0.01 + 0.001
    x_full = torch.randn(m, k + pad_x, generator=g).to(torch.bfloat16)
    packed, scale, x = packed_full[:, :n], scale_full[:, :n], x_full[:, :k]
    y = int4_matmul(x_full.to(DEV)[:, :k], packed_full.to(DEV)[:, :n], scale_full.to(DEV)[:, :n])
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    y_ref = orc.fused_reference(x.float().numpy(), packed.numpy(), scale.numpy())
    check_tolerance(y, y_ref, f"sweep {case}: M={m} K={k} N={n} pad_x={pad_x} pad_w={pad_w}")


@pytest.mark.parametrize("case", range(12))
def test_random_grouped_sweep_vs_oracle(case):
    """int4_matmul_grouped with 1-5 problems: shared activations (one M, one K) or per-problem
    activations with their own M and K, mixing decode- and GEMM-sized problems in one call."""
    from w4a16 import int4_matmul_grouped

    rng = np.random.default_rng(SWEEP_SEED + 1000 + case)
    count = int(rng.integers(1, 6))
    shared = bool(rng.integers(0, 2))
    ms = [1, 3, 8, 16, 31, 33, 64, 100, 150, 257]
    m0, k0 = int(rng.choice(ms)), 128 * int(rng.integers(1, 13))
    shapes = [(m0, k0) if shared else (int(rng.choice(ms)), 128 * int(rng.integers(1, 13))) for _ in range(count)]
    ns = [int(rng.integers(1, 1537)) for _ in range(count)]
    say(f"grouped sweep case={case} shared={shared} problems={[(m, k, n) for (m, k), n in zip(shapes, ns)]}")
    g = torch.Generator().manual_seed(SWEEP_SEED + 1000 + case)
    ws = [(torch.randint(-128, 128, (k // 2, n), generator=g, dtype=torch.int8),
           torch.rand(k // 128, n, generator=g) * 0.01 + 0.001) for (m, k), n in zip(shapes, ns)]
    xs = [torch.randn(m, k, generator=g).to(torch.bfloat16) for m, k in (shapes[:1] if shared else shapes)]
    dws = [(p.to(DEV), sc.to(DEV)) for p, sc in ws]
    ys = int4_matmul_grouped(xs[0].to(DEV) if shared else [x.to(DEV) for x in xs], dws)
    assert len(ys) == count
    for i, ((m, k), n) in enumerate(zip(shapes, ns)):
        x = xs[0] if shared else xs[i]
        assert ys[i].shape == (m, n)
        y_ref = orc.fused_reference(x.float().numpy(), ws[i][0].numpy(), ws[i][1].numpy())
        check_tolerance(ys[i], y_ref, f"grouped {case}.{i}: M={m} K={k} N={n}")


@pytest.mark.parametrize("m,k,n", [(1536, 384, 4000), (1536, 640, 4096), (1500, 128, 4096)])
def test_gemm_two_k_halves(m, k, n):
    """192..256 tiles of 128 x 256: one 8-wave workgroup per tile whose two K
    halves are summed in LDS.  Odd group counts leave one half a group short
    (K=384, 640), K=128 leaves one half empty, N=4000 takes the generic loads."""
    from w4a16 import int4_matmul, synth

    say(f"gemm two K halves m={m} k={k} n={n}")
    packed, scale = synth.make_weight(k, n, seed=k + n)
    x = synth.make_activations(m, k, seed=m + k)
    y = int4_matmul(x.to(DEV), packed.to(DEV), scale.to(DEV))
    check_tolerance(y, orc.fused_reference(x.float().numpy(), packed.numpy(), scale.numpy()), f"M={m} K={k} N={n}")


def test_unaligned_and_strided_activations():
    """Row stride > K, an activation pointer off 16-byte alignment (generic loads),
    and a transposed view (made contiguous by the wrapper)."""
    from w4a16 import int4_matmul

    for m in (3, 40):
        say(f"strided m={m}")
        x, packed, scale = rand_problem(m, 512, 256, seed=m)
        y_ref = orc.fused_reference(x.float().cpu().numpy(), packed.cpu().numpy(), scale.cpu().numpy())
        big = torch.zeros(m, 512 + 8, dtype=torch.bfloat16, device=DEV)
        big[:, :512] = x
        check_tolerance(int4_matmul(big[:, :512], packed, scale), y_ref, f"ldx=520 M={m}")
        flat = torch.zeros(m * 512 + 1, dtype=torch.bfloat16, device=DEV)
        xu = flat[1:].view(m, 512)
        xu.copy_(x)
        check_tolerance(int4_matmul(xu, packed, scale), y_ref, f"unaligned M={m}")
        xt = x.t().contiguous().t()
        check_tolerance(int4_matmul(xt, packed, scale), y_ref, f"transposed M={m}")


def test_overlapping_rows_and_single_row_strides():
    """Views the reference's stride-honouring Triton kernel accepts
    (engine/kernels/quant.py:275): rows that overlap (x.expand, row stride 0),
    a single row whose row stride is below K, and strided weight views."""
    from w4a16 import int4_matmul, int4_matmul_grouped

    for m in (1, 5, 64):
        say(f"expanded rows m={m}")
        x1, packed, scale = rand_problem(1, 512, 256, seed=40 + m)
        xe = x1[0].expand(m, 512)
        assert m == 1 or xe.stride() == (0, 1)  # torch keeps stride K on a size-1 dim
        y_ref = np.repeat(orc.fused_reference(x1.float().cpu().numpy(), packed.cpu().numpy(),
                                              scale.cpu().numpy()), m, axis=0)
        check_tolerance(int4_matmul(xe, packed, scale), y_ref, f"expand M={m}")
        (yg,) = int4_matmul_grouped(xe, [(packed, scale)])
        check_tolerance(yg, y_ref, f"expand grouped M={m}")
    say("single row, row stride 1")
    x1, packed, scale = rand_problem(1, 512, 256, seed=50)
    xs = x1.as_strided((1, 512), (1, 1))
    y_ref = orc.fused_reference(x1.float().cpu().numpy(), packed.cpu().numpy(), scale.cpu().numpy())
    check_tolerance(int4_matmul(xs, packed, scale), y_ref, "single row stride 1")
    say("column-major weights")
    x, packed, scale = rand_problem(3, 512, 256, seed=51)
    y_ref = orc.fused_reference(x.float().cpu().numpy(), packed.cpu().numpy(), scale.cpu().numpy())
    pt = packed.t().contiguous().t()
    st = scale.t().contiguous().t()
    check_tolerance(int4_matmul(x, pt, st), y_ref, "column-major packed/scale")


def test_empty_and_zero_k():
    from w4a16 import int4_matmul

    _, packed, scale = rand_problem(1, 256, 64, seed=3)
    y = int4_matmul(torch.empty(0, 256, dtype=torch.bfloat16, device=DEV), packed, scale)
    assert y.shape == (0, 64)
    y = int4_matmul(torch.empty(4, 0, dtype=torch.bfloat16, device=DEV),
                    torch.empty(0, 64, dtype=torch.int8, device=DEV), torch.empty(0, 64, device=DEV))
    assert y.shape == (4, 64) and torch.count_nonzero(y) == 0
    y = int4_matmul(torch.empty(40, 0, dtype=torch.bfloat16, device=DEV),
                    torch.empty(0, 64, dtype=torch.int8, device=DEV), torch.empty(0, 64, device=DEV))
    assert y.shape == (40, 64) and torch.count_nonzero(y) == 0


def test_errors_on_device():
    from w4a16 import int4_matmul

    x, packed, scale = rand_problem(2, 256, 64, seed=4)
    with pytest.raises(AssertionError):
        int4_matmul(x, packed, scale, group_size=64)
    with pytest.raises(ValueError):
        int4_matmul(x[:, :128], packed, scale)
    with pytest.raises(TypeError):
        int4_matmul(x.float(), packed, scale)


def test_fused_linear_reshapes_leading_dims():
    from w4a16 import _Int4Weight, linear, synth

    packed, scale = synth.make_weight(512, 384, seed=9)
    w4 = _Int4Weight(packed.to(DEV), scale.to(DEV), 128, (384, 512))
    x = synth.make_activations(6, 512, seed=10).reshape(2, 3, 512)
    y = linear(x.to(DEV), w4)
    assert y.shape == (2, 3, 384)
    y_ref = orc.fused_reference(x.reshape(6, 512).float().numpy(), packed.numpy(), scale.numpy())
    check_tolerance(y.reshape(6, 384), y_ref, "fused_linear [2,3,512]")
    dense = w4.dequantize(torch.float32)
    np.testing.assert_array_equal(dense.cpu().numpy(), orc.dequantize(packed.numpy(), scale.numpy()).T)


def test_split_k_deterministic_and_slots_reset():
    """Repeated and interleaved calls sharing one workspace give identical bits.

    The decode calls' published-partial slots must be empty again after every
    call, whatever ran in between: here a split-K GEMM (M=64) and a two-subtile call
    (M=24) use the same workspace between decode calls."""
    from w4a16 import int4_matmul

    shapes = [(1, 4096, 12288), (64, 1024, 512), (4, 12288, 4096), (24, 4096, 1024), (16, 4096, 1024), (1, 4096, 1024)]
    probs = [rand_problem(m, k, n, seed=m + k) for (m, k, n) in shapes]
    first = [int4_matmul(*p) for p in probs]
    for _ in range(3):
        for p, y0 in zip(probs, first):
            assert torch.equal(int4_matmul(*p), y0)


@pytest.mark.parametrize("m", [1, 5, 16, 24, 40, 300])
def test_grouped_shared_activations(m):
    """q/k/v-style group (one x, three weights, ragged N) in one launch."""
    from w4a16 import int4_matmul, int4_matmul_grouped, synth

    say(f"grouped shared-x m={m}")
    k = 1024
    weights = [synth.make_weight(k, n, seed=300 + n) for n in (1024, 256, 320)]
    x = synth.make_activations(m, k, seed=7 + m)
    outs = int4_matmul_grouped(x.to(DEV), [(p.to(DEV), s.to(DEV)) for p, s in weights])
    for (p, s), y in zip(weights, outs):
        assert y.shape == (m, p.shape[1])
        check_tolerance(y, orc.fused_reference(x.float().numpy(), p.numpy(), s.numpy()), f"grouped N={p.shape[1]}")
        if m <= 16:  # decode path: identical arithmetic per problem, so identical bits
            assert torch.equal(y, int4_matmul(x.to(DEV), p.to(DEV), s.to(DEV)))


@pytest.mark.parametrize("m", [1, 8, 24, 96])
def test_grouped_distinct_activations(m):
    """MoE-style group: each problem has its own activations and K."""
    from w4a16 import int4_matmul_grouped, synth

    say(f"grouped distinct-x m={m}")
    specs = [(512, 768), (1024, 256), (256, 512), (768, 1024)]
    weights = [synth.make_weight(k, n, seed=k + n) for k, n in specs]
    xs = [synth.make_activations(m, k, seed=k + m) for k, _ in specs]
    outs = int4_matmul_grouped([x.to(DEV) for x in xs], [(p.to(DEV), s.to(DEV)) for p, s in weights])
    for x, (p, s), y in zip(xs, weights, outs):
        check_tolerance(y, orc.fused_reference(x.float().numpy(), p.numpy(), s.numpy()), f"moe K={x.shape[1]}")


def test_grouped_mixed_m_across_kernels():
    """Experts with their own token counts: one table mixes decode (M <= 16),
    two-subtile decode (16 < M <= 32), GEMM (M > 32), an unaligned-x GEMM row block and
    an empty expert; 16 problems, the table maximum."""
    from w4a16 import int4_matmul, int4_matmul_grouped, synth

    say("grouped mixed M")
    ms = [1, 3, 16, 0, 17, 32, 33, 130, 2, 7, 64, 1, 5, 9, 40, 12]
    k, n = 512, 384
    weights = [synth.make_weight(k, n, seed=900 + i) for i in range(len(ms))]
    xs = []
    for i, m in enumerate(ms):
        x = synth.make_activations(m, k, seed=950 + i).to(DEV)
        if i == 14:  # row stride not a multiple of 8 elements: staged through the decode path
            buf = torch.zeros(m, k + 3, dtype=torch.bfloat16, device=DEV)
            buf[:, :k] = x
            x = buf[:, :k]
        xs.append(x)
    dw = [(p.to(DEV), s.to(DEV)) for p, s in weights]
    outs = int4_matmul_grouped(xs, dw)
    for i, (m, x, (p, s), y) in enumerate(zip(ms, xs, weights, outs)):
        assert y.shape == (m, n)
        if m == 0:
            continue
        check_tolerance(y, orc.fused_reference(x.float().cpu().numpy(), p.numpy(), s.numpy()), f"expert {i} M={m}")
        if m <= 16 and i != 14:  # same decode arithmetic as a lone call
            assert torch.equal(y, int4_matmul(x, *dw[i]))


@pytest.mark.parametrize("m", [1, 20, 64])
def test_zero_subnormal_and_extreme_scales(m):
    """Zero / subnormal scale groups contribute nothing (exactly on the decode
    path, < 1e-20 per unit on the GEMM path); large scale ratios between groups."""
    from w4a16 import int4_matmul

    say(f"scales m={m}")
    k, n = 1024, 512
    g = torch.Generator().manual_seed(m)
    packed = torch.randint(-128, 128, (k // 2, n), generator=g, dtype=torch.int8)
    scale = torch.rand(k // 128, n, generator=g) * 0.01 + 1e-3
    scale[1, :64] = 0.0                          # zero groups
    scale[:, 64:70] = 0.0                        # all-zero columns
    scale[2, 100:140] = 1e-39                    # subnormal
    scale[3, 200:240] = 1e4                      # large jumps between groups
    scale[5, 200:240] = 1e-6
    scale[6, 300:330] = -0.02                    # negative scales
    x = torch.randn(m, k, generator=g).bfloat16()
    y = int4_matmul(x.to(DEV), packed.to(DEV), scale.to(DEV))
    ref = orc.fused_reference(x.float().numpy(), packed.numpy(), scale.numpy())
    check_tolerance(y, ref, f"scales M={m}")
    yc = y.float().cpu().numpy()
    assert np.all(np.abs(yc[:, 64:70]) <= 1e-15)


def test_quantize_llama_on_device_matches_dense():
    """quantize_llama -> quantized_to_device -> linear: matches dequantize-then-matmul."""
    from w4a16 import linear, quantize_llama, quantized_to_device
    from test_host import _mini_model

    model, _ = _mini_model(d=512, f=768, layers=1, kv=256)
    q_model = quantized_to_device(quantize_llama(model, 128), DEV)
    blk = q_model.w.layer(0)
    x = torch.randn(5, 512).bfloat16()
    for suffix in ("self_attn.q_proj.weight", "mlp.gate_proj.weight"):
        w4 = blk[suffix]
        y = linear(x.to(DEV), w4)
        y_ref = orc.fused_reference(x.float().numpy(), w4.packed.cpu().numpy(), w4.scale.cpu().numpy())
        check_tolerance(y, y_ref, suffix)
    # down_proj: K = 768
    w4 = blk["mlp.down_proj.weight"]
    x = torch.randn(40, 768).bfloat16()
    y = linear(x.to(DEV), w4)
    check_tolerance(y, orc.fused_reference(x.float().numpy(), w4.packed.cpu().numpy(), w4.scale.cpu().numpy()),
                    "down_proj M=40")


def test_int4_checkpoint_loads_to_device_and_matches(tmp_path):
    """save_int4 -> load_quantized_llama(device=cuda): identical bytes, identical outputs."""
    from w4a16 import linear, load_quantized_llama, quantize_llama, quantized_to_device, save_int4
    from test_host import _mini_model

    say("int4 checkpoint round trip on device")
    model, _ = _mini_model(d=512, f=768, layers=1, kv=256)
    q = quantized_to_device(quantize_llama(model, 128), DEV)
    path = str(tmp_path / "q.safetensors")
    save_int4(q, path)
    fresh, _ = _mini_model(d=512, f=768, layers=1, kv=256)
    q2 = load_quantized_llama(fresh, path, device=DEV)
    x = torch.randn(3, 512).bfloat16().to(DEV)
    for suffix in ("self_attn.q_proj.weight", "mlp.up_proj.weight"):
        a, b = q.w.layer(0)[suffix], q2.w.layer(0)[suffix]
        assert b.packed.is_cuda and torch.equal(a.packed, b.packed) and torch.equal(a.scale, b.scale)
        assert torch.equal(linear(x, a), linear(x, b))


def test_graph_capture_replays_match_eager():
    """int4_matmul captured in a HIP graph: each replay, separated by eager work
    and synchronisation, must reproduce the eager result bit for bit."""
    from w4a16 import int4_matmul

    from w4a16 import int4_matmul_grouped

    cases = [rand_problem(m, k, n, seed=50 + m) for (m, k, n) in [(1, 4096, 12288), (8, 4096, 1024), (64, 1024, 2048)]]
    xg, pg, sg = rand_problem(1, 4096, 1024, seed=99)
    _, pg2, sg2 = rand_problem(1, 4096, 3072, seed=98)
    eager = [int4_matmul(*c) for c in cases] + int4_matmul_grouped(xg, [(pg, sg), (pg2, sg2)])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    def body():
        return [int4_matmul(*c) for c in cases] + int4_matmul_grouped(xg, [(pg, sg), (pg2, sg2)])

    with torch.cuda.stream(s):
        body()  # warm up on the capture stream: creates its workspace
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        outs = body()
    for rep in range(4):
        for o in outs:
            o.zero_()
        junk = torch.randn(1024, 1024, device=DEV) @ torch.randn(1024, 1024, device=DEV)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep}"
        del junk


# ---------------------------------------------------------------------------
# Benchmark configs at full size
# ---------------------------------------------------------------------------

def full_size_check(m, k, n, seed, label):
    from w4a16 import dequantize_weight_int4, int4_matmul, synth

    say(f"full-size {label}: M={m} K={k} N={n}")
    packed, scale = synth.make_weight(k, n, seed=seed, device=DEV)
    x = synth.make_activations(m, k, seed=seed + 1, device=DEV)
    y = int4_matmul(x, packed, scale)
    w = dequantize_weight_int4(packed, scale)                    # bit-exact (tested above)
    y_ref = (x.float() @ w).double().cpu().numpy()                # fp32 dequantize-then-matmul
    check_tolerance(y, y_ref, label)
    # float64 oracle on sampled columns
    cols = torch.randperm(n, generator=torch.Generator().manual_seed(seed))[:48].sort().values
    y64 = orc.fused_reference(x.float().cpu().numpy(), packed[:, cols.to(DEV)].cpu().numpy(),
                              scale[:, cols.to(DEV)].cpu().numpy())
    check_tolerance(y[:, cols.to(DEV)], y64, label + " (fp64 oracle, 48 cols)")
    del w


@pytest.mark.parametrize("name,k,n", [("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
                                      ("gate", 4096, 12288), ("up", 4096, 12288), ("down", 12288, 4096)])
def test_config2_qwen3_8b_decode(name, k, n):
    full_size_check(1, k, n, seed=sum(map(ord, name)), label=f"qwen3-8b {name} M=1")


@pytest.mark.parametrize("m", [4, 8, 16, 32])
@pytest.mark.parametrize("k,n", [(4096, 12288), (12288, 4096)])
def test_config3_qwen3_8b_batched(m, k, n):
    full_size_check(m, k, n, seed=m * 31 + k, label=f"qwen3-8b M={m} {k}x{n}")


@pytest.mark.parametrize("name,k,n", [("q", 4096, 4096), ("k", 4096, 1024), ("o", 4096, 4096),
                                      ("gate", 4096, 12288), ("down", 12288, 4096)])
def test_config4_qwen3_8b_prefill(name, k, n):
    full_size_check(2048, k, n, seed=len(name) * 97 + k, label=f"qwen3-8b {name} M=2048")


@pytest.mark.parametrize("name,m,k,n", [("q", 1, 5120, 8192), ("kv", 1, 5120, 1024), ("o", 1, 8192, 5120),
                                        ("gate", 1, 5120, 25600), ("down", 1, 25600, 5120),
                                        ("q", 4096, 5120, 8192), ("kv", 4096, 5120, 1024), ("o", 4096, 8192, 5120),
                                        ("gate", 4096, 5120, 25600), ("down", 4096, 25600, 5120)])
def test_config5_qwen3_32b(name, m, k, n):
    full_size_check(m, k, n, seed=m + k + n, label=f"qwen3-32b {name} M={m}")


@pytest.mark.parametrize("m,k,n", [(1, 8, 1), (1, 64, 15), (2, 256, 16), (7, 1000, 100), (16, 4096, 1000),
                                   (1, 4096, 4099), (3, 520, 64)])
def test_lm_head_bf16_gemv(m, k, n):
    """Dense bf16 decode GEMV (logits = x @ lm_head.T) against float64."""
    from w4a16 import lm_head

    say(f"lm_head m={m} k={k} n={n}")
    g = torch.Generator().manual_seed(m * 7 + k + n)
    x = torch.randn(m, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16()
    y = lm_head(x.to(DEV), w.to(DEV))
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    ref = x.double().numpy() @ w.double().numpy().T
    check_tolerance(y, ref, f"lm_head {m}x{k}x{n}")


def test_lm_head_shapes_and_errors():
    from w4a16 import _native, lm_head

    say("lm_head shapes and errors")
    x = torch.randn(2, 3, 256).bfloat16().to(DEV)
    w = (torch.randn(512, 256) * 0.02).bfloat16().to(DEV)
    y = lm_head(x, w)
    assert y.shape == (2, 3, 512)
    check_tolerance(y.reshape(6, 512), x.reshape(6, 256).double().cpu().numpy() @ w.double().cpu().numpy().T, "3d")
    big = torch.randn(40, 256).bfloat16().to(DEV)  # M > 16: library GEMM
    assert torch.equal(lm_head(big, w), big @ w.T)
    with pytest.raises(ValueError):
        _native.bf16_gemv(torch.randn(1, 12).bfloat16().to(DEV), torch.randn(4, 12).bfloat16().to(DEV))
    with pytest.raises(TypeError):
        lm_head(x.cpu(), w.cpu())
    z = _native.bf16_gemv(torch.empty(1, 0, dtype=torch.bfloat16, device=DEV),
                          torch.empty(5, 0, dtype=torch.bfloat16, device=DEV))
    assert torch.equal(z.float().cpu(), torch.zeros(1, 5))


def test_lm_head_qwen3_8b_full_size():
    """The real output projection: vocab 151936 x d_model 4096 (1.24 GB bf16), M = 1."""
    from w4a16 import lm_head

    say("lm_head full size")
    g = torch.Generator(device=DEV).manual_seed(5)
    w = (torch.randn(151936, 4096, generator=g, device=DEV) * 0.02).bfloat16()
    x = torch.randn(1, 4096, generator=g, device=DEV).bfloat16()
    y = lm_head(x, w)
    ref = (x.double() @ w.double().T).cpu().numpy()
    assert_parity(y.double().cpu().numpy(), ref, "lm_head full size")
    del w


# ---------------------------------------------------------------------------
# SwiGLU gate/up pair (w4a16_swiglu)
#
# Bar: oracle/tolerance.py against the float64 oracle h64, with r = 1 bf16
# rounding for the fused forms (the decode pair, and the GEMM pair kernel at
# GEMM-sized M: epilogue on the fp32 sums) and r = 6 for the fallback at
# GEMM-sized M (operands not aligned for the pair kernel), which rounds gate
# and up to bf16 before the epilogue as the reference does
# (engine/llama_mlp.py:30-32 rounds each linear output).
# ---------------------------------------------------------------------------

def check_swiglu(h: torch.Tensor, h_ref: np.ndarray, m: int, label: str, roundings: int | None = None) -> None:
    """The parity bar with r = 1 for the fused forms (decode M, and the GEMM pair kernel) and r = 6
    for the grouped GEMM + elementwise form, which rounds gate and up to bf16 first."""
    hv = h.float().cpu().numpy().astype(np.float64)
    if roundings is None:
        roundings = 1 if m <= 32 else 6
    rel = assert_parity(hv, h_ref, label, roundings)
    say(f"  {label}: max(excess)/rms={rel:.3e}")


@pytest.mark.parametrize("m,k,n", [(1, 1024, 1536), (2, 128, 512), (5, 512, 1000), (16, 2048, 768),
                                   (17, 1024, 512), (32, 512, 1024), (33, 1024, 640), (200, 768, 1280)])
def test_swiglu_vs_oracle(m, k, n):
    from w4a16 import int4_swiglu, synth

    say(f"swiglu m={m} k={k} n={n}")
    gate = synth.make_weight(k, n, seed=70 + n)
    up = synth.make_weight(k, n, seed=71 + n)
    x = synth.make_activations(m, k, seed=72 + m)
    h = int4_swiglu(x.to(DEV), *[(p.to(DEV), s.to(DEV)) for p, s in (gate, up)])
    assert h.shape == (m, n) and h.dtype == torch.bfloat16
    check_swiglu(h, orc.swiglu_reference(x.float().numpy(), gate, up), m, f"swiglu M={m} K={k} N={n}")


@pytest.mark.parametrize("case", range(10))
def test_random_swiglu_sweep_vs_oracle(case):
    from w4a16 import int4_swiglu

    rng = np.random.default_rng(SWEEP_SEED + 2000 + case)
    m = int(rng.choice([1, 2, 7, 16, 25, 32, 40, 64, 65, 130, 300]))
    k, n = 128 * int(rng.integers(1, 13)), int(rng.integers(1, 1537))
    say(f"swiglu sweep case={case} m={m} k={k} n={n}")
    g = torch.Generator().manual_seed(SWEEP_SEED + 2000 + case)
    gate, up = [(torch.randint(-128, 128, (k // 2, n), generator=g, dtype=torch.int8),
                 torch.rand(k // 128, n, generator=g) * 0.01 + 0.001) for _ in range(2)]
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    h = int4_swiglu(x.to(DEV), *[(p.to(DEV), sc.to(DEV)) for p, sc in (gate, up)])
    assert h.shape == (m, n) and h.dtype == torch.bfloat16
    check_swiglu(h, orc.swiglu_reference(x.float().numpy(), gate, up), m, f"swiglu sweep {case}: M={m} K={k} N={n}")


@pytest.mark.parametrize("m", [1, 4, 16, 24, 2048])
def test_swiglu_qwen3_8b_full_size(m):
    """gate/up of Qwen3-8B (K=4096, N=12288) against silu(g) * u from two
    int4_matmul calls; M <= 32 also bit-stable over repeats (slots reset)."""
    from w4a16 import int4_matmul, int4_swiglu, synth

    say(f"swiglu full-size M={m}")
    k, n = 4096, 12288
    gate = synth.make_weight(k, n, seed=81, device=DEV)
    up = synth.make_weight(k, n, seed=82, device=DEV)
    x = synth.make_activations(m, k, seed=83, device=DEV)
    h = int4_swiglu(x, gate, up)
    g, u = int4_matmul(x, *gate).double(), int4_matmul(x, *up).double()
    h_ref = (g * torch.sigmoid(g) * u).cpu().numpy()
    # The reference-side g and u are themselves bf16-rounded: r = 6 at every M.
    rel = assert_parity(h.double().cpu().numpy(), h_ref, "vs two int4_matmul", roundings=6)
    say(f"  vs two int4_matmul: max(excess)/rms={rel:.3e}")
    for _ in range(3):
        assert torch.equal(int4_swiglu(x, gate, up), h)
    # Sampled columns against the float64 oracle.  Every M here is a fused form (the decode pair,
    # or at M = 2048 the GEMM pair kernel), which rounds only h: half an ulp.
    cols = torch.randperm(n, generator=torch.Generator().manual_seed(m))[:48].sort().values.to(DEV)
    sub = [(p[:, cols].cpu().numpy(), s[:, cols].cpu().numpy()) for p, s in (gate, up)]
    check_swiglu(h[:, cols], orc.swiglu_reference(x.float().cpu().numpy(), *sub), m, "fp64 oracle, 48 cols",
                 roundings=1)


@pytest.mark.parametrize("m,odd_lds", [(2100, False), (2100, True), (2048, False)])
def test_swiglu_gemm_pair_kernel_and_fallback(m, odd_lds):
    """GEMM-sized SwiGLU: the pair kernel (gate and up column blocks in one workgroup, epilogue on
    fp32 sums) with a partial last row tile, and the grouped GEMM + elementwise fallback that an
    odd scale row stride selects.  Both against the float64 oracle on sampled columns."""
    from w4a16 import int4_swiglu, synth

    k, n = 256, 2048  # 17 x 16 tiles of 128 x 128 at M = 2100: one full round and a partial row tile
    say(f"swiglu gemm pair m={m} odd_lds={odd_lds}")
    gate = synth.make_weight(k, n, seed=91, device=DEV)
    up = synth.make_weight(k, n, seed=92, device=DEV)
    if odd_lds:
        wide = torch.zeros(k // 128, n + 1, device=DEV)
        wide[:, :n] = gate[1]
        gate = (gate[0], wide[:, :n])
    x = synth.make_activations(m, k, seed=93, device=DEV)
    h = int4_swiglu(x, gate, up)
    assert torch.equal(int4_swiglu(x, gate, up), h)
    cols = torch.randperm(n, generator=torch.Generator().manual_seed(7))[:64].sort().values.to(DEV)
    sub = [(p[:, cols].cpu().numpy(), s[:, cols].contiguous().cpu().numpy()) for p, s in (gate, up)]
    ref = orc.swiglu_reference(x.float().cpu().numpy(), *sub)
    check_swiglu(h[:, cols], ref, m, f"M={m} {'fallback' if odd_lds else 'pair kernel'}",
                 roundings=6 if odd_lds else 1)


def test_swiglu_shares_workspace_and_edge_cases():
    """Interleaved swiglu / linear calls on one workspace stay bit-stable; empty
    and K = 0 inputs; unaligned activations; shape mismatch raises."""
    from w4a16 import int4_matmul, int4_swiglu

    x1, g1, s1 = rand_problem(1, 4096, 12288, seed=11)
    _, u1, t1 = rand_problem(1, 4096, 12288, seed=12)
    x2, p2, q2 = rand_problem(64, 1024, 512, seed=13)
    h0 = int4_swiglu(x1, (g1, s1), (u1, t1))
    y0 = int4_matmul(x2, p2, q2)
    y1 = int4_matmul(x1, g1, s1)
    for _ in range(3):
        assert torch.equal(int4_swiglu(x1, (g1, s1), (u1, t1)), h0)
        assert torch.equal(int4_matmul(x2, p2, q2), y0)
        assert torch.equal(int4_matmul(x1, g1, s1), y1)
    e = int4_swiglu(torch.empty(0, 4096, dtype=torch.bfloat16, device=DEV), (g1, s1), (u1, t1))
    assert e.shape == (0, 12288)
    z = torch.empty(0, 64, dtype=torch.int8, device=DEV)
    zs = torch.empty(0, 64, device=DEV)
    h = int4_swiglu(torch.empty(3, 0, dtype=torch.bfloat16, device=DEV), (z, zs), (z, zs))
    assert h.shape == (3, 64) and torch.count_nonzero(h) == 0
    for m in (3, 40):
        x, gp, gs = rand_problem(m, 512, 256, seed=20 + m)
        _, up, us = rand_problem(m, 512, 256, seed=30 + m)
        flat = torch.zeros(m * 512 + 1, dtype=torch.bfloat16, device=DEV)
        xu = flat[1:].view(m, 512)
        xu.copy_(x)
        ref = orc.swiglu_reference(x.float().cpu().numpy(), (gp.cpu().numpy(), gs.cpu().numpy()),
                                   (up.cpu().numpy(), us.cpu().numpy()))
        check_swiglu(int4_swiglu(xu, (gp, gs), (up, us)), ref, m, f"unaligned M={m}")
    with pytest.raises(ValueError):
        int4_swiglu(x1, (g1, s1), (u1[:, :1024], t1[:, :1024]))


def test_swiglu_mlp_layer_matches_unfused():
    """swiglu_mlp with INT4 weights is down(int4_swiglu(x)): h meets the bar
    against the float64 oracle, the block output equals linear(h, down) bit
    for bit, and that output meets the bar against the float64 product of h."""
    from w4a16 import _Int4Weight, int4_swiglu, linear, swiglu_mlp, synth

    k, n = 512, 768
    ws = {}
    for name, (kk, nn), seed in (("gate", (k, n), 1), ("up", (k, n), 2), ("down", (n, k), 3)):
        p, s = synth.make_weight(kk, nn, seed=600 + seed, device=DEV)
        ws[f"mlp.{name}_proj.weight"] = _Int4Weight(p, s, 128, (nn, kk))
    g_w, u_w, d_w = (ws[f"mlp.{p}_proj.weight"] for p in ("gate", "up", "down"))
    for m in (1, 48):
        x = synth.make_activations(2 * m, k, seed=610 + m, device=DEV).reshape(2, m, k)
        out = swiglu_mlp(x, ws)
        assert out.shape == (2, m, k)
        xf = x.reshape(-1, k)
        h = int4_swiglu(xf, (g_w.packed, g_w.scale), (u_w.packed, u_w.scale))
        h64 = orc.swiglu_reference(xf.float().cpu().numpy(), (g_w.packed.cpu().numpy(), g_w.scale.cpu().numpy()),
                                   (u_w.packed.cpu().numpy(), u_w.scale.cpu().numpy()))
        check_swiglu(h, h64, 2 * m, f"swiglu_mlp h m={m}")
        assert torch.equal(out.reshape(-1, k), linear(h, d_w))
        y64 = orc.fused_reference(h.float().cpu().numpy(), d_w.packed.cpu().numpy(), d_w.scale.cpu().numpy())
        check_tolerance(out.reshape(-1, k), y64, f"swiglu_mlp out m={m}")


def test_qkv_projections_grouped_matches_linear():
    """qkv_projections (one grouped launch) equals three linear() calls; decode
    sizes bit for bit (same decode arithmetic), prefill sizes to the bar."""
    from w4a16 import _Int4Weight, linear, qkv_projections, synth

    d, nq, nkv = 512, 512, 128
    ws = {}
    for name, n, seed in (("q", nq, 1), ("k", nkv, 2), ("v", nkv, 3)):
        p, s = synth.make_weight(d, n, seed=700 + seed, device=DEV)
        ws[f"self_attn.{name}_proj.weight"] = _Int4Weight(p, s, 128, (n, d))
    for m in (1, 3, 96):
        x = synth.make_activations(2 * m, d, seed=710 + m, device=DEV).reshape(2, m, d)
        q, k, v = qkv_projections(x, ws)
        for out, name, n in ((q, "q", nq), (k, "k", nkv), (v, "v", nkv)):
            assert out.shape == (2, m, n)
            ref = linear(x, ws[f"self_attn.{name}_proj.weight"])
            if m <= 16:
                assert torch.equal(out, ref), (name, m)
            else:
                w = ws[f"self_attn.{name}_proj.weight"]
                y64 = orc.fused_reference(x.reshape(-1, d).float().cpu().numpy(), w.packed.cpu().numpy(),
                                          w.scale.cpu().numpy())
                check_tolerance(out.reshape(-1, n), y64, f"qkv {name} M={2 * m}")
