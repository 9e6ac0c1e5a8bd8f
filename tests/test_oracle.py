"""Pins the CPU oracle (oracle/int4_oracle.py) before anything is checked against it.

Checks come from the reference's own tests (tests/test_int4_quant.py:35-95),
from the golden fixture written element by element from the format's
definition (tests/golden/make_golden.py), from closed forms (4-bit two's
complement, round-half-to-even) and from brute force on small inputs.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import int4_oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "int4_golden.npz")


def twos_complement_4bit(v: int) -> int:
    return v - 16 if v & 0x8 else v


def test_unpack_exhaustive_all_256_bytes():
    """Every byte: high nibble -> even row, low nibble -> odd row, sign-extended."""
    b = np.arange(256, dtype=np.uint8).view(np.int8).reshape(256, 1)
    hi, lo = orc.unpack_nibbles(b)
    for v in range(256):
        assert int(hi[v, 0]) == twos_complement_4bit(v >> 4), v
        assert int(lo[v, 0]) == twos_complement_4bit(v & 0xF), v
    # -8 (nibble 0x8) is decodable although the quantizer never emits it.
    assert hi.min() == -8 and lo.min() == -8 and hi.max() == 7 and lo.max() == 7


def test_golden_fixture_codes_dequant_and_product():
    g = np.load(GOLDEN)
    gs = int(g["group_size"])
    np.testing.assert_array_equal(orc.codes(g["packed"]), g["codes"])
    np.testing.assert_array_equal(orc.dequantize(g["packed"], g["scale"], gs), g["dequant"])
    np.testing.assert_array_equal(orc.fused_reference(g["x"], g["packed"], g["scale"], gs), g["y"])


@pytest.mark.parametrize("d_in,d_out,gs", [(256, 128, 128), (512, 256, 128), (1024, 512, 64)])
def test_roundtrip_error_bound(d_in, d_out, gs):
    """test_int4_quant.py:35-52: max |w - w_hat| <= max_scale / 2."""
    torch.manual_seed(0)
    w = torch.randn(d_in, d_out).numpy()
    packed, scale = orc.quantize(w, gs)
    w_hat = orc.dequantize(packed, scale, gs)
    assert np.abs(w - w_hat).max() <= np.abs(scale).max() / 2 + 1e-6


def test_nibble_packing_lossless():
    """test_int4_quant.py:55-64: integers in [-7, 7] with max 7 round-trip exactly."""
    torch.manual_seed(1)
    w = torch.randint(-7, 8, (128, 64)).float().numpy()
    w[0, :] = 7.0  # amax 7 in every column -> scale exactly 1
    packed, scale = orc.quantize(w, 128)
    assert np.all(scale == 1.0)
    np.testing.assert_array_equal(orc.dequantize(packed, scale, 128), w)


def test_compression_ratio():
    """test_int4_quant.py:85-95."""
    w = np.random.default_rng(0).standard_normal((4096, 4096)).astype(np.float32)
    packed, scale = orc.quantize(w, 128)
    ratio = w.nbytes / (packed.nbytes + scale.size * 2)
    assert ratio > 3.5


def test_quantize_round_half_even_and_amax():
    """Ties go to even (torch.round), the amax element maps to +-7, codes clamp at 7."""
    col = np.zeros(128, dtype=np.float32)
    col[:8] = [7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]
    packed, scale = orc.quantize(col.reshape(128, 1), 128)
    assert scale[0, 0] == np.float32(1.0)
    q = orc.codes(packed)[:8, 0].tolist()
    assert q == [7, 0, 2, 2, 0, -2, -2, 4]
    # Negative amax -> -7; every other code within [-7, 7].
    w = np.random.default_rng(3).standard_normal((256, 16)).astype(np.float32)
    w[5, 3] = -50.0
    packed, scale = orc.quantize(w, 128)
    c = orc.codes(packed)
    assert c[5, 3] == -7 and np.abs(c).max() == 7
    assert np.all(np.abs(c).max(axis=0) == 7)


@pytest.mark.parametrize("device_division", [False, True])
def test_quantize_matches_elementwise_restatement(device_division):
    """Bit-exact against an element-by-element restatement of quant.py:105-118
    (host division, or torch's device rule amax * float32(1/7) for the scale)."""
    rng = np.random.default_rng(7)
    d_in, d_out, gs = 256, 24, 128
    w = (rng.standard_normal((d_in, d_out)) * 0.02).astype(np.float32)
    packed, scale = orc.quantize(w, gs, device_division=device_division)
    inv7 = np.float32(1.0) / np.float32(7.0)
    for g in range(d_in // gs):
        for n in range(d_out):
            amax = np.float32(max(abs(float(v)) for v in w[g * gs:(g + 1) * gs, n]))
            q7 = np.float32(amax * inv7) if device_division else np.float32(amax / np.float32(7.0))
            s = max(q7, np.float32(1e-8))
            assert scale[g, n] == s
            for r in range(gs):
                k = g * gs + r
                qv = int(np.clip(np.rint(np.float32(w[k, n] / s)), -7, 7))
                byte = int(packed[k // 2, n]) & 0xFF
                nib = (byte >> 4) if k % 2 == 0 else (byte & 0xF)
                assert nib == (qv & 0xF), (k, n)


def test_scale_indexing_distinct_powers_of_two():
    """All-ones codes and a distinct power-of-two scale per (group, column):
    dequant[k, n] must equal scale[k // gs, n] exactly, so any index slip shows."""
    for gs, d_in, d_out in [(128, 512, 8), (64, 256, 5)]:
        groups = d_in // gs
        packed = np.full((d_in // 2, d_out), 0x11, dtype=np.uint8).view(np.int8)
        e = np.arange(groups * d_out).reshape(groups, d_out)
        scale = np.ldexp(np.float32(1.0), -(e % 60) - 1).astype(np.float32)
        w = orc.dequantize(packed, scale, gs)
        for k in range(d_in):
            np.testing.assert_array_equal(w[k], scale[k // gs])


def test_fused_reference_brute_force():
    """Triple loop with per-group partials (quant.py:188-234) on integer data: exact."""
    rng = np.random.default_rng(11)
    for m, k, n in [(1, 128, 16), (3, 256, 7), (4, 384, 5)]:
        packed = rng.integers(0, 256, size=(k // 2, n), dtype=np.uint8).view(np.int8)
        scale = np.ldexp(np.float32(1.0), rng.integers(-6, 3, size=(k // 128, n))).astype(np.float32)
        x = rng.integers(-5, 6, size=(m, k)).astype(np.float32)
        q = [[twos_complement_4bit((int(packed[kk // 2, j]) & 0xFF) >> (4 if kk % 2 == 0 else 0) & 0xF)
              for j in range(n)] for kk in range(k)]
        y = orc.fused_reference(x, packed, scale)
        for i in range(m):
            for j in range(n):
                acc = 0.0
                for g in range(k // 128):
                    part = sum(int(x[i, kk]) * q[kk][j] for kk in range(g * 128, (g + 1) * 128))
                    acc += part * float(scale[g, j])
                assert y[i, j] == acc


def test_fused_reference_one_hot_closed_form():
    """x = e_k picks row k: y[m, n] = q[k_m, n] * scale[k_m // 128, n]."""
    rng = np.random.default_rng(5)
    k, n = 512, 33
    packed = rng.integers(0, 256, size=(k // 2, n), dtype=np.uint8).view(np.int8)
    scale = rng.standard_normal((k // 128, n)).astype(np.float32)
    rows = [0, 1, 127, 128, 255, 256, 511]
    x = np.zeros((len(rows), k), dtype=np.float32)
    for i, r in enumerate(rows):
        x[i, r] = 1.0
    y = orc.fused_reference(x, packed, scale)
    c = orc.codes(packed)
    for i, r in enumerate(rows):
        np.testing.assert_array_equal(y[i], c[r].astype(np.float64) * scale[r // 128].astype(np.float64))


def test_bf16_round_matches_torch():
    v = np.random.default_rng(2).standard_normal(100000).astype(np.float32) * 100
    v[:4] = [np.inf, -np.inf, 0.0, -0.0]
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(orc.bf16_round(v), ref)


def test_cpu_path_reference_bound_and_agreement():
    """test_int4_quant.py:67-82 bound, and the torch CPU path agrees with float64."""
    torch.manual_seed(2)
    m, d_in, d_out = 4, 256, 128
    w = torch.randn(d_in, d_out)
    a = torch.randn(m, d_in)
    packed, scale = orc.quantize(w.numpy(), 128)
    out = orc.cpu_path(a, torch.from_numpy(packed), torch.from_numpy(scale))
    ref = a @ w
    assert ((ref - out).norm() / ref.norm()).item() < 0.25
    y64 = orc.fused_reference(a.numpy(), packed, scale)
    np.testing.assert_allclose(out.numpy(), y64, rtol=1e-5, atol=1e-4)
    # bf16 activations: the reference rounds the scale to bf16 first (quant.py:265).
    ab = a.to(torch.bfloat16)
    outb = orc.cpu_path(ab, torch.from_numpy(packed), torch.from_numpy(scale))
    assert outb.dtype == torch.bfloat16
    wb = orc.dequantize_bf16(packed, scale)
    yb = ab.float().numpy().astype(np.float64) @ wb.astype(np.float64)
    err = np.abs(outb.float().numpy() - yb).max()
    assert err <= 2e-2 * np.sqrt(np.mean(yb ** 2)) + 1e-6


def test_silu_closed_forms():
    v = np.linspace(-30.0, 30.0, 601)
    s = orc.silu(v)
    assert orc.silu(np.array([0.0]))[0] == 0.0
    # x*sigma(x) - (-x)*sigma(-x) = x*(sigma(x) + sigma(-x)) = x
    np.testing.assert_allclose(s - orc.silu(-v), v, rtol=0, atol=1e-12)
    # sigma(ln 3) = 3/4
    assert abs(orc.silu(np.array([np.log(3.0)]))[0] - 0.75 * np.log(3.0)) < 1e-15
    # limits: -> x for large x, -> 0 (from below) for very negative x, finite at +-1000
    assert abs(orc.silu(np.array([40.0]))[0] - 40.0) < 1e-12
    assert -1e-12 < orc.silu(np.array([-40.0]))[0] < 0
    assert np.isfinite(orc.silu(np.array([-1000.0, 1000.0]))).all()


def test_swiglu_reference_with_summing_up_weight():
    """Up weight with every code 1 and scale 1 makes u the row sum of x, so
    h = silu(x @ Wg) * sum(x) exactly; a swapped gate/up or a dropped silu fails."""
    rng = np.random.default_rng(5)
    k, n, m = 256, 24, 3
    gp = rng.integers(-128, 128, (k // 2, n), dtype=np.int8)
    gs = rng.uniform(0.001, 0.01, (k // 128, n)).astype(np.float32)
    up = np.full((k // 2, n), 0x11, dtype=np.int8)
    us = np.ones((k // 128, n), dtype=np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    h = orc.swiglu_reference(x, (gp, gs), (up, us))
    g = orc.fused_reference(x, gp, gs)
    want = g / (1.0 + np.exp(-g)) * x.astype(np.float64).sum(1, keepdims=True)
    np.testing.assert_allclose(h, want, rtol=1e-12, atol=1e-12)
    assert not np.allclose(h, orc.swiglu_reference(x, (up, us), (gp, gs)))
