"""CPU oracle for the INT4 W4A16 path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of bench.py
may import this module, and only as the checker (or, for cpu_baseline, as the
timed stand-in for the reference's CPU path).  The product package ``w4a16``
never imports it: its contraction runs only in the HIP kernels.

Contents, each restating the reference's algorithm:

* ``unpack_nibbles``  -- engine/kernels/quant.py:140-150 (int8 arithmetic shifts)
* ``quantize``        -- engine/kernels/quant.py:81-119
* ``dequantize``      -- engine/kernels/quant.py:122-156
* ``fused_reference`` -- the value _int4_matmul_kernel computes
                         (engine/kernels/quant.py:186-238) in float64
* ``cpu_path``        -- the reference's CPU branch of int4_matmul
                         (engine/kernels/quant.py:264-266) in torch on the host
* ``silu`` / ``swiglu_reference`` -- silu (engine/layers.py:28-30) and the
                         gate/up half of the SwiGLU MLP, silu(x @ Wg) * (x @ Wu)
                         (engine/llama_mlp.py:30-32), in float64

Byte and integer work is numpy; the CPU path is torch on the host because that
is what the reference runs there.

How each function is pinned (tests/test_oracle.py):
  unpack_nibbles   exhaustively against the 4-bit two's complement definition
                   for all 256 byte values, and against the golden fixture.
  quantize         reference invariants (test_int4_quant.py:35-95: round-trip
                   error <= scale/2, lossless integer packing, ratio > 3.5),
                   round-half-to-even ties, amax -> +-7, and bit-exact agreement
                   with an independent element-by-element Python restatement
                   (both division rules); the device rule itself is checked
                   against torch on the GPU (tests/test_gpu_contract.py).
  dequantize       scale indexing with distinct power-of-two scales per
                   (group, column) and all-ones codes (any index slip is
                   bit-visible), and the golden fixture.
  fused_reference  brute-force triple loop on small integer problems (exact),
                   and the closed form for one-hot activations.
  silu             closed forms: silu(0) = 0, silu(x) - silu(-x) = x,
                   silu(x) -> x (x -> +inf) and -> 0 (x -> -inf), silu(ln 3)
                   = 0.75 ln 3; swiglu_reference against fused_reference
                   with an all-ones-sum up weight (u = sum of x).
  cpu_path         test_int4_quant.py:67-82 bound (rel. error < 0.25 vs the
                   unquantized product) and agreement with fused_reference
                   within bf16 rounding.
"""

from __future__ import annotations

import numpy as np

INT4_MAX = 7


def unpack_nibbles(packed: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(even_rows, odd_rows) int8 codes in [-8, 7] from packed int8 bytes.

    quant.py:141: ``high = packed >> 4`` on int8 (arithmetic shift);
    quant.py:145-146: ``low = ((packed & 0xF).to(int8) << 4) >> 4``.
    """
    p = np.asarray(packed).astype(np.int8, copy=False)
    high = (p >> 4).astype(np.int8)
    low = ((p & np.int8(0x0F)).astype(np.int8) << 4).astype(np.int8) >> 4
    return high, low.astype(np.int8)


def codes(packed: np.ndarray) -> np.ndarray:
    """Full [K, N] int8 code matrix: row 2i = high nibble, row 2i+1 = low nibble."""
    high, low = unpack_nibbles(packed)
    k_half, n = high.shape
    out = np.empty((2 * k_half, n), dtype=np.int8)
    out[0::2] = high
    out[1::2] = low
    return out


def quantize(w: np.ndarray, group_size: int = 128, device_division: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric per-group INT4 quantization of w[d_in, d_out] (float32).

    Steps of quant.py:99-119: scale = max(amax_group|w| / 7, 1e-8) in float32;
    q = clip(round_half_even(w / scale), -7, 7); byte i = (q[2i] & 0xF) << 4 |
    (q[2i+1] & 0xF).

    ``device_division``: the same op sequence as torch runs it on a GPU
    tensor.  torch's device kernel for ``tensor / python_scalar`` multiplies by
    the float32 reciprocal of the scalar instead of dividing (its true-division
    kernel's CPU-scalar fast path), so the scale line ``amax / 7``
    (quant.py:108) becomes ``amax * float32(1 / 7)``, which differs from the
    quotient by one ulp for some amax.  ``w / scale`` (tensor by tensor) stays a
    true division.  The reference quantizes on the GPU for models up to 8B
    (main.py:474-478), so that is what its bytes are there.
    """
    w = np.asarray(w, dtype=np.float32)
    d_in, d_out = w.shape
    if d_in % group_size != 0:
        raise ValueError(f"d_in={d_in} not divisible by group_size={group_size}")
    if d_in % 2 != 0:
        raise ValueError(f"d_in={d_in} must be even for nibble packing")
    g = d_in // group_size
    wg = w.reshape(g, group_size, d_out)
    amax = np.abs(wg).max(axis=1)
    if device_division:
        scale = (amax * (np.float32(1.0) / np.float32(INT4_MAX))).astype(np.float32)
    else:
        scale = (amax / np.float32(INT4_MAX)).astype(np.float32)
    scale = np.maximum(scale, np.float32(1e-8))
    q = np.rint(wg / scale[:, None, :]).clip(-INT4_MAX, INT4_MAX).astype(np.int8).reshape(d_in, d_out)
    even = (q[0::2] & 0x0F).astype(np.uint8)
    odd = (q[1::2] & 0x0F).astype(np.uint8)
    packed = ((even << 4) | odd).astype(np.uint8).view(np.int8)
    return packed, scale


def dequantize(packed: np.ndarray, scale: np.ndarray, group_size: int = 128) -> np.ndarray:
    """w[k, n] = q[k, n] * scale[k // group_size, n], in scale's dtype (quant.py:148-156)."""
    q = codes(packed)
    d_in, d_out = q.shape
    g = d_in // group_size
    s = np.asarray(scale)
    w = q.reshape(g, group_size, d_out).astype(s.dtype) * s[:, None, :]
    return w.reshape(d_in, d_out)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16, returned as float32 (torch's rounding rule)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out)


def dequantize_bf16(packed: np.ndarray, scale: np.ndarray, group_size: int = 128) -> np.ndarray:
    """dequantize_weight_int4(packed, scale.to(bfloat16)): bf16 scale, bf16 product (as float32)."""
    s = bf16_round(np.asarray(scale, dtype=np.float32))
    return bf16_round(dequantize(packed, s, group_size))


def fused_reference(x: np.ndarray, packed: np.ndarray, scale: np.ndarray, group_size: int = 128) -> np.ndarray:
    """y = x @ (q * scale) in float64: the exact value the fused kernel approximates.

    x holds the bf16 activations as float32/float64 values.  In float64 the
    group-wise order of quant.py:221-234 (per-group dot, times scale, summed)
    and a plain dense product differ only by float64 rounding.
    """
    w = dequantize(packed, np.asarray(scale, dtype=np.float64), group_size)
    return np.asarray(x, dtype=np.float64) @ w


def silu(v: np.ndarray) -> np.ndarray:
    """v * sigmoid(v) in float64 (engine/layers.py:28-30), overflow-free for large |v|."""
    v = np.asarray(v, dtype=np.float64)
    e = np.exp(-np.abs(v))
    sig = np.where(v >= 0, 1.0 / (1.0 + e), e / (1.0 + e))
    return v * sig


def swiglu_reference(x: np.ndarray, gate: tuple, up: tuple, group_size: int = 128) -> np.ndarray:
    """h = silu(x @ Wg) * (x @ Wu) in float64 (engine/llama_mlp.py:30-32).

    gate and up are (packed, scale) pairs; each product is fused_reference.
    """
    g = fused_reference(x, gate[0], gate[1], group_size)
    u = fused_reference(x, up[0], up[1], group_size)
    return silu(g) * u


def cpu_path(x, packed, scale, group_size: int = 128):
    """The reference's host branch of int4_matmul (quant.py:264-266), in torch on the CPU.

    ``w = dequantize(packed, scale.to(x.dtype))`` then ``x @ w``.  Inputs are
    torch tensors; used as the CPU baseline that bench.py times.
    """
    import torch

    even = packed >> 4
    odd = ((packed & 0x0F).to(torch.int8) << 4) >> 4
    k_half, n = packed.shape
    q = torch.stack((even, odd), dim=1).reshape(2 * k_half, n)
    s = scale.to(x.dtype)
    w = (q.reshape(-1, group_size, n).to(s.dtype) * s[:, None, :]).reshape(2 * k_half, n)
    return x @ w
