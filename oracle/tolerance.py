"""The parity bar of the fused W4A16 outputs -- TEST INFRASTRUCTURE ONLY
(imported by tests/ and ``__graft_entry__.smoke()``, never by the product).

One bar for every floating-point output of the path:

    max over elements of  |y - y_ref| - r * ulp_bf16(y_ref) / 2   <=   1e-3 * RMS(y_ref)

* ``y_ref`` is the exact (float64) value of the same packed weights, scales
  and bf16 activations (oracle.int4_oracle.fused_reference and friends).
* ``r`` is the number of bf16 roundings the reference itself applies on the
  way to ``y``: 1 for every single projection (the output store), for the
  lm_head GEMV and for the fused SwiGLU forms, which round only h.  The
  GEMM-sized SwiGLU fallback rounds gate and up to bf16 before
  ``silu(g) * u`` as the reference does (engine/llama_mlp.py:30-32): the
  rounding of g reaches h scaled by at most |g silu'(g) / silu(g)| <= 4 and
  that of u by 1, so r = 1 + 2 * (4 + 1) / 2 rounded up: 6.
* ``1e-3 * RMS`` is ten times tighter than the north-star bound
  ``max|y - y_ref| <= 1e-2 * RMS(y_ref)``.  The ulp term is needed because a
  bf16 output alone cannot meet 1e-2 * RMS at elements above ~2.5 RMS (half a
  bf16 ulp is 2^-9 relative), which the reference's kernel could not meet
  either.
"""

from __future__ import annotations

import numpy as np

RMS_FRACTION = 1e-3


def ulp_bf16(v) -> np.ndarray:
    """Spacing of bfloat16 values at |v| (normal range; 2^-133 floor)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.ldexp(1.0, (e - 7).astype(np.int64))


def excess(y, y_ref, roundings: int = 1) -> tuple[float, float]:
    """(max excess over the ulp allowance, RMS of y_ref)."""
    yv = np.asarray(y, dtype=np.float64)
    ref = np.asarray(y_ref, dtype=np.float64)
    rms = float(np.sqrt(np.mean(ref ** 2))) if ref.size else 0.0
    if not ref.size:
        return 0.0, rms
    ex = np.abs(yv - ref) - roundings * ulp_bf16(ref) / 2
    return float(np.max(ex)), rms


def assert_parity(y, y_ref, label: str = "", roundings: int = 1) -> float:
    """Raise AssertionError unless y meets the bar; returns max excess / RMS."""
    yv = np.asarray(y, dtype=np.float64)
    if not np.isfinite(yv).all():
        raise AssertionError(f"{label}: non-finite output")
    ex, rms = excess(yv, y_ref, roundings)
    if not ex <= RMS_FRACTION * rms:
        raise AssertionError(f"{label}: max excess {ex:.4g} > {RMS_FRACTION:g} * RMS ({rms:.4g})")
    return ex / rms if rms else 0.0
