"""Projection dispatch -- the ``linear`` primitive of engine/layers.py:33-50."""

from __future__ import annotations

import torch


def linear(x: torch.Tensor, weight) -> torch.Tensor:
    """``y = x @ W.T``; INT4 weights (anything with ``fused_linear``) take the fused kernel.

    Same duck-typed dispatch as engine/layers.py:48-50: an ``_Int4Weight``
    routes to ``fused_linear`` (the HIP W4A16 kernel), a dense ``(d_out, d_in)``
    tensor to a plain matmul.
    """
    if hasattr(weight, "fused_linear"):
        return weight.fused_linear(x)
    return x @ weight.T
