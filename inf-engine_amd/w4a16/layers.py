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


def silu(x: torch.Tensor) -> torch.Tensor:
    """x * sigmoid(x) (engine/layers.py:28-30)."""
    return x * torch.sigmoid(x)


def swiglu_mlp(x: torch.Tensor, weights: dict) -> torch.Tensor:
    """``down(silu(gate(x)) * up(x))`` -- the SwiGLU block of engine/llama_mlp.py:19-33.

    When gate and up are INT4 weights (group size 128) on a HIP device, the
    pair runs as one fused ``int4_swiglu`` call; anything else follows the
    reference's three ``linear`` calls.
    """
    from .quant import int4_swiglu

    g, u, d = weights["mlp.gate_proj.weight"], weights["mlp.up_proj.weight"], weights["mlp.down_proj.weight"]
    fused = (
        all(hasattr(w, "packed") and getattr(w, "group_size", None) == 128 for w in (g, u))
        and x.is_cuda and g.shape == u.shape
    )
    if not fused:
        return linear(silu(linear(x, g)) * linear(x, u), d)
    lead = x.shape[:-1]
    h = int4_swiglu(x.reshape(-1, x.shape[-1]), (g.packed, g.scale), (u.packed, u.scale), g.group_size)
    return linear(h.reshape(*lead, g.shape[0]), d)


def qkv_projections(x: torch.Tensor, weights: dict) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``q, k, v = linear(x, W_q), linear(x, W_k), linear(x, W_v)`` (engine/llama_attention.py:83-85).

    With INT4 weights (group size 128) on a HIP device the three projections
    share one grouped launch (``int4_matmul_grouped``); otherwise three
    ``linear`` calls as in the reference.  Shapes as the reference:
    ``x (..., d_model)`` -> ``(..., d_out)`` each.
    """
    from .quant import int4_matmul_grouped

    ws = [weights[f"self_attn.{n}_proj.weight"] for n in ("q", "k", "v")]
    fused = all(hasattr(w, "packed") and getattr(w, "group_size", None) == 128 for w in ws) and x.is_cuda
    if not fused:
        return tuple(linear(x, w) for w in ws)
    lead = x.shape[:-1]
    outs = int4_matmul_grouped(x.reshape(-1, x.shape[-1]), [(w.packed, w.scale) for w in ws], 128)
    return tuple(o.reshape(*lead, w.shape[0]) for o, w in zip(outs, ws))


def lm_head(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Logits ``x @ weight.T`` for a dense bf16 ``weight[vocab, d_model]`` (engine/llama_model.py:148).

    Decode-sized inputs (at most 16 rows after flattening the leading
    dimensions) run the HBM-bound bf16 GEMV kernel of ``libw4a16.so``; larger
    inputs, where the product is a plain GEMM, use torch's library GEMM.
    Device tensors only.
    """
    from . import _native

    if not x.is_cuda or not weight.is_cuda:
        raise TypeError("w4a16.lm_head runs only on HIP device tensors")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError(f"lm_head expects bf16 activations and weight, got {x.dtype} and {weight.dtype}")
    lead = x.shape[:-1]
    a = x.reshape(-1, x.shape[-1])
    if a.shape[0] > 16:
        return (a @ weight.T).reshape(*lead, weight.shape[0])
    with torch.cuda.device(a.device):
        return _native.bf16_gemv(a, weight).reshape(*lead, weight.shape[0])
