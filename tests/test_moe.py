"""MoE MLP with batched INT4 experts (w4a16.moe) against a per-expert loop.

``per_expert_moe`` restates the reference's algorithm (engine/llama_moe.py:44-105):
shared expert, softmax router, renormalised top-K, and one SwiGLU per active
expert accumulated in ascending expert order.  It issues one projection call
per expert, the reference's launch pattern, through whichever ``linear`` it is
given.
"""

from __future__ import annotations

import types

import numpy as np
import pytest
import torch

from oracle import int4_oracle as orc


def per_expert_moe(x, weights, config, linear):
    S = x.shape[0] * x.shape[1]
    xf = x.reshape(S, -1)

    def swiglu(h, g, u, d):
        a, b = linear(h, g), linear(h, u)
        return linear(a * torch.sigmoid(a) * b, d)

    out = torch.zeros_like(xf)
    if "mlp.shared_expert.gate_proj.weight" in weights:
        out = out + swiglu(xf, *(weights[f"mlp.shared_expert.{p}_proj.weight"] for p in ("gate", "up", "down")))
    probs = torch.softmax(linear(xf, weights["mlp.gate.weight"]), dim=-1)
    w, ids = torch.topk(probs, config.n_experts_per_tok, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    routed = torch.zeros_like(xf)
    for e in sorted(set(ids.flatten().tolist())):
        tw = ((ids == e) * w).sum(dim=-1)
        sel = tw > 0
        if sel.any():
            y = swiglu(xf[sel], *(weights[f"mlp.experts.{e}.{p}_proj.weight"] for p in ("gate", "up", "down")))
            routed[sel] += y * tw[sel, None]
    return (out + routed).reshape(x.shape)


def _moe_block(d=256, inter=128, n_experts=8, shared=True, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    w = {"mlp.gate.weight": (torch.randn(n_experts, d, generator=g) * 0.5).to(dtype)}
    names = [f"mlp.experts.{e}" for e in range(n_experts)] + (["mlp.shared_expert"] if shared else [])
    for nm in names:
        w[f"{nm}.gate_proj.weight"] = (torch.randn(inter, d, generator=g) * 0.05).to(dtype)
        w[f"{nm}.up_proj.weight"] = (torch.randn(inter, d, generator=g) * 0.05).to(dtype)
        w[f"{nm}.down_proj.weight"] = (torch.randn(d, inter, generator=g) * 0.05).to(dtype)
    return w


@pytest.mark.parametrize("shared", [True, False])
def test_moe_routing_matches_per_expert_loop_dense(shared):
    """Dense experts on the CPU: same routing and accumulation order, so identical results."""
    from w4a16 import linear
    from w4a16.moe import moe_mlp

    cfg = types.SimpleNamespace(n_experts_per_tok=3)
    w = _moe_block(shared=shared)
    x = torch.randn(2, 5, 256, generator=torch.Generator().manual_seed(1))
    assert torch.equal(moe_mlp(x, w, cfg), per_expert_moe(x, w, cfg, linear))


def _quantized(w, device):
    from w4a16.quantize import _quantize_projection

    out = {}
    for k, v in w.items():
        if k == "mlp.gate.weight":
            out[k] = v.to(device, torch.bfloat16)
        else:
            q = _quantize_projection(v, 128)
            q.packed, q.scale = q.packed.to(device), q.scale.to(device)
            out[k] = q
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("tokens", [1, 6, 64])
def test_moe_int4_batched_matches_per_expert_calls(tokens):
    """INT4 experts on the GPU: grouped launches vs one int4_matmul per projection,
    and both against float64 dequantize-then-matmul of each expert's output."""
    from w4a16 import linear
    from w4a16.moe import experts_forward, moe_mlp

    print(f"moe int4 tokens={tokens}", flush=True)
    cfg = types.SimpleNamespace(n_experts_per_tok=4)
    w = _quantized(_moe_block(n_experts=16, seed=tokens), "cuda:0")
    x = (torch.randn(1, tokens, 256, generator=torch.Generator().manual_seed(2))).bfloat16().to("cuda:0")
    got = moe_mlp(x, w, cfg).float()
    ref = per_expert_moe(x, w, cfg, linear).float()
    rms = ref.pow(2).mean().sqrt().item()
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max().item() <= 2e-2 * rms, "grouped vs per-expert launches"

    # Expert outputs themselves: each within the kernel tolerance of the oracle.
    xs = [x.reshape(-1, 256)[: max(1, tokens // (i + 1))] for i in range(3)]
    experts = [tuple(w[f"mlp.experts.{e}.{p}_proj.weight"] for p in ("gate", "up", "down")) for e in range(3)]
    outs = experts_forward(xs, experts)
    for xi, (g, u, d), y in zip(xs, experts, outs):
        xn = xi.float().cpu().numpy()
        a = orc.fused_reference(xn, g.packed.cpu().numpy(), g.scale.cpu().numpy())
        b = orc.fused_reference(xn, u.packed.cpu().numpy(), u.scale.cpu().numpy())
        a_bf = torch.from_numpy(a).float().bfloat16()
        b_bf = torch.from_numpy(b).float().bfloat16()
        h = (a_bf * torch.sigmoid(a_bf) * b_bf).float().numpy()
        yr = orc.fused_reference(h, d.packed.cpu().numpy(), d.scale.cpu().numpy())
        r = float(np.sqrt(np.mean(yr ** 2)))
        assert np.abs(y.float().cpu().numpy() - yr).max() <= 2e-2 * r
