"""Seeded synthetic problems on the benchmark shapes (no checkpoints are available).

Weights follow the recipe of the benchmark configs: a Linear-layout bf16 matrix
``W[N, K] ~ N(0, 0.02)``, transposed to ``(K, N)`` and quantized with
``quantize_weight_int4`` at group size 128, exactly as ``quantize_llama`` does
(engine/quantize.py:185-189).  Activations are ``x[M, K] ~ N(0, 1)`` in bf16.
"""

from __future__ import annotations

import torch

from .quant import quantize_weight_int4

# (name, K = d_in, N = d_out) of one decoder block.
QWEN3_8B = (
    ("q_proj", 4096, 4096),
    ("k_proj", 4096, 1024),
    ("v_proj", 4096, 1024),
    ("o_proj", 4096, 4096),
    ("gate_proj", 4096, 12288),
    ("up_proj", 4096, 12288),
    ("down_proj", 12288, 4096),
)
QWEN3_32B = (
    ("q_proj", 5120, 8192),
    ("k_proj", 5120, 1024),
    ("v_proj", 5120, 1024),
    ("o_proj", 8192, 5120),
    ("gate_proj", 5120, 25600),
    ("up_proj", 5120, 25600),
    ("down_proj", 25600, 5120),
)
QWEN3_06B_GATE = ("gate_proj", 1024, 3072)
QWEN3_8B_LAYERS = 36
QWEN3_32B_LAYERS = 64


def make_weight(k: int, n: int, seed: int, device="cpu", group_size: int = 128):
    """(packed[K/2, N] int8, scale[K/128, N] fp32) from a seeded N(0, 0.02) bf16 weight."""
    gen = torch.Generator(device=device).manual_seed(seed)
    w_lin = (torch.randn(n, k, generator=gen, device=device) * 0.02).to(torch.bfloat16)
    return quantize_weight_int4(w_lin.T.contiguous().float(), group_size)


def make_activations(m: int, k: int, seed: int, device="cpu") -> torch.Tensor:
    gen = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(m, k, generator=gen, device=device).to(torch.bfloat16)


def algorithmic_bytes(m: int, k: int, n: int, group_size: int = 128) -> int:
    """Bytes one call must move at minimum: packed + scales + x + y."""
    return k * n // 2 + (k // group_size) * n * 4 + m * k * 2 + m * n * 2


def algorithmic_flops(m: int, k: int, n: int) -> int:
    return 2 * m * k * n
