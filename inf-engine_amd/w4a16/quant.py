"""INT4 W4A16 weight format and fused matmul -- the surface of engine/kernels/quant.py.

Same names, arguments, layouts and error types as the reference module's INT4
half (engine/kernels/quant.py:77-281):

* ``quantize_weight_int4(w, group_size)``  -> ``(packed[K/2, N] int8, scale[K/g, N])``
* ``dequantize_weight_int4(packed, scale, group_size)`` -> ``w[K, N]`` in ``scale.dtype``
* ``int4_matmul(a, packed, scale, group_size=128)`` -> ``a @ w`` in bf16

``int4_matmul`` and device-tensor ``dequantize_weight_int4`` run the gfx950 HIP
kernels of ``libw4a16.so`` through the C ABI; there is no Triton and no other
device backend.  Host tensors keep the reference's host semantics
(engine/kernels/quant.py:264-266): dequantize with the scales cast to the
activation dtype, then ``a @ w`` in torch on the CPU.  A device tensor never
takes that branch: if the library is missing, a device call raises.
"""

from __future__ import annotations

import torch

from . import _native

_INT4_MAX = 7        # symmetric code range [-7, 7] produced by the quantizer
_NIBBLES_PER_BYTE = 2
FUSED_GROUP_SIZE = 128


def quantize_weight_int4(w: torch.Tensor, group_size: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-group INT4 quantization of a ``(d_in, d_out)`` weight.

    Follows engine/kernels/quant.py:81-119 operation for operation, so the
    packed bytes and scales are bit-identical to the reference's on the same
    input: per (group, column) ``scale = max(amax|w| / 7, 1e-8)``, codes
    ``clamp(round_half_even(w / scale), -7, 7)``, and rows ``2i`` / ``2i+1``
    packed into the high / low nibble of byte ``i``.

    This is one-time weight preparation in torch on whatever device ``w`` lives
    (the reference does the same, engine/quantize.py:187-188); it is not the
    measured path.

    Raises:
        ValueError: ``d_in`` not divisible by ``group_size`` or odd.
    """
    d_in, d_out = w.shape
    if d_in % group_size != 0:
        raise ValueError(f"d_in={d_in} not divisible by group_size={group_size}")
    if d_in % _NIBBLES_PER_BYTE != 0:
        raise ValueError(f"d_in={d_in} must be even for nibble packing")
    groups = d_in // group_size
    grouped = w.reshape(groups, group_size, d_out)
    scale = (grouped.abs().amax(dim=1) / _INT4_MAX).clamp(min=1e-8)          # (G, d_out)
    codes = (grouped / scale[:, None, :].expand_as(grouped)).round()
    codes = codes.clamp(-_INT4_MAX, _INT4_MAX).to(torch.int8).reshape(d_in, d_out)
    hi = (codes[0::2] & 0x0F).to(torch.uint8)
    lo = (codes[1::2] & 0x0F).to(torch.uint8)
    packed = ((hi << 4) | lo).to(torch.int8)
    return packed, scale


def _dequantize_host(packed: torch.Tensor, scale: torch.Tensor, group_size: int) -> torch.Tensor:
    d_half, d_out = packed.shape
    d_in = d_half * _NIBBLES_PER_BYTE
    even = packed >> 4                                       # int8 arithmetic shift: sign-extends
    odd = ((packed & 0x0F).to(torch.int8) << 4) >> 4
    codes = torch.stack((even, odd), dim=1).reshape(d_in, d_out)
    groups = d_in // group_size
    w = codes.reshape(groups, group_size, d_out).to(scale.dtype) * scale[:, None, :]
    return w.reshape(d_in, d_out)


def dequantize_weight_int4(packed: torch.Tensor, scale: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """Unpack INT4 weights to ``(d_in, d_out)`` in ``scale.dtype``.

    Semantics of engine/kernels/quant.py:122-156: even rows come from the high
    nibble (int8 arithmetic shift), odd rows from the sign-extended low nibble,
    and row ``k`` is multiplied by ``scale[k // group_size]``.

    Device tensors run the HIP ``w4a16_dequant`` kernel (float32 or bfloat16
    scales).  Host tensors are unpacked with torch on the host, as the
    reference does for host tensors; this is a format utility, not the fused
    contraction.
    """
    d_half, d_out = packed.shape
    d_in = d_half * _NIBBLES_PER_BYTE
    if group_size <= 0 or d_in % group_size != 0:
        raise ValueError(f"d_in={d_in} not divisible by group_size={group_size}")
    if scale.shape != (d_in // group_size, d_out):
        raise ValueError(f"scale shape {tuple(scale.shape)} != {(d_in // group_size, d_out)}")
    if not packed.is_cuda:
        return _dequantize_host(packed, scale, group_size)
    if scale.device != packed.device:
        raise ValueError("packed and scale must be on the same device")
    if scale.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"device dequantize supports float32/bfloat16 scales, got {scale.dtype}")
    with torch.cuda.device(packed.device):
        return _native.dequant(packed, scale.float(), group_size, scale.dtype)


def _host_matmul(a: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, group_size: int) -> torch.Tensor:
    """Host branch of int4_matmul (engine/kernels/quant.py:264-266): dense
    weights in ``a.dtype`` (the scales are cast to it first), then ``a @ w``."""
    if packed.is_cuda or scale.is_cuda:
        raise ValueError("a, packed and scale must be on the same device")
    w = dequantize_weight_int4(packed, scale.to(a.dtype), group_size)
    return a @ w


def _check_operands(a: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, group_size: int) -> torch.Tensor:
    """Shape / dtype / device checks shared by the device entry points; returns fp32 scale."""
    if not a.is_cuda:
        raise TypeError("the grouped and SwiGLU W4A16 entry points run on HIP device tensors only")
    assert group_size == FUSED_GROUP_SIZE, f"fused INT4 kernel requires group_size=128, got {group_size}"
    if a.dim() != 2 or packed.dim() != 2 or scale.dim() != 2:
        raise ValueError("int4_matmul expects a[M,K], packed[K/2,N], scale[K/128,N]")
    m, k = a.shape
    k_half, n = packed.shape
    if k != 2 * k_half:
        raise ValueError(f"a has K={k} but packed has {k_half} rows (expected K/2)")
    if k % group_size != 0:
        raise ValueError(f"K={k} not divisible by group_size={group_size}")
    if scale.shape != (k // group_size, n):
        raise ValueError(f"scale shape {tuple(scale.shape)} != {(k // group_size, n)}")
    if a.dtype != torch.bfloat16:
        raise TypeError(f"int4_matmul activations must be bfloat16, got {a.dtype}")
    if packed.dtype not in (torch.int8, torch.uint8):
        raise TypeError(f"packed weights must be int8, got {packed.dtype}")
    if packed.device != a.device or scale.device != a.device:
        raise ValueError("a, packed and scale must be on the same device")
    return scale if scale.dtype == torch.float32 else scale.float()


def int4_matmul_grouped(a, weights, group_size: int = 128) -> list[torch.Tensor]:
    """Several INT4 projections at once: ``[a_i @ dequantize(packed_i, scale_i)]``.

    ``a`` is one ``(M, K)`` bf16 tensor shared by every projection (q/k/v or
    gate/up of a block) or a list of per-projection activations, each with its
    own M (a set of MoE experts with their token counts).  ``weights`` is a list
    of ``(packed, scale)`` pairs, at most 16.  Decode-sized projections (M <= 32,
    or M <= 64 on small shapes) share one decode launch and the rest one GEMM launch.  Results equal
    ``int4_matmul`` on each pair up to fp32 summation order.  No reference
    counterpart: the reference calls ``int4_matmul`` once per projection
    (engine/llama_attention.py:83-85, engine/llama_mlp.py:30-33,
    engine/llama_moe.py:90-105).
    """
    xs = list(a) if isinstance(a, (list, tuple)) else [a] * len(weights)
    if len(xs) != len(weights):
        raise ValueError("need one activation tensor per weight (or a single shared one)")
    prepared = [(packed, _check_operands(x, packed, scale, group_size)) for x, (packed, scale) in zip(xs, weights)]
    with torch.cuda.device(xs[0].device):
        return _native.linear_grouped(xs, prepared, group_size)


def int4_matmul(a: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """Fused W4A16 matmul ``a @ dequantize(packed, scale)`` without a dense weight.

    Drop-in for engine/kernels/quant.py:243-281.  On a HIP device ``a`` is
    ``(M, K)`` bf16, ``packed`` ``(K/2, N)`` int8, ``scale`` ``(K/128, N)``
    float32; the result is ``(M, N)`` bf16, allocated on the caller's stream.
    The call enqueues on the current stream and never synchronises, so it can
    be captured in a HIP graph (the split-K workspace is allocated inside the
    capture if the capturing stream has none yet).  M <= 32 (M <= 64 on small
    shapes) runs the HBM-bound decode kernel, larger M the MFMA GEMM.

    Host tensors take the reference's host branch (quant.py:264-266): any
    float ``a``, result in ``a.dtype``, any group size.

    Raises:
        AssertionError: ``group_size != 128`` on a device (as engine/kernels/quant.py:267).
        ValueError: inconsistent shapes.
        TypeError: non-bf16 device activations.
    """
    if not a.is_cuda:
        return _host_matmul(a, packed, scale, group_size)
    scale = _check_operands(a, packed, scale, group_size)
    with torch.cuda.device(a.device):
        return _native.linear(a, packed, scale, group_size)


def int4_swiglu(a: torch.Tensor, gate, up, group_size: int = 128) -> torch.Tensor:
    """SwiGLU gate/up pair ``silu(a @ Wg) * (a @ Wu)`` in one call.

    ``gate`` and ``up`` are ``(packed, scale)`` pairs of the same shape.  The
    reference computes ``silu(linear(x, gate)) * linear(x, up)``
    (engine/llama_mlp.py:30-32, engine/llama_moe.py:44) as two int4_matmul
    launches and two elementwise kernels.  Here decode-sized M is one decode
    launch with the epilogue on the fp32 sums; GEMM-sized M is the row sums
    plus one pair GEMM launch that stores ``silu(g) * u`` from the fp32 tiles
    (operands it cannot take go through a grouped GEMM plus one elementwise
    pass).  Device tensors only; same checks and exceptions as ``int4_matmul``.
    """
    (gp, gs), (up_p, us) = gate, up
    if gp.shape != up_p.shape or gs.shape != us.shape:
        raise ValueError(f"gate {tuple(gp.shape)} and up {tuple(up_p.shape)} weights differ in shape")
    gs = _check_operands(a, gp, gs, group_size)
    us = _check_operands(a, up_p, us, group_size)
    with torch.cuda.device(a.device):
        return _native.swiglu(a, (gp, gs), (up_p, us), group_size)
