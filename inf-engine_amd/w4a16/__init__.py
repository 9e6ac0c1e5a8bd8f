"""w4a16 -- MI355X-native INT4-weight / bf16-activation linear.

Drop-in for the INT4 surface of waleedalfar/inf-engine: ``int4_matmul`` and the
format helpers of engine/kernels/quant.py, ``_Int4Weight`` / ``quantize_llama``
of engine/quantize.py and ``linear`` of engine/layers.py, plus an on-disk INT4
format (``save_int4`` / ``load_int4`` / ``load_quantized_llama``) so a model is
quantized once rather than at every load.  The contraction runs
in hand-written gfx950 HIP kernels behind the C ABI of include/w4a16.h.
"""

from .checkpoint import load_int4, load_quantized_llama, save_int4
from . import moe
from .layers import linear, lm_head, qkv_projections, swiglu_mlp
from .quant import (
    dequantize_weight_int4,
    int4_matmul,
    int4_matmul_grouped,
    int4_swiglu,
    quantize_weight_int4,
)
from .quantize import QuantizedLlamaWeights, _Int4Weight, quantize_llama, quantized_to_device

__all__ = [
    "linear",
    "lm_head",
    "swiglu_mlp",
    "qkv_projections",
    "int4_swiglu",
    "int4_matmul",
    "int4_matmul_grouped",
    "quantize_weight_int4",
    "dequantize_weight_int4",
    "quantize_llama",
    "quantized_to_device",
    "QuantizedLlamaWeights",
    "_Int4Weight",
    "save_int4",
    "load_int4",
    "load_quantized_llama",
    "moe",
]
