"""Model-level INT4 wrapper -- the surface of engine/quantize.py.

``_Int4Weight`` carries one projection's packed weights and is what
``layers.linear`` dispatches on; ``quantize_llama`` swaps every projection of a
model for one; ``quantized_to_device`` moves a host-quantized model to a GPU.

The reference builds these around its own ``LlamaModel`` / ``LlamaWeights``
classes (engine/llama_model.py, engine/llama_weights.py), which are outside this
package.  ``quantize_llama`` therefore accepts any model object shaped like the
reference's: ``model.config`` with ``n_layer`` (and ``is_moe`` / ``n_experts``
for MoE), ``model.w`` with ``layer(i) -> dict`` and the flat tensor dict ``_t``,
plus ``embed_tokens`` / ``lm_head`` / ``norm_weight`` properties.
"""

from __future__ import annotations

import copy
from dataclasses import dataclass

import torch

from .quant import dequantize_weight_int4, int4_matmul, quantize_weight_int4

# Projection keys quantized per block (engine/quantize.py:37-45).
_LINEAR_SUFFIXES = (
    "self_attn.q_proj.weight",
    "self_attn.k_proj.weight",
    "self_attn.v_proj.weight",
    "self_attn.o_proj.weight",
    "mlp.gate_proj.weight",
    "mlp.up_proj.weight",
    "mlp.down_proj.weight",
)

# MoE expert projections, relative to an expert prefix (engine/quantize.py:48).
_EXPERT_PROJ_SUFFIXES = ("gate_proj.weight", "up_proj.weight", "down_proj.weight")


@dataclass
class _Int4Weight:
    """Packed INT4 projection (engine/quantize.py:51-73).

    packed: ``(d_in // 2, d_out)`` int8 -- column layout, K major.
    scale:  ``(d_in // group_size, d_out)`` float32.
    shape:  original ``(d_out, d_in)`` Linear layout.
    """

    packed: torch.Tensor
    scale: torch.Tensor
    group_size: int
    shape: tuple[int, int]

    def dequantize(self, dtype: torch.dtype) -> torch.Tensor:
        """Dense weight in ``(d_out, d_in)`` Linear layout and ``dtype``."""
        w_col = dequantize_weight_int4(self.packed, self.scale.to(dtype), self.group_size)
        return w_col.T.contiguous()

    def fused_linear(self, x: torch.Tensor) -> torch.Tensor:
        """``x @ W.T`` for ``x[..., d_in]`` -> ``[..., d_out]`` through the fused kernel."""
        lead = x.shape[:-1]
        out = int4_matmul(x.reshape(-1, x.shape[-1]), self.packed, self.scale, self.group_size)
        return out.reshape(*lead, self.shape[0])


def _quantize_projection(w: torch.Tensor, group_size: int) -> _Int4Weight:
    """Linear-layout ``(d_out, d_in)`` weight -> ``_Int4Weight`` (engine/quantize.py:185-189)."""
    w_col = w.T.contiguous()
    packed, scale = quantize_weight_int4(w_col.float(), group_size)
    return _Int4Weight(packed, scale, group_size, tuple(w.shape))


class QuantizedLlamaWeights:
    """Weights view whose projections are ``_Int4Weight`` (engine/quantize.py:76-152)."""

    def __init__(self, orig, int4: dict[str, _Int4Weight], dtype: torch.dtype) -> None:
        self._orig = orig
        self._int4 = int4
        self._dtype = dtype

    @property
    def embed_tokens(self) -> torch.Tensor:
        return self._orig.embed_tokens

    @property
    def lm_head(self) -> torch.Tensor:
        return self._orig.lm_head

    @property
    def norm_weight(self) -> torch.Tensor:
        return self._orig.norm_weight

    @property
    def config(self):
        return self._orig.config

    def _expert_suffixes(self):
        cfg = self._orig.config
        if not getattr(cfg, "is_moe", False):
            return ()
        names = [f"mlp.shared_expert.{p}" for p in _EXPERT_PROJ_SUFFIXES]
        for j in range(cfg.n_experts):
            names.extend(f"mlp.experts.{j}.{p}" for p in _EXPERT_PROJ_SUFFIXES)
        return names

    def layer(self, i: int) -> dict:
        """Block ``i``'s weight dict with quantized projections swapped in."""
        prefix = f"model.layers.{i}."
        out = self._orig.layer(i)
        for suffix in (*_LINEAR_SUFFIXES, *self._expert_suffixes()):
            w4 = self._int4.get(prefix + suffix)
            if w4 is not None:
                out[suffix] = w4
        return out

    def expert_weights(self, layer_idx: int, expert_id: int) -> dict:
        """Routed expert ``expert_id`` of ``layer_idx`` with INT4 projections."""
        prefix = f"model.layers.{layer_idx}.mlp.experts.{expert_id}."
        out = self._orig.expert_weights(layer_idx, expert_id)
        for proj in _EXPERT_PROJ_SUFFIXES:
            w4 = self._int4.get(prefix + proj)
            if w4 is not None:
                out[proj] = w4
        return out


def _block_suffixes(config) -> list[str]:
    """Projection names inside one decoder block (engine/quantize.py:37-48, 172-217)."""
    names = list(_LINEAR_SUFFIXES)
    if getattr(config, "is_moe", False):
        names += [f"mlp.shared_expert.{p}" for p in _EXPERT_PROJ_SUFFIXES]
        for j in range(config.n_experts):
            names += [f"mlp.experts.{j}.{p}" for p in _EXPERT_PROJ_SUFFIXES]
    return names


def projection_keys(config) -> list[str]:
    """Flat weight names of every projection ``quantize_llama`` may quantize."""
    return [f"model.layers.{i}.{s}" for i in range(config.n_layer) for s in _block_suffixes(config)]


def quantize_llama(model, group_size: int = 128):
    """Quantize every linear projection of ``model`` to INT4 W4A16 (engine/quantize.py:155-242).

    Returns a shallow copy of ``model`` whose ``w`` is a ``QuantizedLlamaWeights``;
    the dense projection tensors are dropped from the original weights' ``_t``
    dict, as the reference does to release their memory.  Embeddings, norms and
    ``lm_head`` stay dense.
    """
    config = model.config
    orig = model.w
    dtype = orig.embed_tokens.dtype
    int4: dict[str, _Int4Weight] = {}
    dense_bytes = 0
    packed_bytes = 0

    for i in range(config.n_layer):
        prefix = f"model.layers.{i}."
        block = orig.layer(i)
        for suffix in _block_suffixes(config):
            w = block.get(suffix)
            if w is None:
                continue
            w4 = _quantize_projection(w, group_size)
            int4[prefix + suffix] = w4
            dense_bytes += w.numel() * w.element_size()
            packed_bytes += w4.packed.numel() * w4.packed.element_size() + w4.scale.numel() * w4.scale.element_size()

    ratio = dense_bytes / max(packed_bytes, 1)
    print(f"w4a16: {len(int4)} projections of {config.n_layer} blocks now INT4, "
          f"weights {dense_bytes / 1e9:.2f} -> {packed_bytes / 1e9:.2f} GB (x{ratio:.1f} smaller)")
    for key in int4:
        orig._t.pop(key, None)
    if torch.cuda.is_available():
        torch.cuda.empty_cache()

    q_model = copy.copy(model)
    q_model.w = QuantizedLlamaWeights(orig, int4, dtype)
    return q_model


def quantized_to_device(model, device: str):
    """Move a ``quantize_llama`` model's tensors to ``device`` in place (engine/quantize.py:245-269)."""
    w = model.w
    if not isinstance(w, QuantizedLlamaWeights):
        raise TypeError("quantized_to_device requires a model from quantize_llama()")
    for key in list(w._orig._t.keys()):
        w._orig._t[key] = w._orig._t[key].to(device)
    for w4 in w._int4.values():
        w4.packed = w4.packed.to(device)
        w4.scale = w4.scale.to(device)
    for name in ("rope_cos", "rope_sin"):
        if hasattr(model, name):
            setattr(model, name, getattr(model, name).to(device))
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return model
