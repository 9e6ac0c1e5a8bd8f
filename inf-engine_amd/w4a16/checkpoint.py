"""On-disk INT4 format: packed weights and scales in one safetensors file.

The reference re-quantizes every projection from the dense checkpoint at each
load (engine/quantize.py:155-242, called from main.py:464-478).  This module
stores the result of ``quantize_llama`` once, so later loads read the packed
bytes directly.  Nothing is re-laid-out: the file holds the same tensors the
fused kernel consumes.

File layout (safetensors, so loading executes nothing from the file):

* ``<key>.packed``  int8    ``[d_in / 2, d_out]``  (high nibble = even K row)
* ``<key>.scale``   float32 ``[d_in / group_size, d_out]``

where ``<key>`` is the reference's flat weight name, e.g.
``model.layers.3.mlp.gate_proj.weight``.  The safetensors metadata holds:

* ``format``: ``w4a16-int4``
* ``version``: ``1``
* ``projections``: JSON object ``key -> [d_out, d_in, group_size]``
"""

from __future__ import annotations

import json
import os

import torch

FORMAT = "w4a16-int4"
VERSION = "1"


def _weights_of(obj):
    """The ``key -> _Int4Weight`` dict of a quantized model, its weights, or the dict itself."""
    from .quantize import QuantizedLlamaWeights

    if isinstance(obj, dict):
        return obj
    w = getattr(obj, "w", obj)
    if isinstance(w, QuantizedLlamaWeights):
        return w._int4
    raise TypeError("expected a quantize_llama() model, its QuantizedLlamaWeights, or a dict of _Int4Weight")


def save_int4(obj, path: str) -> int:
    """Write every INT4 projection of ``obj`` to ``path``; returns the number saved.

    ``obj`` is a model returned by ``quantize_llama``, its ``QuantizedLlamaWeights``
    or a ``{key: _Int4Weight}`` dict.  Tensors are copied to host memory.
    """
    from safetensors.torch import save_file

    from .quantize import _Int4Weight

    weights = _weights_of(obj)
    tensors: dict[str, torch.Tensor] = {}
    meta: dict[str, list[int]] = {}
    for key, w4 in weights.items():
        if not isinstance(w4, _Int4Weight):
            raise TypeError(f"{key}: not an _Int4Weight")
        d_out, d_in = w4.shape
        _check_shapes(key, w4.packed, w4.scale, d_out, d_in, w4.group_size)
        tensors[f"{key}.packed"] = w4.packed.detach().to("cpu", torch.int8).contiguous()
        tensors[f"{key}.scale"] = w4.scale.detach().to("cpu", torch.float32).contiguous()
        meta[key] = [int(d_out), int(d_in), int(w4.group_size)]
    tmp = path + ".tmp"
    save_file(tensors, tmp, metadata={"format": FORMAT, "version": VERSION, "projections": json.dumps(meta)})
    os.replace(tmp, path)
    return len(meta)


def _check_shapes(key, packed, scale, d_out, d_in, group_size) -> None:
    if group_size <= 0 or d_in % group_size != 0 or d_in % 2 != 0:
        raise ValueError(f"{key}: d_in={d_in} incompatible with group_size={group_size}")
    if tuple(packed.shape) != (d_in // 2, d_out):
        raise ValueError(f"{key}: packed shape {tuple(packed.shape)} != {(d_in // 2, d_out)}")
    if tuple(scale.shape) != (d_in // group_size, d_out):
        raise ValueError(f"{key}: scale shape {tuple(scale.shape)} != {(d_in // group_size, d_out)}")


def load_int4(path: str, device="cpu") -> dict:
    """Read a file written by ``save_int4``; returns ``{key: _Int4Weight}`` on ``device``.

    Raises:
        ValueError: not a w4a16-int4 file, an unknown version, or tensors whose
            shapes or dtypes disagree with the recorded projection shapes.
    """
    from safetensors import safe_open

    from .quantize import _Int4Weight

    out = {}
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: not a {FORMAT} file (format={meta.get('format')!r})")
        if meta.get("version") != VERSION:
            raise ValueError(f"{path}: unsupported {FORMAT} version {meta.get('version')!r}")
        projections = json.loads(meta["projections"])
        names = set(f.keys())
        for key, (d_out, d_in, group_size) in projections.items():
            for suffix in (".packed", ".scale"):
                if key + suffix not in names:
                    raise ValueError(f"{path}: missing tensor {key + suffix}")
            packed = f.get_tensor(key + ".packed")
            scale = f.get_tensor(key + ".scale")
            if packed.dtype != torch.int8 or scale.dtype != torch.float32:
                raise ValueError(f"{key}: expected int8 packed and float32 scale, got {packed.dtype}, {scale.dtype}")
            _check_shapes(key, packed, scale, d_out, d_in, group_size)
            out[key] = _Int4Weight(packed.to(device), scale.to(device), int(group_size), (int(d_out), int(d_in)))
    return out


def load_quantized_llama(model, path: str, device=None):
    """``quantize_llama(model)`` without re-quantizing: projections come from ``path``.

    ``model`` is shaped like the reference's ``LlamaModel`` (see ``quantize_llama``);
    its dense projection tensors, if loaded, are dropped.  ``device`` defaults to
    the device of ``model.w.embed_tokens``.  Every projection that
    ``quantize_llama`` would create must be in the file, and nothing else.
    """
    import copy

    from .quantize import QuantizedLlamaWeights, projection_keys

    orig = model.w
    dev = device if device is not None else orig.embed_tokens.device
    int4 = load_int4(path, dev)
    expected = set(projection_keys(model.config))
    # A checkpoint may lack projections the dense model also lacks (e.g. no shared expert).
    missing = sorted(k for k in expected - set(int4) if k in orig._t)
    extra = sorted(set(int4) - expected)
    if missing or extra:
        raise ValueError(f"{path}: projections do not match the model (missing {missing[:3]}, extra {extra[:3]})")
    for key in int4:
        orig._t.pop(key, None)
    q_model = copy.copy(model)
    q_model.w = QuantizedLlamaWeights(orig, int4, orig.embed_tokens.dtype)
    return q_model
