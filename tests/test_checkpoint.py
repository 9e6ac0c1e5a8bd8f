"""INT4 on-disk format (w4a16.checkpoint): round trips and validation, on the CPU."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from test_host import _mini_model


def test_save_load_round_trip_is_bit_exact(tmp_path):
    from w4a16 import _Int4Weight, load_int4, quantize_llama, save_int4

    model, _ = _mini_model()
    q = quantize_llama(model)
    path = str(tmp_path / "m.int4.safetensors")
    assert save_int4(q, path) == 14
    loaded = load_int4(path)
    assert set(loaded) == set(q.w._int4)
    for key, w4 in q.w._int4.items():
        got = loaded[key]
        assert isinstance(got, _Int4Weight)
        assert got.shape == w4.shape and got.group_size == w4.group_size
        assert got.packed.dtype == torch.int8 and got.scale.dtype == torch.float32
        assert torch.equal(got.packed, w4.packed) and torch.equal(got.scale, w4.scale)


def test_load_quantized_llama_matches_quantize_llama(tmp_path):
    from w4a16 import load_quantized_llama, quantize_llama, save_int4

    model, _ = _mini_model()
    q = quantize_llama(model)
    path = str(tmp_path / "m.safetensors")
    save_int4(q.w, path)
    fresh, dense = _mini_model()
    q2 = load_quantized_llama(fresh, path)
    for i in range(2):
        a, b = q.w.layer(i), q2.w.layer(i)
        assert set(a) == set(b)
        for k in a:
            if hasattr(a[k], "packed"):
                assert torch.equal(a[k].packed, b[k].packed) and torch.equal(a[k].scale, b[k].scale)
                assert f"model.layers.{i}.{k}" not in fresh.w._t  # dense projection released
            else:
                assert torch.equal(a[k], b[k])


def test_load_rejects_foreign_and_inconsistent_files(tmp_path):
    from safetensors.torch import save_file

    from w4a16 import load_int4, save_int4
    from w4a16.quantize import _Int4Weight

    plain = str(tmp_path / "plain.safetensors")
    save_file({"w": torch.zeros(2, 2)}, plain)
    with pytest.raises(ValueError, match="not a w4a16-int4"):
        load_int4(plain)

    good = {"k": _Int4Weight(torch.zeros(128, 8, dtype=torch.int8), torch.ones(2, 8), 128, (8, 256))}
    path = str(tmp_path / "g.safetensors")
    save_int4(good, path)
    meta = {"format": "w4a16-int4", "version": "1", "projections": json.dumps({"k": [8, 512, 128]})}
    bad = str(tmp_path / "bad.safetensors")
    save_file({"k.packed": torch.zeros(128, 8, dtype=torch.int8), "k.scale": torch.ones(2, 8)}, bad, metadata=meta)
    with pytest.raises(ValueError, match="packed shape"):
        load_int4(bad)
    meta2 = dict(meta, version="9")
    save_file({"k.packed": torch.zeros(128, 8, dtype=torch.int8), "k.scale": torch.ones(2, 8)}, bad, metadata=meta2)
    with pytest.raises(ValueError, match="version"):
        load_int4(bad)
    meta3 = dict(meta, projections=json.dumps({"k": [8, 256, 128]}))
    save_file({"k.packed": torch.zeros(128, 8, dtype=torch.int8), "k.scale": torch.ones(2, 8, dtype=torch.float64)},
              bad, metadata=meta3)
    with pytest.raises(ValueError, match="float32"):
        load_int4(bad)
    with pytest.raises(ValueError, match="shape"):
        save_int4({"k": _Int4Weight(torch.zeros(64, 8, dtype=torch.int8), torch.ones(2, 8), 128, (8, 256))},
                  str(tmp_path / "x.safetensors"))


def test_load_quantized_llama_rejects_mismatched_checkpoint(tmp_path):
    from w4a16 import load_quantized_llama, quantize_llama, save_int4

    model, _ = _mini_model(layers=1)
    path = str(tmp_path / "one.safetensors")
    save_int4(quantize_llama(model), path)
    two, _ = _mini_model(layers=2)
    with pytest.raises(ValueError, match="missing"):
        load_quantized_llama(two, path)
