"""The safetensors loader (mlx/src/model/loader.rs:13-44) and the quantized
key scheme (mlx/src/nn/linear.rs:97-126) on a checkpoint written here with
the library's own packing restated by the oracle.  No GPU needed."""
import json

import numpy as np
import pytest
import safetensors.numpy as sn
import torch

import oracle
from ironmlx_amd import loader


def _write(tmp_path):
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    wq, s, b = oracle.affine_quantize(w, "f32", 64, 4, "f16")
    sn.save_file({"model.layers.0.mlp.gate_proj.weight": wq,
                  "model.layers.0.mlp.gate_proj.scales": s,
                  "model.layers.0.mlp.gate_proj.biases": b}, str(tmp_path / "model-00001-of-00002.safetensors"))
    sn.save_file({"model.norm.weight": np.ones(256, np.float16),
                  "lm_head.weight": wq[:8].copy()}, str(tmp_path / "model-00002-of-00002.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"model_type": "llama",
                                                      "quantization": {"group_size": 64, "bits": 4}}))
    return wq, s, b


def test_load_merges_files_in_order(tmp_path):
    wq, s, b = _write(tmp_path)
    weights = loader.load_model_weights(str(tmp_path), device=None)
    assert set(weights) == {"model.layers.0.mlp.gate_proj.weight", "model.layers.0.mlp.gate_proj.scales",
                            "model.layers.0.mlp.gate_proj.biases", "model.norm.weight", "lm_head.weight"}
    g = weights["model.layers.0.mlp.gate_proj.weight"]
    assert g.dtype == torch.uint32 and np.array_equal(g.view(torch.int32).numpy().view(np.uint32), wq)
    assert weights["model.layers.0.mlp.gate_proj.scales"].dtype == torch.float16
    q = loader.load_quantization(str(tmp_path))
    assert (q.group_size, q.bits, q.mode) == (64, 4, "affine")
    layers = loader.quantized_layers(weights, q)
    assert list(layers) == ["model.layers.0.mlp.gate_proj"]
    assert layers["model.layers.0.mlp.gate_proj"].biases is not None


def test_load_errors(tmp_path):
    with pytest.raises(RuntimeError, match="no .safetensors files found"):
        loader.load_model_weights(str(tmp_path), device=None)
    _write(tmp_path)
    weights = loader.load_model_weights(str(tmp_path), device=None)
    bad = loader.QuantizationConfig(32, 4, "affine")
    with pytest.raises(ValueError, match="do not match"):
        loader.quantized_layers(weights, bad)
