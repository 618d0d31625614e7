"""On-disk weights of mlx-community checkpoints, as ironmlx loads them.

* :func:`load_model_weights` -- ``load_model_weights`` of
  mlx/src/model/loader.rs:13-44: every ``*.safetensors`` file of a model
  directory, in file-name order, merged into one name -> tensor map.
* :func:`load_quantization` -- the ``quantization`` block of ``config.json``
  (mlx/src/model/config.rs:25, :32-51) as a :class:`nn.QuantizationConfig`.
* :func:`quantized_layers` -- the quantized linear layers of a weight map: the
  key scheme ``{prefix}.weight`` (uint32 packed codes) + ``{prefix}.scales`` +
  optional ``{prefix}.biases`` that ``LinearLayer`` dispatches on
  (mlx/src/nn/linear.rs:97-126), checked against the packed shapes the kernels
  take.

The tensors are read with the safetensors library (no code in the file is
executed) and moved to the device once; the packed words stay uint32 and the
scales / biases keep their stored dtype, so they feed the library unchanged.
"""
from __future__ import annotations

import json
import os
from typing import Dict, Optional

import torch
from safetensors.torch import load_file

from .nn import QuantizationConfig, QuantizedLinear


def load_model_weights(model_dir: str, device: Optional[str] = "cuda") -> Dict[str, torch.Tensor]:
    """All ``*.safetensors`` files of ``model_dir`` in sorted file-name order;
    a later file's tensor replaces an earlier one of the same name."""
    try:
        names = sorted(n for n in os.listdir(model_dir) if n.endswith(".safetensors"))
    except OSError as e:
        raise RuntimeError(f"failed to read dir: {e}") from e
    if not names:
        raise RuntimeError("no .safetensors files found")
    weights: Dict[str, torch.Tensor] = {}
    for n in names:
        for k, v in load_file(os.path.join(model_dir, n), device="cpu").items():
            weights[k] = v.to(device) if device is not None else v
    return weights


def load_quantization(model_dir: str) -> Optional[QuantizationConfig]:
    """The ``quantization`` block of ``config.json`` (absent: None)."""
    with open(os.path.join(model_dir, "config.json")) as f:
        cfg = json.load(f)
    return QuantizationConfig.from_dict(cfg.get("quantization"))


def quantized_layers(weights: Dict[str, torch.Tensor],
                     q: QuantizationConfig) -> Dict[str, QuantizedLinear]:
    """Every ``{prefix}`` with ``{prefix}.scales`` and a uint32 ``{prefix}.weight``
    as a QuantizedLinear; raises on shapes that do not match the packing."""
    out: Dict[str, QuantizedLinear] = {}
    for key, s in weights.items():
        if not key.endswith(".scales"):
            continue
        prefix = key[: -len(".scales")]
        w = weights.get(f"{prefix}.weight")
        if w is None or w.dtype != torch.uint32:
            continue
        b = weights.get(f"{prefix}.biases")
        K = w.shape[-1] * 32 // q.bits
        if w.shape[:-1] != s.shape[:-1] or s.shape[-1] * q.group_size != K:
            raise ValueError(f"{prefix}: weight {tuple(w.shape)} and scales {tuple(s.shape)} do not match "
                             f"group_size={q.group_size}, bits={q.bits}")
        if q.mode == "affine" and (b is None or b.shape != s.shape):
            raise ValueError(f"{prefix}: affine quantization needs biases shaped like the scales")
        out[prefix] = QuantizedLinear(w, s, b, q.group_size, q.bits, q.mode)
    return out
