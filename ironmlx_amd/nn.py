"""Callers of the quantized ops, mirroring ironmlx's `nn` / model layer.

These are the reference's users of the drop-in boundary, restated over
:mod:`ironmlx_amd.ops` so the path can be exercised end to end:

* :class:`QuantizationConfig`  -- mlx/src/model/config.rs:32-51
* :class:`QuantizedLinear`, :class:`LinearLayer` -- mlx/src/nn/linear.rs:9-157
* :class:`QuantizedEmbedding`  -- mlx/src/nn/embedding.rs:39-96
* :class:`MLP` / :class:`Expert` (SwiGLU) -- mlx/src/nn/mlp.rs:11-33,
  mlx/src/nn/moe.rs:10-33
* :func:`split_fused_experts`  -- the fused gate_up_proj split of
  mlx/src/model/qwen35.rs:591-778, kept as stacked [E, N, K/pack] tensors
* :class:`MoEMLP`              -- mlx/src/nn/moe.rs:55-183, with the
  per-expert host loop replaced by two sorted :func:`ops.gather_qmm` passes

The quantized products run in libiqmm.so.  Routing (softmax / top-k), the
SwiGLU elementwise step, the dense router and the weighted combine use torch
device ops; they are outside the quantized path.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import torch
import torch.nn.functional as F

from . import ops


@dataclass
class QuantizationConfig:
    """`quantization` block of a model config.json (config.rs:32-51)."""
    group_size: int = 64
    bits: int = 4
    mode: str = "affine"

    @classmethod
    def from_dict(cls, d: Optional[dict]) -> Optional["QuantizationConfig"]:
        if d is None:
            return None
        return cls(int(d.get("group_size", 64)), int(d.get("bits", 4)), str(d.get("mode", "affine")))


def _get(weights: Dict[str, torch.Tensor], prefix: str, name: str) -> torch.Tensor:
    key = f"{prefix}.{name}" if prefix else name
    if key not in weights:
        raise KeyError(f"missing weight: {key}")
    return weights[key]


class QuantizedLinear:
    """Packed weight + per-group scales/biases; forward is
    ``quantized_matmul(x, w, s, b, transpose=True, gs, bits, mode)``
    (linear.rs:51-63).  ``mode`` defaults to "affine" like ``new`` (:22-31)."""

    def __init__(self, weight, scales, biases, group_size=64, bits=4, mode="affine"):
        self.weight, self.scales, self.biases = weight, scales, biases
        self.group_size, self.bits, self.mode = group_size, bits, mode

    def __call__(self, x: torch.Tensor, stream=None) -> torch.Tensor:
        return ops.quantized_matmul(x, self.weight, self.scales, self.biases, True,
                                    self.group_size, self.bits, self.mode, stream)

    forward = __call__

    def parameters(self):
        out = [("weight", self.weight), ("scales", self.scales)]
        if self.biases is not None:
            out.append(("biases", self.biases))
        return out

    def load_weights(self, weights, prefix):
        self.weight = _get(weights, prefix, "weight")
        self.scales = _get(weights, prefix, "scales")
        key = f"{prefix}.biases" if prefix else "biases"
        self.biases = weights.get(key)


class Linear:
    """Dense fallback of LinearLayer (linear.rs:131-157): x @ w^T + bias."""

    def __init__(self, weight, bias=None):
        self.weight, self.bias = weight, bias

    def __call__(self, x, stream=None):
        return F.linear(x, self.weight, self.bias)


class LinearLayer:
    """Dispatch to quantized or dense by the presence of ``{prefix}.scales``
    (linear.rs:97-126)."""

    @staticmethod
    def from_weights(weights, prefix, group_size=64, bits=4, mode="affine"):
        scales_key = f"{prefix}.scales" if prefix else "scales"
        if scales_key in weights:
            q = QuantizedLinear(None, None, None, group_size, bits, mode)
            q.load_weights(weights, prefix)
            return q
        bias_key = f"{prefix}.bias" if prefix else "bias"
        return Linear(_get(weights, prefix, "weight"), weights.get(bias_key))


class QuantizedEmbedding:
    """Dequantize the table, then gather rows (embedding.rs:62-73)."""

    def __init__(self, weight, scales, biases, group_size=64, bits=4, mode="affine"):
        self.weight, self.scales, self.biases = weight, scales, biases
        self.group_size, self.bits, self.mode = group_size, bits, mode

    def __call__(self, tokens: torch.Tensor, stream=None) -> torch.Tensor:
        table = ops.dequantize(self.weight, self.scales, self.biases, self.group_size, self.bits,
                               self.mode, stream)
        return table.index_select(0, tokens.reshape(-1).long()).reshape(*tokens.shape, -1)

    def as_linear(self, x: torch.Tensor, stream=None) -> torch.Tensor:
        """Tied lm_head: x @ dequant(table)^T (llama.rs:158-162)."""
        return ops.quantized_matmul(x, self.weight, self.scales, self.biases, True,
                                    self.group_size, self.bits, self.mode, stream)


class MLP:
    """down(silu(gate(x)) * up(x)) (mlp.rs:27-33)."""

    def __init__(self, gate_proj, up_proj, down_proj):
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def __call__(self, x, stream=None):
        g = self.gate_proj(x, stream)
        u = self.up_proj(x, stream)
        return self.down_proj(F.silu(g) * u, stream)


Expert = MLP  # moe.rs:10-33 has the same composition


@dataclass
class StackedExperts:
    """One projection of all experts: w [E, N, K*bits/32], s/b [E, N, K/gs]."""
    weight: torch.Tensor
    scales: torch.Tensor
    biases: Optional[torch.Tensor]
    group_size: int = 64
    bits: int = 4
    mode: str = "affine"


def split_fused_experts(weights: Dict[str, torch.Tensor], prefix: str, group_size=64, bits=4,
                        mode="affine") -> Dict[str, StackedExperts]:
    """Split ``{prefix}.mlp.experts.gate_up_proj.{weight,scales,biases}``
    [E, 2I, .] into gate (rows [0, I)) and up (rows [I, 2I)), and take
    ``down_proj`` [E, H, .] as is (qwen35.rs:655-775).  The halves are kept
    stacked over experts (one contiguous copy each) for gather_qmm instead of
    being sliced into E separate layers."""
    base = f"{prefix}.mlp.experts"
    gu_w = weights[f"{base}.gate_up_proj.weight"]
    gu_s = weights[f"{base}.gate_up_proj.scales"]
    gu_b = weights.get(f"{base}.gate_up_proj.biases")
    half_w, half_s = gu_w.shape[1] // 2, gu_s.shape[1] // 2

    def half(t, h, lo):
        return None if t is None else t[:, lo * h:(lo + 1) * h].contiguous()

    out = {
        "gate": StackedExperts(half(gu_w, half_w, 0), half(gu_s, half_s, 0),
                               half(gu_b, half_s, 0), group_size, bits, mode),
        "up": StackedExperts(half(gu_w, half_w, 1), half(gu_s, half_s, 1),
                             half(gu_b, half_s, 1), group_size, bits, mode),
        "down": StackedExperts(weights[f"{base}.down_proj.weight"],
                               weights[f"{base}.down_proj.scales"],
                               weights.get(f"{base}.down_proj.biases"), group_size, bits, mode),
    }
    return out


def _gqmm(x, e: StackedExperts, rhs, sorted_indices=True, stream=None):
    return ops.gather_qmm(x, e.weight, e.scales, e.biases, None, rhs, True, e.group_size, e.bits,
                          e.mode, sorted_indices, stream)


class MoEMLP:
    """Router softmax -> top-k (normalised when ``norm_topk_prob``) -> experts
    -> weighted sum, plus a sigmoid-gated shared expert (moe.rs:55-183).

    The reference evaluates routing on the host and runs one quantized_matmul
    per used expert per projection (moe.rs:86-143); here the (token, slot)
    rows are sorted by expert on the device and each projection is a single
    sorted gather_qmm over the stacked expert tensors."""

    def __init__(self, gate: Linear, experts: Dict[str, StackedExperts], shared_expert: MLP,
                 shared_expert_gate: Linear, num_experts_per_tok: int, norm_topk_prob: bool = True):
        self.gate, self.experts = gate, experts
        self.shared_expert, self.shared_expert_gate = shared_expert, shared_expert_gate
        self.k, self.norm_topk_prob = num_experts_per_tok, norm_topk_prob

    def route(self, x_flat):
        logits = self.gate(x_flat)
        probs = torch.softmax(logits.float(), dim=-1)
        scores, idx = torch.topk(probs, self.k, dim=-1)
        if self.norm_topk_prob:
            scores = scores / scores.sum(-1, keepdim=True)
        return scores, idx

    def experts_forward(self, x_flat, scores, idx, stream=None):
        n, d = x_flat.shape
        flat = idx.reshape(-1)
        order = torch.argsort(flat, stable=True)
        rhs = flat[order].to(torch.int32).contiguous()
        xs = x_flat[order // self.k].reshape(n * self.k, 1, d).contiguous()
        g = _gqmm(xs, self.experts["gate"], rhs, stream=stream)
        u = _gqmm(xs, self.experts["up"], rhs, stream=stream)
        h = (F.silu(g) * u).contiguous()
        y = _gqmm(h, self.experts["down"], rhs, stream=stream).reshape(n * self.k, -1)
        w = scores.reshape(-1)[order].to(y.dtype).unsqueeze(-1)
        out = torch.zeros((n, y.shape[-1]), dtype=torch.float32, device=y.device)
        out.index_add_(0, order // self.k, (y * w).float())
        return out.to(x_flat.dtype)

    def __call__(self, x, stream=None):
        b, l, d = x.shape
        x_flat = x.reshape(b * l, d)
        scores, idx = self.route(x_flat)
        out = self.experts_forward(x_flat, scores, idx, stream)
        shared = self.shared_expert(x_flat, stream)
        gate = torch.sigmoid(self.shared_expert_gate(x_flat))
        return (out + shared * gate).reshape(b, l, d)
