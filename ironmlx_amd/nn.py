"""Callers of the quantized ops, mirroring ironmlx's `nn` / model layer.

These are the reference's users of the drop-in boundary, restated over
:mod:`ironmlx_amd.ops` so the path can be exercised end to end:

* :class:`QuantizationConfig`  -- mlx/src/model/config.rs:32-51
* :class:`QuantizedLinear`, :class:`LinearLayer` -- mlx/src/nn/linear.rs:9-157
* :class:`QuantizedEmbedding`  -- mlx/src/nn/embedding.rs:39-96
* :class:`MLP` / :class:`Expert` (SwiGLU) -- mlx/src/nn/mlp.rs:11-33,
  mlx/src/nn/moe.rs:10-33; :class:`FusedMLP` runs gate and up as one fused
  SwiGLU call over a stacked gate_up weight
* :func:`split_fused_experts`  -- the fused gate_up_proj split of
  mlx/src/model/qwen35.rs:591-778, kept as stacked [E, N, K/pack] tensors
* :func:`stack_fused_experts` -- the same tensors kept unsplit for the fused
  gate_up SwiGLU gather
* :class:`MoEMLP`              -- mlx/src/nn/moe.rs:55-183, with the
  per-expert host loop replaced by sorted :func:`ops.gather_qmm` passes and
  the routing (softmax / top-k / normalise, the sort by expert, the weighted
  combine) run on the device by the library

The quantized products and the routing run in libiqmm.so.  The dense router
and shared-expert gate (plain Linear) and the unfused SwiGLU step of
:class:`MLP` use torch device ops; they are outside the quantized path.
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
        """Rows of dequantize(table) for the token ids, gathered without
        dequantizing the whole table (bit-identical to embedding.rs:62-72)."""
        idx = tokens if tokens.dtype in (torch.int32, torch.int64) else tokens.long()
        return ops.dequantize_rows(self.weight, self.scales, self.biases, idx.contiguous(),
                                   self.group_size, self.bits, self.mode, stream)

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


class FusedMLP:
    """down(silu(gate(x)) * up(x)) with gate and up stacked into one
    [2I, K/pack] weight (gate rows first) and evaluated by one fused SwiGLU
    call: x is read once and the elementwise step runs in the product's
    epilogue (one launch at decode).  Same rounding as :class:`MLP`."""

    def __init__(self, gate_up: QuantizedLinear, down_proj):
        self.gate_up, self.down_proj = gate_up, down_proj

    @classmethod
    def from_mlp(cls, mlp: MLP) -> "FusedMLP":
        g, u = mlp.gate_proj, mlp.up_proj
        if not (isinstance(g, QuantizedLinear) and isinstance(u, QuantizedLinear)):
            raise TypeError("FusedMLP needs quantized gate and up projections")
        if (g.group_size, g.bits, g.mode) != (u.group_size, u.bits, u.mode):
            raise ValueError("gate and up must share group_size, bits and mode")
        cat = lambda a, b: None if a is None else torch.cat([a, b], dim=0).contiguous()
        gu = QuantizedLinear(cat(g.weight, u.weight), cat(g.scales, u.scales),
                             cat(g.biases, u.biases), g.group_size, g.bits, g.mode)
        return cls(gu, mlp.down_proj)

    def __call__(self, x, stream=None):
        gu = self.gate_up
        h = ops.quantized_swiglu(x, gu.weight, gu.scales, gu.biases, gu.group_size, gu.bits,
                                 gu.mode, stream)
        return self.down_proj(h, stream)


class FusedQKV:
    """q, k and v projections of one attention layer stacked row-wise into a
    single QuantizedLinear ([Nq + Nk + Nv, K/pack]) so decode reads x once and
    runs one GEMV instead of three; returns the (q, k, v) column blocks.
    Each block equals its own projection's output (the rows are independent)."""

    def __init__(self, q: QuantizedLinear, k: QuantizedLinear, v: QuantizedLinear):
        params = {(p.group_size, p.bits, p.mode) for p in (q, k, v)}
        if len(params) != 1:
            raise ValueError("q, k and v must share group_size, bits and mode")
        cat = lambda *t: None if t[0] is None else torch.cat(t, dim=0).contiguous()
        self.linear = QuantizedLinear(cat(q.weight, k.weight, v.weight), cat(q.scales, k.scales, v.scales),
                                      cat(q.biases, k.biases, v.biases), q.group_size, q.bits, q.mode)
        self.sizes = [q.weight.shape[0], k.weight.shape[0], v.weight.shape[0]]

    def __call__(self, x, stream=None):
        return torch.split(self.linear(x, stream), self.sizes, dim=-1)


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


def stack_fused_experts(weights: Dict[str, torch.Tensor], prefix: str, group_size=64, bits=4,
                        mode="affine") -> Dict[str, StackedExperts]:
    """The expert tensors of qwen35.rs:655-775 kept as loaded: the fused
    gate_up_proj [E, 2I, .] (gate rows first) for :func:`ops.gather_qmm_swiglu`
    and down_proj [E, H, .]; no copies."""
    base = f"{prefix}.mlp.experts"
    return {
        "gate_up": StackedExperts(weights[f"{base}.gate_up_proj.weight"],
                                  weights[f"{base}.gate_up_proj.scales"],
                                  weights.get(f"{base}.gate_up_proj.biases"), group_size, bits, mode),
        "down": StackedExperts(weights[f"{base}.down_proj.weight"],
                               weights[f"{base}.down_proj.scales"],
                               weights.get(f"{base}.down_proj.biases"), group_size, bits, mode),
    }


def _gqmm(x, e: StackedExperts, rhs, lhs=None, sorted_indices=True, stream=None):
    return ops.gather_qmm(x, e.weight, e.scales, e.biases, lhs, rhs, True, e.group_size, e.bits,
                          e.mode, sorted_indices, stream)


class MoEMLP:
    """Router softmax -> top-k (normalised when ``norm_topk_prob``) -> experts
    -> weighted sum, plus a sigmoid-gated shared expert (moe.rs:55-183).

    The reference evaluates routing on the host and runs one quantized_matmul
    per used expert per projection (moe.rs:86-143); here routing, the sort of
    the (token, slot) rows by expert and the weighted combine run on the
    device (no host synchronisation), and each projection is a single sorted
    gather_qmm over the stacked expert tensors -- with ``experts["gate_up"]``
    (:func:`stack_fused_experts`) gate, up and the SwiGLU are one fused call.
    Like the reference (moe.rs:146-172), the result is float32."""

    def __init__(self, gate: Linear, experts: Dict[str, StackedExperts], shared_expert: MLP,
                 shared_expert_gate: Linear, num_experts_per_tok: int, norm_topk_prob: bool = True):
        self.gate, self.experts = gate, experts
        self.shared_expert, self.shared_expert_gate = shared_expert, shared_expert_gate
        self.k, self.norm_topk_prob = num_experts_per_tok, norm_topk_prob

    def num_experts(self) -> int:
        return int(self.experts["down"].weight.shape[0])

    def route(self, x_flat, stream=None):
        """(scores float32 [T, k], experts int32 [T, k]) (moe.rs:66-82)."""
        logits = self.gate(x_flat).contiguous()
        return ops.moe_route(logits, self.k, self.norm_topk_prob, stream)

    # at most this many (token, slot) rows skip the sort: every row is its own
    # GEMV (the grouped kernel has nothing to share), so rows stay in (token,
    # slot) order and the index maps are fixed per token count
    UNSORTED_ROWS = 16

    def _identity_maps(self, n, device):
        key = (n, device)
        cache = self.__dict__.setdefault("_maps", {})
        if key not in cache:
            rows = torch.arange(n * self.k, device=device, dtype=torch.int32)
            cache[key] = ((rows // self.k).contiguous(), rows)
        return cache[key]

    def experts_forward(self, x_flat, scores, idx, stream=None):
        n, d = x_flat.shape
        E = self.num_experts()
        idx = idx.to(torch.int32).contiguous()
        if n * self.k <= self.UNSORTED_ROWS:
            tokens, inverse = self._identity_maps(n, x_flat.device)
            rhs, srt = idx.reshape(-1), False
        else:
            tokens, rhs, inverse, _ = ops.moe_sort(idx, E, stream)
            srt = True
        x3 = x_flat.reshape(n, 1, d).contiguous()
        if "gate_up" in self.experts:
            gu = self.experts["gate_up"]
            h = ops.gather_qmm_swiglu(x3, gu.weight, gu.scales, gu.biases, tokens, rhs,
                                      gu.group_size, gu.bits, gu.mode, srt, stream)
        else:
            g = _gqmm(x3, self.experts["gate"], rhs, tokens, srt, stream=stream)
            u = _gqmm(x3, self.experts["up"], rhs, tokens, srt, stream=stream)
            h = (F.silu(g) * u).contiguous()
        y = _gqmm(h, self.experts["down"], rhs, sorted_indices=srt, stream=stream)
        return ops.moe_combine(y, inverse, idx, scores.contiguous(), E, stream)

    def _token_path(self, x_flat) -> bool:
        """One decode token with fused affine 4-bit gate_up experts: route,
        experts and combine run as :func:`ops.moe_token` (two launches)."""
        gu, dn = self.experts.get("gate_up"), self.experts["down"]
        if x_flat.shape[0] != 1 or gu is None:
            return False
        return all(e.mode == "affine" and e.bits == 4 and e.group_size in (32, 64, 128) and
                   e.biases is not None and e.scales.dtype == x_flat.dtype for e in (gu, dn)) and \
            x_flat.dtype in (torch.bfloat16, torch.float16) and self.num_experts() <= 512 and \
            self.k <= min(32, self.num_experts()) and gu.group_size == dn.group_size and \
            x_flat.shape[1] % 32 == 0 and x_flat.shape[1] <= 8192 and \
            gu.weight.shape[1] % 64 == 0 and gu.weight.shape[1] // 2 <= 2048

    def token_forward(self, x_flat, logits, stream=None):
        gu, dn = self.experts["gate_up"], self.experts["down"]
        return ops.moe_token(logits, x_flat.contiguous(), (gu.weight, gu.scales, gu.biases),
                             (dn.weight, dn.scales, dn.biases), self.k, self.norm_topk_prob,
                             gu.group_size, 4, stream)

    def __call__(self, x, stream=None):
        b, l, d = x.shape
        x_flat = x.reshape(b * l, d)
        if self._token_path(x_flat):
            out = self.token_forward(x_flat, self.gate(x_flat).contiguous(), stream)
        else:
            scores, idx = self.route(x_flat, stream)
            out = self.experts_forward(x_flat, scores, idx, stream)
        shared = self.shared_expert(x_flat, stream)
        gate = torch.sigmoid(self.shared_expert_gate(x_flat))
        return (out + (shared * gate).float()).reshape(b, l, d)
