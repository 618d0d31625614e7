"""Host-side caller logic that needs no GPU: config parsing, quantized /
dense dispatch by key (mlx/src/nn/linear.rs:97-126) and the fused-expert
split layout (mlx/src/model/qwen35.rs:655-775)."""
import torch

from ironmlx_amd import nn


def test_quantization_config_defaults():
    assert nn.QuantizationConfig.from_dict({}) == nn.QuantizationConfig(64, 4, "affine")
    assert nn.QuantizationConfig.from_dict({"bits": 8, "group_size": 32}).bits == 8
    assert nn.QuantizationConfig.from_dict(None) is None


def test_linear_layer_dispatch():
    wq = {"l.weight": torch.zeros(4, 8, dtype=torch.int32), "l.scales": torch.zeros(4, 1),
          "l.biases": torch.zeros(4, 1)}
    q = nn.LinearLayer.from_weights(wq, "l", 64, 4)
    assert isinstance(q, nn.QuantizedLinear) and q.biases is not None
    wd = {"l.weight": torch.zeros(4, 8), "l.bias": torch.ones(4)}
    d = nn.LinearLayer.from_weights(wd, "l")
    assert isinstance(d, nn.Linear)
    assert torch.equal(d(torch.zeros(2, 8)), torch.ones(2, 4))


def test_split_fused_experts_layout():
    E, I, H, gs = 3, 8, 64, 32
    p = "model.layers.0"
    gu_w = torch.arange(E * 2 * I * (H // 8), dtype=torch.int32).reshape(E, 2 * I, H // 8)
    gu_s = torch.randn(E, 2 * I, H // gs)
    weights = {f"{p}.mlp.experts.gate_up_proj.weight": gu_w,
               f"{p}.mlp.experts.gate_up_proj.scales": gu_s,
               f"{p}.mlp.experts.gate_up_proj.biases": gu_s + 1,
               f"{p}.mlp.experts.down_proj.weight": torch.zeros(E, H, I // 8, dtype=torch.int32),
               f"{p}.mlp.experts.down_proj.scales": torch.zeros(E, H, 1),
               f"{p}.mlp.experts.down_proj.biases": torch.zeros(E, H, 1)}
    out = nn.split_fused_experts(weights, p, gs, 4)
    assert out["gate"].weight.shape == (E, I, H // 8)
    assert torch.equal(out["gate"].weight, gu_w[:, :I])
    assert torch.equal(out["up"].weight, gu_w[:, I:])
    assert torch.equal(out["up"].biases, gu_s[:, I:] + 1)
    assert out["gate"].weight.is_contiguous() and out["down"].weight.shape == (E, H, I // 8)
