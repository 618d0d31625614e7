"""GPU checks of the caller layer: QuantizedLinear == quantized_matmul,
QuantizedEmbedding == dequantize + row gather, FusedMLP against MLP, and
MoEMLP (device routing, sorted gather_qmm, fused or split gate / up) against
the reference's per-expert loop restated with quantized_matmul
(mlx/src/nn/moe.rs:84-170)."""
import pytest
import torch
import torch.nn.functional as F

from ironmlx_amd import nn, ops

pytestmark = pytest.mark.gpu


def _q(W, gs=64, bits=4):
    return ops.quantize(W, gs, bits)


def test_quantized_linear_and_embedding():
    torch.manual_seed(0)
    W = (torch.randn(96, 256, device="cuda") * 0.02).to(torch.bfloat16)
    w, s, b = _q(W)
    lin = nn.QuantizedLinear(w, s, b, 64, 4)
    x = torch.randn(3, 5, 256, device="cuda").to(torch.bfloat16)
    assert torch.equal(lin(x), ops.quantized_matmul(x, w, s, b, True, 64, 4, "affine"))
    emb = nn.QuantizedEmbedding(w, s, b, 64, 4)
    tok = torch.tensor([[3, 0, 95]], device="cuda")
    table = ops.dequantize(w, s, b, 64, 4)
    assert torch.equal(emb(tok), table[tok])


def test_fused_mlp_matches_mlp():
    torch.manual_seed(2)
    H, I = 512, 1536
    dt = torch.bfloat16
    lin = lambda o, i: nn.QuantizedLinear(*_q((torch.randn(o, i, device="cuda") * 0.02).to(dt)), 64, 4)
    mlp = nn.MLP(lin(I, H), lin(I, H), lin(H, I))
    fused = nn.FusedMLP.from_mlp(mlp)
    for M in (1, 5, 200):
        x = torch.randn(M, H, device="cuda").to(dt)
        ref, got = mlp(x).float(), fused(x).float()
        assert ((got - ref).abs().max() / ref.abs().max()).item() <= 1e-2


def test_fused_qkv_matches_projections():
    torch.manual_seed(3)
    dt = torch.bfloat16
    lin = lambda o, i: nn.QuantizedLinear(*_q((torch.randn(o, i, device="cuda") * 0.02).to(dt)), 64, 4)
    q, k, v = lin(512, 1024), lin(128, 1024), lin(128, 1024)
    f = nn.FusedQKV(q, k, v)
    for M in (1, 7):
        x = torch.randn(M, 1024, device="cuda").to(dt)
        for got, ref in zip(f(x), (q(x), k(x), v(x))):
            assert ((got.float() - ref.float()).abs().max() / ref.float().abs().max()).item() <= 1e-2


@pytest.mark.parametrize("T", [37, 2, 1])
@pytest.mark.parametrize("fused", [False, True])
def test_moe_matches_per_expert_loop(fused, T):
    # T = 2 (8 rows) skips the sort: one GEMV row per (token, slot); T = 1 with
    # the fused gate_up experts runs the one-token kernels (ops.moe_token)
    torch.manual_seed(1)
    E, H, I, k = 16, 256, 128, 4
    dt = torch.bfloat16
    def stack(n_out, n_in):
        W = (torch.randn(E * n_out, n_in, device="cuda") * 0.02).to(dt)
        w, s, b = _q(W)
        return w.view(E, n_out, -1), s.view(E, n_out, -1), b.view(E, n_out, -1)
    gate_up = stack(2 * I, H)
    down = stack(H, I)
    p = "layers.0"
    weights = {f"{p}.mlp.experts.gate_up_proj.weight": gate_up[0],
               f"{p}.mlp.experts.gate_up_proj.scales": gate_up[1],
               f"{p}.mlp.experts.gate_up_proj.biases": gate_up[2],
               f"{p}.mlp.experts.down_proj.weight": down[0],
               f"{p}.mlp.experts.down_proj.scales": down[1],
               f"{p}.mlp.experts.down_proj.biases": down[2]}
    experts = (nn.stack_fused_experts if fused else nn.split_fused_experts)(weights, p, 64, 4)
    split = nn.split_fused_experts(weights, p, 64, 4)
    router = nn.Linear((torch.randn(E, H, device="cuda") * 0.1).to(dt))
    sh = [nn.QuantizedLinear(*_q((torch.randn(o, i, device="cuda") * 0.02).to(dt)), 64, 4)
          for (o, i) in [(I, H), (I, H), (H, I)]]
    shared = nn.MLP(*sh)
    sgate = nn.Linear((torch.randn(1, H, device="cuda") * 0.1).to(dt))
    moe = nn.MoEMLP(router, experts, shared, sgate, k, True)
    x = torch.randn(1, T, H, device="cuda").to(dt)
    got = moe(x).float()

    # reference: host loop over used experts, one quantized_matmul per projection
    xf = x.reshape(T, H)
    scores, idx = moe.route(xf)
    ref = torch.zeros(T, H, device="cuda")
    for e in range(E):
        rows, slots = (idx == e).nonzero(as_tuple=True)
        if rows.numel() == 0:
            continue
        xe = xf[rows]
        def proj(name, v):
            st = split[name]
            return ops.quantized_matmul(v, st.weight[e], st.scales[e], st.biases[e], True, 64, 4)
        ye = proj("down", F.silu(proj("gate", xe)) * proj("up", xe))
        ref.index_add_(0, rows, ye.float() * scores[rows, slots].unsqueeze(-1))
    ref = ref + (shared(xf).float() * torch.sigmoid(sgate(xf).float()))
    err = ((got.reshape(T, H) - ref).abs().max() / ref.abs().max()).item()
    assert err <= 1e-2, err


def test_checkpoint_layer_runs(tmp_path):
    """A quantized layer read from a safetensors checkpoint (loader.rs:13-44
    key scheme) feeds the kernels unchanged."""
    import numpy as np
    import safetensors.numpy as sn
    import oracle
    from ironmlx_amd import loader
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((512, 1024)) * 0.02).astype(np.float32)
    wq, s, b = oracle.affine_quantize(w, "f32", 64, 4, "f16")
    sn.save_file({"p.weight": wq, "p.scales": s, "p.biases": b}, str(tmp_path / "model.safetensors"))
    weights = loader.load_model_weights(str(tmp_path))
    lin = loader.quantized_layers(weights, nn.QuantizationConfig())["p"]
    x = rng.standard_normal((3, 1024)).astype(np.float16)
    got = lin(torch.from_numpy(x).cuda()).cpu().numpy().astype(np.float64)
    ref = oracle.qmm(x, "f16", wq, s, b, "f16", True, 64, 4).astype(np.float64)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-2
