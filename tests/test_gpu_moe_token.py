"""One decode token's routed experts in two launches (iqmm_moe_token): the
routing of moe_route, the fused gate_up SwiGLU of each routed expert, the
down projections and the ordered combine of moe_combine
(mlx/src/nn/moe.rs:55-183 for T = 1), against the oracle's restatement of the
same steps: moe_route, qmv_affine per expert row, swiglu (each step rounded
to the 16-bit type), qmv_affine of the down projection rounded to that type,
and moe_combine over the token's rows in slot order.

Bar: the routing is exact (same expert ids, checked through the result's
support); the result within 1e-2 of max |ref| (bf16 / fp16), the north-star
tolerance for the quantized products.  Shapes: Qwen3.5-MoE (E = 256, k = 8,
H = 2048, I = 512), small and ragged group sizes, fp16, fp32 logits."""
import numpy as np
import pytest
import torch

import oracle
from helpers import as_f64, from_np, rand_affine, rel_err, to_np, words_to_torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from ironmlx_amd import ops as _ops
    return _ops


def _reference(logits_np, ldt, x_np, dt, gu, dn, E, k, H, I, D, gs, norm=True):
    scores, experts = oracle.moe_route(logits_np.reshape(1, E), ldt, k, norm)
    gw, gsc, gbi = gu
    dw, dsc, dbi = dn
    ys = []
    for slot in range(k):
        e = int(experts[0, slot])
        if e < 0:
            ys.append(np.zeros(D, oracle.NP_STORAGE[dt]))
            continue
        g = oracle.qmv_affine(x_np.reshape(1, H), dt, gw[e], gsc[e], gbi[e], dt, gs, 4, odt=dt)
        h = oracle.swiglu(g, dt)
        ys.append(oracle.qmv_affine(h, dt, dw[e], dsc[e], dbi[e], dt, gs, 4, odt=dt).reshape(D))
    y = np.stack(ys)
    return oracle.moe_combine(y, dt, np.arange(k, dtype=np.int32), experts, scores, E), experts


CASES = [  # E, k, H, I, D, gs, dt, logits dtype
    (256, 8, 2048, 512, 2048, 64, "bf16", "bf16"),
    (16, 4, 256, 128, 256, 64, "bf16", "f32"),
    (64, 6, 1024, 96, 1000, 32, "f16", "f16"),
    (8, 2, 4096, 2048, 320, 128, "bf16", "bf16"),
    (300, 8, 512, 256, 512, 64, "bf16", "bf16"),
]


@pytest.mark.parametrize("E,k,H,I,D,gs,dt,ldt", CASES)
def test_moe_token_vs_oracle(ops, E, k, H, I, D, gs, dt, ldt):
    print(f"moe_token E={E} k={k} H={H} I={I} D={D} gs={gs} {dt}", flush=True)
    rng = np.random.default_rng(E + k + H + I)
    gu = rand_affine(rng, 2 * I, H, gs, 4, dt, (E,))
    dn = rand_affine(rng, D, I, gs, 4, dt, (E,))
    x = oracle.from_float(rng.standard_normal(H).astype(np.float32), dt)
    lg = oracle.from_float(rng.standard_normal(E).astype(np.float32) * 2, ldt) if ldt != "f32" else \
        rng.standard_normal(E).astype(np.float32) * 2
    ref, experts = _reference(lg, ldt, x, dt, gu, dn, E, k, H, I, D, gs)
    T = lambda a: from_np(a, dt)  # noqa: E731
    got = ops.moe_token(from_np(lg, ldt).reshape(1, E), T(x).reshape(1, H),
                        (words_to_torch(gu[0]), T(gu[1]), T(gu[2])),
                        (words_to_torch(dn[0]), T(dn[1]), T(dn[2])), k, True, gs, 4)
    torch.cuda.synchronize()
    assert got.shape == (1, D) and got.dtype == torch.float32
    assert rel_err(got.cpu().numpy().reshape(D), ref.reshape(D)) <= 1e-2


def test_moe_token_matches_unfused_block(ops):
    """Against the library's own route + gather_qmm_swiglu + gather_qmm +
    moe_combine on the same token (the path it replaces)."""
    from ironmlx_amd import nn
    torch.manual_seed(3)
    E, k, H, I = 256, 8, 2048, 512
    dt = torch.bfloat16

    def stack(n_out, n_in):
        w, s, b = ops.quantize((torch.randn(E * n_out, n_in, device="cuda") * 0.02).to(dt), 64, 4)
        return nn.StackedExperts(w.view(E, n_out, -1), s.view(E, n_out, -1), b.view(E, n_out, -1))
    experts = {"gate_up": stack(2 * I, H), "down": stack(H, I)}
    moe = nn.MoEMLP(None, experts, None, None, k, True)
    x = torch.randn(1, H, device="cuda").to(dt)
    logits = torch.randn(1, E, device="cuda").to(dt)
    sc, ex = ops.moe_route(logits, k, True)
    ref = moe.experts_forward(x, sc, ex)
    got = moe.token_forward(x, logits)
    torch.cuda.synchronize()
    err = ((got - ref).abs().max() / ref.abs().max()).item()
    assert err <= 1e-2, err


def test_moe_token_nan_logits_give_zero_row(ops):
    """No candidate expert (NaN logits): every slot is skipped, as the combine
    skips invalid experts, and the token's row is zero."""
    E, k, H, I, D = 16, 2, 256, 64, 128
    rng = np.random.default_rng(0)
    gu = rand_affine(rng, 2 * I, H, 64, 4, "bf16", (E,))
    dn = rand_affine(rng, D, I, 64, 4, "bf16", (E,))
    T = lambda a: from_np(a, "bf16")  # noqa: E731
    logits = torch.full((1, E), float("nan"), device="cuda").to(torch.bfloat16)
    x = torch.randn(1, H, device="cuda").to(torch.bfloat16)
    got = ops.moe_token(logits, x, (words_to_torch(gu[0]), T(gu[1]), T(gu[2])),
                        (words_to_torch(dn[0]), T(dn[1]), T(dn[2])), k, True, 64, 4)
    torch.cuda.synchronize()
    assert torch.equal(got, torch.zeros_like(got))
