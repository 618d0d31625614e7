"""GPU parity of the fused SwiGLU, the quantized-table row gather and the
on-device MoE routing (route / sort / combine), through the C ABI.

Bars: the row gather, the routing (scores and expert ids), the sort and the
combine are bit-exact against the oracle on the same inputs.  The fused
SwiGLU is bit-exact against the oracle's SwiGLU applied to the library's own
quantized_matmul / gather_qmm of the same fused weight (the fused kernels
compute the same sums), and its product is within the matmul tolerance of
the oracle's quantized matmul.
Reference surface: mlx/src/nn/mlp.rs:27-33, mlx/src/nn/activations.rs:7-10,
mlx/src/nn/embedding.rs:62-72, mlx/src/nn/moe.rs:55-183.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import (TDT, as_f64, from_np, rand_affine, rand_fp, rel_err, to_np,
                     words_to_torch)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from ironmlx_amd import ops as _ops
    from ironmlx_amd import _lib
    _lib.load()
    return _ops


def _bits(t: torch.Tensor, dt: str) -> np.ndarray:
    a = to_np(t, dt)
    return np.ascontiguousarray(a).view(np.uint32 if dt == "f32" else np.uint16)


def _weights(rng, mode, rows, K, dt, lead=()):
    if mode == "affine":
        w, s, b = rand_affine(rng, rows, K, 64, 4, dt, lead)
        return words_to_torch(w), from_np(s, dt), from_np(b, dt), (w, s, b)
    w, sc = rand_fp(rng, rows, K, mode, lead)
    return words_to_torch(w), torch.from_numpy(sc).cuda(), None, (w, sc, None)


# ------------------------------------------------------------------ fused SwiGLU
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("mode", ["affine", "mxfp4", "nvfp4"])
@pytest.mark.parametrize("M,I,K", [(1, 300, 1024), (1, 2048, 4096), (1, 14336, 4096), (1, 4096, 14336),
                                   (3, 512, 1024), (16, 1000, 2048), (128, 1024, 1024),
                                   (4, 14336, 4096), (16, 4096, 4096), (32, 4100, 2048), (8, 2048, 4096)])
def test_quantized_swiglu(ops, dt, mode, M, I, K):
    print(f"swiglu {mode} {dt} M={M} I={I} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + I + K)
    w, s, b, _ = _weights(rng, mode, 2 * I, K, dt)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M + I)).to(TDT[dt]).cuda()
    got = ops.quantized_swiglu(x, w, s, b, mode=mode)
    gu = ops.quantized_matmul(x, w, s, b, True, mode=mode)
    torch.cuda.synchronize()
    assert got.shape == (M, I)
    ref = oracle.swiglu(to_np(gu, dt), dt)
    # the factored decode-width kernels (affine 4-bit, 2 <= M <= 32) may split
    # K over their waves differently in the fused form: within tolerance there;
    # every other path computes exactly the sums of the unfused product
    fac = mode == "affine" and 2 <= M <= 32
    if fac:
        assert rel_err(as_f64(to_np(got, dt), dt), as_f64(ref, dt)) <= 1e-2
    else:
        assert np.array_equal(_bits(got, dt), np.ascontiguousarray(ref).view(np.uint16))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_quantized_swiglu_vs_oracle_product(ops, dt):
    # the fused path's math, end to end against the oracle's matmul
    rng = np.random.default_rng(5)
    I, K = 384, 1024
    w, s, b = rand_affine(rng, 2 * I, K, 64, 4, dt)
    xn = oracle.from_float(rng.standard_normal((1, K)).astype(np.float32), dt)
    got = ops.quantized_swiglu(from_np(xn, dt), words_to_torch(w), from_np(s, dt), from_np(b, dt))
    gu = oracle.qmm(xn, dt, w, s, b, dt, True, 64, 4)
    g, u = as_f64(gu, dt)[:, :I], as_f64(gu, dt)[:, I:]
    ref = g / (1.0 + np.exp(-g)) * u
    assert rel_err(as_f64(to_np(got, dt), dt), ref) <= 1e-2


def test_quantized_swiglu_errors(ops):
    w = torch.zeros(301, 128, dtype=torch.int32, device="cuda").view(torch.uint32)
    s = torch.zeros(301, 16, dtype=torch.bfloat16, device="cuda")
    x = torch.zeros(1, 1024, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ops.IqmmError, match="even number of rows"):
        ops.quantized_swiglu(x, w, s, s)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("T,sorted_", [(1, False), (1, True), (64, True), (512, True), (16, False)])
def test_gather_qmm_swiglu(ops, dt, T, sorted_):
    print(f"gather swiglu {dt} T={T} sorted={sorted_}", flush=True)
    rng = np.random.default_rng(T + 3)
    E, I, H, k = 32, 512, 2048, 8
    w, s, b, _ = _weights(rng, "affine", 2 * I, H, dt, lead=(E,))
    x = torch.randn(T, 1, H, generator=torch.Generator().manual_seed(T)).to(TDT[dt]).cuda()
    ex = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32))
    flat = ex.reshape(-1)
    if sorted_:
        order = torch.argsort(flat, stable=True)
        rhs = flat[order].contiguous().cuda()
        lhs = (order // k).to(torch.int32).contiguous().cuda()
    else:
        rhs = flat.contiguous().cuda()
        lhs = (torch.arange(T * k) // k).to(torch.int32).cuda()
    got = ops.gather_qmm_swiglu(x, w, s, b, lhs, rhs, sorted_indices=sorted_)
    # the fused call picks the same kernel family as gather_qmm for these rows
    gu = ops.gather_qmm(x, w, s, b, lhs, rhs, True, sorted_indices=sorted_)
    torch.cuda.synchronize()
    assert got.shape == (T * k, 1, I)
    ref = oracle.swiglu(to_np(gu, dt).reshape(T * k, 2 * I), dt)
    assert np.array_equal(_bits(got, dt).reshape(T * k, I), np.ascontiguousarray(ref).view(np.uint16))


@pytest.mark.parametrize("gs,I", [(32, 512), (128, 512), (64, 520), (32, 520), (128, 520)])
@pytest.mark.parametrize("T", [64, 512])
def test_gather_qmm_swiglu_group_sizes(ops, gs, I, T):
    """The grouped SwiGLU epilogue at every group size (gs 32: four groups per
    128-code chunk group, gs 128: one) and with a ragged I (not a multiple of
    the 32-column tile): bit-exact with the oracle's SwiGLU of the gather_qmm
    product."""
    print(f"gather swiglu gs={gs} I={I} T={T}", flush=True)
    dt = "bf16"
    rng = np.random.default_rng(gs + I + T)
    E, H, k = 32, 2048, 8
    wn, sn, bn = rand_affine(rng, 2 * I, H, gs, 4, dt, (E,))
    w, s, b = words_to_torch(wn), from_np(sn, dt), from_np(bn, dt)
    x = torch.randn(T, 1, H, generator=torch.Generator().manual_seed(T + gs)).to(TDT[dt]).cuda()
    ex = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32))
    flat = ex.reshape(-1)
    order = torch.argsort(flat, stable=True)
    rhs = flat[order].contiguous().cuda()
    lhs = (order // k).to(torch.int32).contiguous().cuda()
    got = ops.gather_qmm_swiglu(x, w, s, b, lhs, rhs, gs, 4, sorted_indices=True)
    gu = ops.gather_qmm(x, w, s, b, lhs, rhs, True, gs, 4, sorted_indices=True)
    torch.cuda.synchronize()
    ref = oracle.swiglu(to_np(gu, dt).reshape(T * k, 2 * I), dt)
    assert np.array_equal(_bits(got, dt).reshape(T * k, I), np.ascontiguousarray(ref).view(np.uint16))
    # and the product itself against the oracle's per-row products
    xs = to_np(x[:, 0], dt)[(order // k).numpy()]
    rn = rhs.cpu().numpy()
    refp = np.zeros((T * k, 2 * I))
    for e in np.unique(rn):
        rows = np.nonzero(rn == e)[0]
        refp[rows] = oracle.qmv_affine(xs[rows], dt, wn[e], sn[e], bn[e], dt, gs, 4, odt="f32", nthreads=8)
    assert rel_err(as_f64(to_np(gu, dt).reshape(T * k, 2 * I), dt), refp) <= 1e-2


@pytest.mark.parametrize("H,I,dt", [(2048, 512, "bf16"), (1024, 520, "f16"), (4096, 264, "bf16")])
def test_gather_stream_few_rows_per_expert(ops, H, I, dt):
    """Sorted gather_qmm with at most 8 rows per expert on average and K of
    1024 or more: the per-expert streaming kernel (K = 1024 / 2048 / 4096:
    two, four and eight waves; a ragged N; one lhs index out of range, whose
    row is NaN).  The product against the oracle's per-row products, and the
    fused SwiGLU bit-exact against the oracle's SwiGLU of that product;
    expert indices outside [0, E) give NaN rows."""
    print(f"gather stream H={H} I={I} {dt}", flush=True)
    rng = np.random.default_rng(H + I)
    E, k, T = 64, 8, 40   # 320 rows over 64 experts: 5 per expert
    wn, sn, bn = rand_affine(rng, 2 * I, H, 64, 4, dt, (E,))
    w, s, b = words_to_torch(wn), from_np(sn, dt), from_np(bn, dt)
    x = torch.randn(T, 1, H, generator=torch.Generator().manual_seed(H)).to(TDT[dt]).cuda()
    ex = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32))
    flat = ex.reshape(-1)
    order = torch.argsort(flat, stable=True)
    rhs_h = flat[order].contiguous()
    rhs_h[:2] = -1       # expert indices outside [0, E) sort first / last: NaN rows
    rhs_h[-1] = E + 5
    rhs = rhs_h.cuda()
    lhs_h = (order // k).to(torch.int32)
    lhs_h[7] = T + 3  # out of range: NaN row
    lhs = lhs_h.contiguous().cuda()
    gu = ops.gather_qmm(x, w, s, b, lhs, rhs, True, 64, 4, sorted_indices=True)
    got = ops.gather_qmm_swiglu(x, w, s, b, lhs, rhs, 64, 4, sorted_indices=True)
    torch.cuda.synchronize()
    g = as_f64(to_np(gu, dt).reshape(T * k, 2 * I), dt)
    bad = [0, 1, 7, T * k - 1]
    assert np.all(np.isnan(g[bad]))
    ok = np.ones(T * k, bool)
    ok[bad] = False
    xs = to_np(x[:, 0], dt)[np.clip(lhs_h.numpy(), 0, T - 1)]
    rn = rhs.cpu().numpy()
    refp = np.zeros((T * k, 2 * I))
    for e in np.unique(rn[ok]):
        rows = np.nonzero((rn == e) & ok)[0]
        refp[rows] = oracle.qmv_affine(xs[rows], dt, wn[e], sn[e], bn[e], dt, 64, 4, odt="f32", nthreads=8)
    assert rel_err(g[ok], refp[ok]) <= 1e-2
    ref = oracle.swiglu(to_np(gu, dt).reshape(T * k, 2 * I)[ok], dt)
    assert np.array_equal(_bits(got, dt).reshape(T * k, I)[ok], np.ascontiguousarray(ref).view(np.uint16))
    assert np.all(np.isnan(as_f64(to_np(got, dt), dt).reshape(T * k, I)[bad]))


# ------------------------------------------------------------------ row gather
@pytest.mark.parametrize("mode,bits,gs", [("affine", 4, 64), ("affine", 3, 32), ("affine", 8, 128),
                                          ("mxfp4", 4, 32), ("mxfp8", 8, 32), ("nvfp4", 4, 16)])
@pytest.mark.parametrize("idt", [torch.int32, torch.int64])
def test_dequantize_rows_bit_exact(ops, mode, bits, gs, idt):
    rng = np.random.default_rng(bits + gs)
    rows, K, dt = 1000, 512, "bf16"
    if mode == "affine":
        w, s, b = rand_affine(rng, rows, K, gs, bits, dt)
        ts, tb = from_np(s, dt), from_np(b, dt)
        table = oracle.dequantize(w, s, b, dt, gs, bits)
    else:
        w, s = rand_fp(rng, rows, K, mode)
        ts, tb, b = torch.from_numpy(s).cuda(), None, None
        table = oracle.dequantize(w, s, None, "f32", None, None, mode)
    idx = np.array([[0, 999, 17, -1], [-1000, 5, 5, 123]], np.int64)
    got = ops.dequantize_rows(words_to_torch(w), ts, tb, torch.from_numpy(idx).to(idt).cuda(),
                              None if mode != "affine" else gs, None if mode != "affine" else bits, mode)
    assert got.shape == (2, 4, K)
    ref = table[idx % rows]
    assert np.array_equal(_bits(got, "bf16"), np.ascontiguousarray(ref).view(np.uint16))


def test_dequantize_rows_out_of_range_nan(ops):
    rng = np.random.default_rng(9)
    w, s, b = rand_affine(rng, 64, 256, 64, 4, "f16")
    idx = torch.tensor([3, 64, -65, 2**40], dtype=torch.int64, device="cuda")
    got = ops.dequantize_rows(words_to_torch(w), from_np(s, "f16"), from_np(b, "f16"), idx)
    table = oracle.dequantize(w, s, b, "f16", 64, 4)
    g = got.cpu().numpy()
    assert np.array_equal(g[0].view(np.uint16), table[3].view(np.uint16))
    assert np.all(np.isnan(g[1:]))


# ------------------------------------------------------------------ routing
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("T,E,k", [(1, 256, 8), (64, 256, 8), (512, 256, 8), (33, 60, 4), (7, 2048, 32),
                                   (5, 3, 3)])
@pytest.mark.parametrize("norm", [True, False])
def test_moe_route_bit_exact(ops, dt, T, E, k, norm):
    rng = np.random.default_rng(T * 3 + E + k)
    lg = oracle.from_float(rng.standard_normal((T, E)).astype(np.float32) * 2, dt)
    scores, experts = ops.moe_route(from_np(lg, dt), k, norm)
    rs, re = oracle.moe_route(lg, dt, k, norm)
    assert np.array_equal(experts.cpu().numpy(), re)
    assert np.array_equal(scores.cpu().numpy().view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("T,k,E", [(1, 8, 256), (64, 8, 256), (512, 8, 256), (4096, 8, 256), (3000, 4, 60),
                                   (17, 2, 65535)])
def test_moe_sort_bit_exact(ops, T, k, E):
    rng = np.random.default_rng(T + k)
    ex = rng.integers(0, E, (T, k)).astype(np.int32)
    if T > 10:
        ex[3, 0] = -5
        ex[9, k - 1] = E
    tokens, srt, inv, offs = ops.moe_sort(torch.from_numpy(ex).cuda(), E)
    rt, rsrt, rinv, roffs = oracle.moe_sort(ex, E)
    for g, r in ((tokens, rt), (srt, rsrt), (inv, rinv), (offs, roffs)):
        assert np.array_equal(g.cpu().numpy(), r)


def test_moe_sort_limits(ops):
    ex = torch.zeros(4097, 8, dtype=torch.int32, device="cuda")
    with pytest.raises(ops.IqmmError, match="32768"):
        ops.moe_sort(ex, 256)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("T,k,E,D", [(1, 8, 256, 2048), (64, 8, 256, 2048), (300, 4, 60, 1000), (5, 3, 17, 1001)])
def test_moe_combine_bit_exact(ops, dt, T, k, E, D):
    rng = np.random.default_rng(T + D)
    lg = oracle.from_float(rng.standard_normal((T, E)).astype(np.float32), dt)
    scores, experts = ops.moe_route(from_np(lg, dt), k, True)
    _, _, inv, _ = ops.moe_sort(experts, E)
    y = torch.randn(T * k, 1, D, generator=torch.Generator().manual_seed(D)).to(TDT[dt]).cuda()
    got = ops.moe_combine(y, inv, experts, scores, E)
    ref = oracle.moe_combine(to_np(y, dt).reshape(T * k, D), dt, inv.cpu().numpy(), experts.cpu().numpy(),
                             scores.cpu().numpy(), E)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------------------ edge cases
def test_moe_empty_and_single(ops):
    """T = 0 tokens (empty outputs, zero offsets), E = 1 / k = 1, and a combine
    width that is not a multiple of the 256-column workgroup."""
    lg = torch.zeros((0, 256), dtype=torch.bfloat16, device="cuda")
    sc, ex = ops.moe_route(lg, 8, True)
    assert sc.shape == (0, 8) and ex.shape == (0, 8)
    tok, srt, inv, off = ops.moe_sort(ex, 256)
    assert tok.numel() == 0 and torch.equal(off.cpu(), torch.zeros(257, dtype=torch.int32))
    y = torch.zeros((0, 1, 64), dtype=torch.bfloat16, device="cuda")
    assert ops.moe_combine(y, inv, ex, sc, 256).shape == (0, 64)

    lg1 = torch.randn((5, 1), device="cuda").to(torch.bfloat16)
    sc1, ex1 = ops.moe_route(lg1, 1, True)
    assert torch.equal(ex1.cpu(), torch.zeros((5, 1), dtype=torch.int32))
    assert torch.equal(sc1.cpu(), torch.ones((5, 1)))

    rng = np.random.default_rng(4)
    T, k, E, D = 9, 3, 16, 1000
    lgn = oracle.from_float(rng.standard_normal((T, E)).astype(np.float32), "bf16")
    sc2, ex2 = ops.moe_route(from_np(lgn, "bf16"), k, False)
    _, _, inv2, _ = ops.moe_sort(ex2, E)
    y2 = torch.randn((T * k, D), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).cuda()
    got = ops.moe_combine(y2, inv2, ex2, sc2, E)
    ref = oracle.moe_combine(to_np(y2, "bf16"), "bf16", inv2.cpu().numpy(), ex2.cpu().numpy(),
                             sc2.cpu().numpy(), E)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_fused_and_gather_empty(ops):
    rng = np.random.default_rng(6)
    w, s, b = rand_affine(rng, 2 * 96, 1024, 64, 4, "bf16")
    tw, ts, tb = words_to_torch(w), from_np(s, "bf16"), from_np(b, "bf16")
    x0 = torch.zeros((0, 1024), dtype=torch.bfloat16, device="cuda")
    assert ops.quantized_swiglu(x0, tw, ts, tb).shape == (0, 96)
    idx0 = torch.zeros((0,), dtype=torch.int32, device="cuda")
    assert ops.dequantize_rows(tw, ts, tb, idx0).shape == (0, 1024)
    # odd I: the last GEMV wave holds a single output
    w3, s3, b3 = rand_affine(rng, 2 * 97, 1024, 64, 4, "bf16")
    x1 = torch.randn((1, 1024), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    got = ops.quantized_swiglu(x1, words_to_torch(w3), from_np(s3, "bf16"), from_np(b3, "bf16"))
    gu = ops.quantized_matmul(x1, words_to_torch(w3), from_np(s3, "bf16"), from_np(b3, "bf16"), True)
    ref = oracle.swiglu(to_np(gu, "bf16"), "bf16")
    assert np.array_equal(_bits(got, "bf16"), np.ascontiguousarray(ref).view(np.uint16))


def test_moe_combine_unsorted_rows(ops):
    """Rows in (token, slot) order with the identity inverse (the sort is
    skipped for decode): still summed in ascending expert order."""
    rng = np.random.default_rng(8)
    T, k, E, D = 2, 8, 256, 2048
    lg = oracle.from_float(rng.standard_normal((T, E)).astype(np.float32), "bf16")
    scores, experts = ops.moe_route(from_np(lg, "bf16"), k, True)
    inv = torch.arange(T * k, dtype=torch.int32, device="cuda")
    y = torch.randn(T * k, 1, D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).cuda()
    got = ops.moe_combine(y, inv, experts, scores, E)
    ref = oracle.moe_combine(to_np(y, "bf16").reshape(T * k, D), "bf16", inv.cpu().numpy(),
                             experts.cpu().numpy(), scores.cpu().numpy(), E)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))
