"""Pins the oracle's SwiGLU and MoE-routing functions (oracle/iqmm_oracle.c,
iqo_expf / iqo_swiglu / iqo_moe_route / iqo_moe_sort / iqo_moe_combine)
before they check the library.  Independent checks only: float64 exp and
softmax, numpy's stable argsort, closed forms of silu, and float64 weighted
sums.  No GPU needed.

Reference behaviour restated: mlx/src/nn/activations.rs:7-10 (silu as
x * sigmoid(x)), mlx/src/nn/mlp.rs:27-33 (silu(gate) * up),
mlx/src/nn/moe.rs:67-82 (softmax, stable argsort of -p, top-k,
normalisation), :92-104 (per-expert token lists), :146-168 (weighted sum).
"""
import numpy as np
import pytest

import oracle


def _ulps(got, ref64):
    sp = np.spacing(np.abs(ref64).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - ref64) / sp


def test_expf_within_one_ulp():
    x = np.linspace(-87.0, 88.0, 100001, dtype=np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, 1e-8, -1e-8, 0.5, -0.5, 0.34657359, 0.34657360])])
    u = _ulps(oracle.expf(x), np.exp(x.astype(np.float64)))
    assert u.max() <= 1.0


def test_expf_special_points():
    e = oracle.expf(np.float32([0.0, 89.0, -104.0, np.inf, -np.inf]))
    assert e[0] == 1.0
    assert np.isinf(e[1]) and e[1] > 0 and np.isinf(e[3])
    assert e[2] == 0.0 and e[4] == 0.0
    assert np.isnan(oracle.expf(np.float32([np.nan]))[0])


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_swiglu_closed_forms(dt):
    # g = 0 -> 0; g large -> sigmoid rounds to 1 -> rn(g * u); g very negative -> 0
    g = np.float32([0.0, 30.0, 30.0, -200.0, 12.0])
    u = np.float32([5.0, 2.0, -0.75, 3.0, 1.5])
    gu = oracle.from_float(np.concatenate([g, u])[None, :], dt)
    out = oracle.to_float(oracle.swiglu(gu, dt), dt)[0]
    assert out[0] == 0.0
    assert out[1] == 60.0 and out[2] == -22.5
    assert out[3] == 0.0
    # 12 * sigmoid(12) in dt, then times 1.5
    s = oracle.to_float(oracle.from_float(np.float32([1.0 / (1.0 + np.exp(-12.0))]), dt), dt)[0]
    a = oracle.to_float(oracle.from_float(np.float32([12.0 * s]), dt), dt)[0]
    assert out[4] == oracle.to_float(oracle.from_float(np.float32([a * 1.5]), dt), dt)[0]


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_swiglu_against_float64(dt):
    rng = np.random.default_rng(0)
    g = rng.standard_normal((64, 96)).astype(np.float32) * 3
    u = rng.standard_normal((64, 96)).astype(np.float32)
    gu = oracle.from_float(np.concatenate([g, u], axis=1), dt)
    gf = oracle.to_float(gu, dt).astype(np.float64)
    ref = gf[:, :96] / (1.0 + np.exp(-gf[:, :96])) * gf[:, 96:]
    got = oracle.to_float(oracle.swiglu(gu, dt), dt).astype(np.float64)
    # three roundings to dt
    eps = {"bf16": 2.0 ** -8, "f16": 2.0 ** -11, "f32": 2.0 ** -24}[dt]
    tiny = {"bf16": 2.0 ** -133, "f16": 2.0 ** -24, "f32": 2.0 ** -149}[dt]  # subnormal spacing
    assert np.all(np.abs(got - ref) <= 4 * eps * np.abs(ref) + 4 * tiny)


def _softmax64(lg):
    z = lg - lg.max(axis=1, keepdims=True)
    e = np.exp(z)
    return e / e.sum(axis=1, keepdims=True)


def test_route_separated_logits_exact():
    # well-separated logits: the selection and order are fixed by float64
    rng = np.random.default_rng(1)
    T, E, k = 32, 256, 8
    lg = np.stack([rng.permutation(E) for _ in range(T)]).astype(np.float32) * np.float32(0.05)
    scores, experts = oracle.moe_route(lg, "f32", k, norm=False)
    p = _softmax64(lg.astype(np.float64))
    ref_idx = np.argsort(-p, axis=1, kind="stable")[:, :k]
    assert np.array_equal(experts, ref_idx)
    ref_p = np.take_along_axis(p, ref_idx, axis=1)
    assert np.allclose(scores, ref_p, rtol=1e-6, atol=0)
    s_norm, e_norm = oracle.moe_route(lg, "f32", k, norm=True)
    assert np.array_equal(e_norm, ref_idx)
    assert np.allclose(s_norm.sum(axis=1), 1.0, atol=1e-6)
    assert np.allclose(s_norm, ref_p / ref_p.sum(axis=1, keepdims=True), rtol=1e-6)


def test_route_ties_take_lower_id():
    lg = np.zeros((2, 16), np.float32)
    lg[0, [3, 9, 12]] = 2.0   # three equal maxima
    lg[1, :] = 1.0            # all equal
    _, ex = oracle.moe_route(lg, "f32", 4, norm=True)
    assert ex[0].tolist() == [3, 9, 12, 0]
    assert ex[1].tolist() == [0, 1, 2, 3]


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_route_rounded_probabilities(dt):
    # probabilities are stored in the logits' dtype before selection: the
    # selection is numpy's stable argsort of those rounded values
    rng = np.random.default_rng(2)
    lg = oracle.from_float(rng.standard_normal((64, 256)).astype(np.float32), dt)
    scores, ex = oracle.moe_route(lg, dt, 8, norm=False)
    p = _softmax64(oracle.to_float(lg, dt).astype(np.float64))
    pr = oracle.to_float(oracle.from_float(p.astype(np.float32), dt), dt)
    ref_idx = np.argsort(-pr, axis=1, kind="stable")[:, :8]
    # float64 vs the oracle's float32 softmax: the rounded values agree except
    # where p sits within float32 error of a rounding boundary
    agree = np.mean(np.all(ex == ref_idx, axis=1))
    assert agree >= 0.95
    ok = np.all(ex == ref_idx, axis=1)
    assert np.array_equal(scores[ok], np.take_along_axis(pr, ref_idx, axis=1)[ok])


def test_sort_matches_numpy_stable():
    rng = np.random.default_rng(3)
    T, k, E = 100, 8, 64
    ex = rng.integers(0, E, (T, k)).astype(np.int32)
    ex[5, 2] = -1
    ex[7, 0] = E + 3     # invalid ids sort last, in row order
    tokens, srt, inv, offs = oracle.moe_sort(ex, E)
    flat = ex.reshape(-1)
    key = np.where((flat >= 0) & (flat < E), flat, E)
    order = np.argsort(key, kind="stable")
    assert np.array_equal(srt, flat[order])
    assert np.array_equal(tokens, order // k)
    assert np.array_equal(inv[order], np.arange(T * k))
    assert np.array_equal(offs, np.searchsorted(key[order], np.arange(E + 1), side="left"))


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_combine_weighted_sum(dt):
    rng = np.random.default_rng(4)
    T, k, E, D = 20, 4, 16, 48
    ex = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    sc = rng.random((T, k)).astype(np.float32)
    _, _, inv, _ = oracle.moe_sort(ex, E)
    y = oracle.from_float(rng.standard_normal((T * k, D)).astype(np.float32), dt)
    out = oracle.moe_combine(y, dt, inv, ex, sc, E)
    yf = oracle.to_float(y, dt).astype(np.float64)
    ref = np.zeros((T, D))
    for t in range(T):
        for s in range(k):
            ref[t] += yf[inv[t * k + s]] * sc[t, s]
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)
    # k = 1: exactly the product
    ex1 = ex[:, :1].copy()
    _, _, inv1, _ = oracle.moe_sort(ex1, E)
    out1 = oracle.moe_combine(y[:T], dt, inv1, ex1, sc[:, :1].copy(), E)
    assert np.array_equal(out1, (oracle.to_float(y[:T], dt)[inv1] * sc[:, :1]).astype(np.float32))
    # invalid experts are skipped; a token with none gets zeros
    ex2 = ex.copy()
    ex2[0, :] = -1
    out2 = oracle.moe_combine(y, dt, inv, ex2, sc, E)
    assert np.all(out2[0] == 0.0)
