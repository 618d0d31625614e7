"""GPU parity: the HIP library (through the C ABI, via ironmlx_amd.ops) against
the CPU oracle on identical seeded inputs.

Bars: dequantize and quantize are bit-exact; matmul outputs are within
max|got-ref| / max|ref| <= 1e-2 for bf16/fp16 outputs (fp32 accumulation) and
<= 2e-2 for the fp8/fp4 modes; fp32 outputs within 1e-4.
Reference surface: mlx/src/ops.rs:653-727, mlx/src/nn/moe.rs:55-183.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import (TDT, as_f64, from_np, rand_affine, rand_fp, rel_err, to_np,
                     words_to_np, words_to_torch)

pytestmark = pytest.mark.gpu

TOL = {"bf16": 1e-2, "f16": 1e-2, "f32": 1e-4}
TOL_FP = {"bf16": 2e-2, "f16": 2e-2, "f32": 1e-4}


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from ironmlx_amd import ops as _ops
    from ironmlx_amd import _lib
    _lib.load()
    return _ops


def _bits_equal(got: torch.Tensor, ref: np.ndarray, dt: str):
    g = to_np(got, dt)
    gb = g.view(np.uint32 if dt == "f32" else np.uint16)
    rb = np.ascontiguousarray(ref).view(np.uint32 if dt == "f32" else np.uint16)
    assert gb.shape == rb.shape
    bad = np.nonzero(gb != rb)
    assert bad[0].size == 0, f"{bad[0].size} mismatches, first at {[b[0] for b in bad]}: " \
                             f"{gb[tuple(b[0] for b in bad)]:#x} vs {rb[tuple(b[0] for b in bad)]:#x}"


# ------------------------------------------------------------------ dequantize
@pytest.mark.parametrize("sdt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_dequantize_affine_bit_exact(ops, bits, gs, sdt):
    rng = np.random.default_rng(100 + bits * 10 + gs)
    w, s, b = rand_affine(rng, 37, 512, gs, bits, sdt)
    got = ops.dequantize(words_to_torch(w), from_np(s, sdt), from_np(b, sdt), gs, bits)
    ref = oracle.dequantize(w, s, b, sdt, gs, bits)
    _bits_equal(got, ref, sdt)


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("K,sdt", [(16384, "bf16"), (4160, "f16")])
def test_dequantize_long_rows_bit_exact(ops, bits, K, sdt):
    """Rows of several 512-word segments (and a partial last one): the
    row-segment kernel's multi-block rows."""
    rng = np.random.default_rng(300 + bits + K % 7)
    w, s, b = rand_affine(rng, 5, K, 64 if K % 64 == 0 else 32, bits, sdt)
    gs = 64 if K % 64 == 0 else 32
    got = ops.dequantize(words_to_torch(w), from_np(s, sdt), from_np(b, sdt), gs, bits)
    ref = oracle.dequantize(w, s, b, sdt, gs, bits)
    _bits_equal(got, ref, sdt)


@pytest.mark.parametrize("odt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8", "nvfp4"])
def test_dequantize_fp_bit_exact(ops, mode, odt):
    rng = np.random.default_rng(7)
    w, sc = rand_fp(rng, 33, 512, mode)
    # include every element code and a spread of scale codes
    got = ops.dequantize(words_to_torch(w), torch.from_numpy(sc).cuda(), None, mode=mode,
                         dtype=TDT[odt])
    ref = oracle.dequantize(w, sc, None, None, None, None, mode, odt=odt)
    _bits_equal(got, ref, odt)


def test_dequantize_special_values(ops):
    # exhaustive codes x special scale/bias bit patterns (zeros, subnormals, max)
    codes = np.tile(np.arange(256, dtype=np.uint32), (12, 1))
    w = oracle.pack(codes, 8)
    sbits = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0x3C00, 0xBC00,
                      0x1400, 0x2E66, 0x5640, 0x0200], np.uint16)
    s = np.repeat(sbits[:, None], 2, axis=1).view(np.float16)
    b = np.repeat(sbits[::-1, None], 2, axis=1).view(np.float16)
    got = ops.dequantize(words_to_torch(w), from_np(s, "f16"), from_np(b, "f16"), 128, 8)
    ref = oracle.dequantize(w, s, b, "f16", 128, 8)
    _bits_equal(got, ref, "f16")
    # every e8m0 scale code (mxfp8), except NaN=255
    codes = np.tile(np.arange(0, 127, dtype=np.uint32), (255, 1))[:, :96]
    w = oracle.pack(codes, 8)
    sc = np.repeat(np.arange(255, dtype=np.uint8)[:, None], 3, axis=1)
    got = ops.dequantize(words_to_torch(w), torch.from_numpy(sc).cuda(), None, mode="mxfp8",
                         dtype=torch.float32)
    ref = oracle.dequantize(w, sc, None, None, None, None, "mxfp8", odt="f32")
    _bits_equal(got, ref, "f32")


# ------------------------------------------------------------------ quantize
@pytest.mark.parametrize("wdt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("bits,gs", [(2, 32), (3, 64), (4, 64), (4, 128), (5, 32), (6, 64),
                                     (8, 128)])
def test_quantize_affine_bit_exact(ops, bits, gs, wdt):
    rng = np.random.default_rng(bits * 1000 + gs)
    wf = (rng.standard_normal((40, 512)) * 0.02).astype(np.float32)
    wf[3, :gs] = 0.0                                  # constant group -> eps scale
    wf[5, :gs] = np.linspace(-1, 2, gs)               # q0 edge snap case
    wn = oracle.from_float(wf, wdt)
    tq, ts, tb = ops.quantize(from_np(wn, wdt), gs, bits)
    rq, rs, rb = oracle.affine_quantize(wn, wdt, gs, bits)
    assert np.array_equal(words_to_np(tq), rq)
    _bits_equal(ts, rs, wdt)
    _bits_equal(tb, rb, wdt)


@pytest.mark.parametrize("wdt", ["f32", "bf16"])
@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8", "nvfp4"])
def test_quantize_fp_bit_exact(ops, mode, wdt):
    rng = np.random.default_rng(3)
    wf = (rng.standard_normal((24, 512)) * 0.02).astype(np.float32)
    wf[1, :32] = 0.0
    wf[2, :32] *= 1e6
    wn = oracle.from_float(wf, wdt)
    tq, ts, tb = ops.quantize(from_np(wn, wdt), mode=mode)
    rq, rs = oracle.fp_quantize(wn, wdt, mode)
    assert tb is None
    assert np.array_equal(words_to_np(tq), rq)
    assert np.array_equal(ts.cpu().numpy(), rs)


# ------------------------------------------------------------------ quantized_matmul
def _qmm_case(ops, rng, M, N, K, xdt, mode="affine", bits=4, gs=64, transpose=True):
    rows, cols = (N, K) if transpose else (K, N)
    sdt = xdt
    if mode == "affine":
        w, s, b = rand_affine(rng, rows, cols, gs, bits, sdt)
        ts, tb = from_np(s, sdt), from_np(b, sdt)
    else:
        w, s = rand_fp(rng, rows, cols, mode)
        b, sdt = None, None
        ts, tb = torch.from_numpy(s).cuda(), None
    x = oracle.from_float(rng.standard_normal((M, K)).astype(np.float32), xdt)
    got = ops.quantized_matmul(from_np(x, xdt), words_to_torch(w), ts, tb, transpose,
                               None if mode != "affine" else gs,
                               None if mode != "affine" else bits, mode)
    ref = oracle.qmm(x, xdt, w, s, b, sdt or "f32", transpose, gs if mode == "affine" else None,
                     bits if mode == "affine" else None, mode, odt="f32")
    assert tuple(got.shape) == (M, N) and got.dtype == TDT[xdt]
    return as_f64(to_np(got, xdt), xdt), ref.astype(np.float64)


@pytest.mark.parametrize("xdt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("M", [1, 3, 8, 17, 130])
def test_qmm_affine4_gs64(ops, M, xdt):
    rng = np.random.default_rng(M)
    got, ref = _qmm_case(ops, rng, M, 320, 1024, xdt)
    assert rel_err(got, ref) <= TOL[xdt]


@pytest.mark.parametrize("M", [1, 5, 64])
@pytest.mark.parametrize("bits", [2, 3, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 128])
def test_qmm_affine_bits(ops, bits, gs, M):
    rng = np.random.default_rng(bits * 7 + gs + M)
    got, ref = _qmm_case(ops, rng, M, 192, 512, "bf16", bits=bits, gs=gs)
    assert rel_err(got, ref) <= TOL["bf16"]


@pytest.mark.parametrize("xdt", ["bf16", "f16"])
@pytest.mark.parametrize("M", [1, 4, 40])
@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8", "nvfp4"])
def test_qmm_fp_modes(ops, mode, M, xdt):
    rng = np.random.default_rng(M + 11)
    got, ref = _qmm_case(ops, rng, M, 256, 512, xdt, mode=mode)
    assert rel_err(got, ref) <= TOL_FP[xdt]


@pytest.mark.parametrize("xdt", ["bf16", "f16"])
@pytest.mark.parametrize("K", [1024, 4096, 14336])
@pytest.mark.parametrize("mode", ["mxfp4", "nvfp4"])
def test_qmv_fp4_gemv(ops, mode, K, xdt):
    # M = 1 fp4 GEMV: e2m1 codes through the byte-table unpack, one (MX) or
    # two (NV) byte scales per 32-code chunk
    rng = np.random.default_rng(K + len(mode))
    got, ref = _qmm_case(ops, rng, 1, 300, K, xdt, mode=mode)
    assert rel_err(got, ref) <= TOL_FP[xdt]


@pytest.mark.parametrize("xdt", ["bf16", "f16"])
@pytest.mark.parametrize("M", [128, 256])
@pytest.mark.parametrize("mode,bits,gs", [("affine", 4, 64), ("affine", 8, 32), ("mxfp4", 4, 32),
                                          ("nvfp4", 4, 16), ("mxfp8", 8, 32)])
def test_qmm_split_k_tiles(ops, mode, bits, gs, M, xdt):
    # few output tiles (M <= 256, N = 1024): 128 x 128 tiles with K split
    # over workgroups, fp32 partials summed in a second pass
    rng = np.random.default_rng(M + bits + gs)
    got, ref = _qmm_case(ops, rng, M, 1024, 4096, xdt, mode=mode, bits=bits, gs=gs)
    tol = TOL if mode == "affine" else TOL_FP
    assert rel_err(got, ref) <= tol[xdt]


@pytest.mark.parametrize("mode,bits,gs,xdt", [("affine", 4, 64, "bf16"), ("affine", 4, 128, "f16"),
                                               ("affine", 8, 32, "bf16"), ("affine", 3, 64, "bf16"),
                                               ("mxfp4", None, None, "bf16"), ("nvfp4", None, None, "f16"),
                                               ("mxfp8", None, None, "bf16")])
@pytest.mark.parametrize("M", [768, 512])
def test_qmm_big_tiles_split_k(ops, mode, bits, gs, xdt, M):
    # 96 (M = 768) or 64 (M = 512) output tiles of 256 x 256 over K = 8192:
    # two or four K ranges of the big tiles, fp32 partials summed in a second
    # pass.  Too large for the CPU oracle in seconds, so the reference is the
    # library's dequantize (bit exact against the oracle in the dequantize
    # tests) times x in fp32.
    N, K = 8192, 8192
    print(f"big-tile split-K {mode} bits={bits} gs={gs} {xdt} M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(11)
    dt = TDT[xdt]
    wf = (torch.randn((N, K), generator=g, device="cuda") * 0.02).to(dt)
    wq, s, b = ops.quantize(wf, gs, bits, mode)
    del wf
    x = torch.randn((M, K), generator=g, device="cuda").to(dt)
    got = ops.quantized_matmul(x, wq, s, b, True, gs, bits, mode).float()
    ref = x.float() @ ops.dequantize(wq, s, b, gs, bits, mode, dtype=dt).float().t()
    err = ((got - ref).abs().max() / ref.abs().max()).item()
    assert err <= (TOL if mode == "affine" else TOL_FP)[xdt]


@pytest.mark.parametrize("xdt", ["bf16", "f16"])
@pytest.mark.parametrize("N,K", [(200, 512), (6144, 1024), (8200, 1152)])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M", [4, 7, 8, 12, 16, 24, 32])
def test_qmm_decode_widths_affine4(ops, M, gs, N, K, xdt):
    # decode batch widths of the 4-bit path.  N = 8200 (ragged 32-row tile)
    # is wide enough for the factored MFMA kernel (M up to two 16-row m
    # tiles, K % 128 == 0; K = 1152 has an odd block count for
    # the split-K tail); N = 200 takes the split-K skinny kernel
    if N > 1000 and xdt == "f16" and M not in (8, 16):
        pytest.skip("f16 wide cases: M = 8, 16 cover the f16 magic constant")
    rng = np.random.default_rng(M * 1000 + gs + K)
    got, ref = _qmm_case(ops, rng, M, N, K, xdt, bits=4, gs=gs)
    assert rel_err(got, ref) <= TOL[xdt]


@pytest.mark.parametrize("xdt", ["bf16", "f16"])
@pytest.mark.parametrize("M,N,K", [(100, 320, 1024), (300, 512, 256), (257, 96, 640), (520, 256, 1536)])
@pytest.mark.parametrize("mode,bits,gs", [("affine", 4, 64), ("affine", 4, 32), ("affine", 4, 128),
                                          ("affine", 8, 64), ("affine", 3, 64), ("mxfp4", 4, 32),
                                          ("nvfp4", 4, 16), ("mxfp8", 8, 32)])
def test_qmm_prefill_tiles(ops, mode, bits, gs, M, N, K, xdt):
    # M > 64 takes the tiled GEMM; the K / group-count mix covers the
    # chunked-load kernel (K % 128 == 0, 8 or 16 groups per scale chunk) and
    # its fallbacks, ragged M and N edges, and K spans shorter than the ring
    rng = np.random.default_rng(M + N + K + bits + gs)
    got, ref = _qmm_case(ops, rng, M, N, K, xdt, mode=mode, bits=bits, gs=gs)
    tol = TOL if mode == "affine" else TOL_FP
    assert rel_err(got, ref) <= tol[xdt]


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("M", [1, 6, 100])
@pytest.mark.parametrize("mode,bits,gs", [("affine", 4, 64), ("affine", 3, 32),
                                          ("affine", 8, 128), ("nvfp4", 4, 16),
                                          ("mxfp8", 8, 32)])
def test_qmm_no_transpose(ops, mode, bits, gs, M, xdt):
    rng = np.random.default_rng(M + bits)
    got, ref = _qmm_case(ops, rng, M, 256, 384, xdt, mode=mode, bits=bits, gs=gs,
                         transpose=False)
    tol = TOL if mode == "affine" else TOL_FP
    assert rel_err(got, ref) <= tol[xdt]


def test_qmm_ragged_edges(ops):
    # N, M not multiples of any tile; K the minimum legal
    for (M, N, K) in [(1, 1, 32), (2, 3, 64), (129, 131, 96), (9, 257, 160)]:
        rng = np.random.default_rng(M * N)
        got, ref = _qmm_case(ops, rng, M, N, K, "bf16", gs=32)
        assert rel_err(got, ref) <= TOL["bf16"], (M, N, K)


def test_qmm_batched_weight_broadcast(ops):
    rng = np.random.default_rng(5)
    B, M, N, K = 3, 4, 64, 256
    w, s, b = rand_affine(rng, N, K, 64, 4, "bf16", lead=(B,))
    x = oracle.from_float(rng.standard_normal((2, 1, M, K)).astype(np.float32), "bf16")
    got = ops.quantized_matmul(from_np(x, "bf16"), words_to_torch(w), from_np(s, "bf16"),
                               from_np(b, "bf16"), True, 64, 4)
    assert tuple(got.shape) == (2, B, M, N)
    g = as_f64(to_np(got, "bf16"), "bf16")
    for i in range(2):
        for j in range(B):
            ref = oracle.qmm(x[i, 0], "bf16", w[j], s[j], b[j], "bf16", True, 64, 4, odt="f32")
            assert rel_err(g[i, j], ref) <= TOL["bf16"]


def test_qmm_leading_dims_fold(ops):
    rng = np.random.default_rng(6)
    w, s, b = rand_affine(rng, 96, 256, 64, 4, "f16")
    x = oracle.from_float(rng.standard_normal((2, 5, 256)).astype(np.float32), "f16")
    got = ops.quantized_matmul(from_np(x, "f16"), words_to_torch(w), from_np(s, "f16"),
                               from_np(b, "f16"))
    assert tuple(got.shape) == (2, 5, 96)
    ref = oracle.qmm(x.reshape(10, 256), "f16", w, s, b, "f16", True, 64, 4, odt="f32")
    assert rel_err(as_f64(to_np(got, "f16"), "f16").reshape(10, 96), ref) <= TOL["f16"]


def test_qmm_empty_and_zero_k(ops):
    rng = np.random.default_rng(0)
    w, s, b = rand_affine(rng, 64, 128, 64, 4, "bf16")
    x = torch.zeros((0, 128), dtype=torch.bfloat16, device="cuda")
    out = ops.quantized_matmul(x, words_to_torch(w), from_np(s, "bf16"), from_np(b, "bf16"))
    assert tuple(out.shape) == (0, 64)


def test_qmm_errors_raise(ops):
    from ironmlx_amd import IqmmError
    rng = np.random.default_rng(0)
    w, s, b = rand_affine(rng, 64, 128, 64, 4, "bf16")
    x = torch.zeros((1, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(IqmmError, match="Invalid quantization mode"):
        ops.quantized_matmul(x, words_to_torch(w), from_np(s, "bf16"), from_np(b, "bf16"),
                             mode="q4")
    with pytest.raises(IqmmError, match="GPU only"):
        ops.quantized_matmul(x.cpu(), words_to_torch(w), from_np(s, "bf16"), from_np(b, "bf16"))


# ------------------------------------------------------------------ gather_qmm
@pytest.mark.parametrize("sorted_idx", [False, True])
@pytest.mark.parametrize("M", [1, 3, 20])
def test_gather_qmm_vs_loop(ops, M, sorted_idx):
    rng = np.random.default_rng(M + 40)
    E, N, K, T, topk = 8, 64, 256, 6, 3
    w, s, b = rand_affine(rng, N, K, 64, 4, "bf16", lead=(E,))
    x = oracle.from_float(rng.standard_normal((T, 1, M, K)).astype(np.float32), "bf16")
    idx = np.stack([rng.choice(E, topk, replace=False) for _ in range(T)]).astype(np.int32)
    if sorted_idx:
        # the sorted form: rows flattened and ordered by expert
        flat = idx.reshape(-1)
        order = np.argsort(flat, kind="stable")
        xs = x.reshape(T, M, K)[order // topk]                # [T*topk, M, K]
        got = ops.gather_qmm(from_np(xs, "bf16"), words_to_torch(w), from_np(s, "bf16"),
                             from_np(b, "bf16"), None, torch.from_numpy(flat[order]).cuda(),
                             sorted_indices=True)
        assert tuple(got.shape) == (T * topk, M, N)
        g = as_f64(to_np(got, "bf16"), "bf16")
        for i, e in enumerate(flat[order]):
            ref = oracle.qmm(xs[i], "bf16", w[e], s[e], b[e], "bf16", True, 64, 4, odt="f32")
            assert rel_err(g[i], ref) <= TOL["bf16"]
    else:
        got = ops.gather_qmm(from_np(x, "bf16"), words_to_torch(w), from_np(s, "bf16"),
                             from_np(b, "bf16"), None, torch.from_numpy(idx).cuda())
        assert tuple(got.shape) == (T, topk, M, N)
        ref = oracle.gather_qmm(x.reshape(T, M, K), "bf16", w, s, b, "bf16",
                                np.broadcast_to(np.arange(T)[:, None], idx.shape), idx,
                                odt="f32")
        assert rel_err(as_f64(to_np(got, "bf16"), "bf16"), ref) <= TOL["bf16"]


def test_gather_qmm_lhs_and_out_of_range(ops):
    rng = np.random.default_rng(9)
    E, N, K, M = 4, 64, 128, 2
    w, s, b = rand_affine(rng, N, K, 32, 4, "f16", lead=(E,))
    x = oracle.from_float(rng.standard_normal((5, M, K)).astype(np.float32), "f16")
    lhs = np.array([0, 4, 2, 2], np.int64)
    rhs = np.array([3, 0, 9, 1], np.uint32)          # 9 is out of range
    got = ops.gather_qmm(from_np(x, "f16"), words_to_torch(w), from_np(s, "f16"),
                         from_np(b, "f16"), torch.from_numpy(lhs).cuda(),
                         torch.from_numpy(rhs.view(np.int32)).cuda().view(torch.uint32),
                         group_size=32)
    g = as_f64(to_np(got, "f16"), "f16")
    for i in range(4):
        if rhs[i] >= E:
            assert np.all(np.isnan(g[i]))
        else:
            ref = oracle.qmm(x[lhs[i]], "f16", w[rhs[i]], s[rhs[i]], b[rhs[i]], "f16", True,
                             32, 4, odt="f32")
            assert rel_err(g[i], ref) <= TOL["f16"]


def test_gather_qmm_sorted_with_lhs_and_invalid(ops):
    """Sorted grouped path: explicit lhs indices, ragged expert counts, an
    unused expert and an out-of-range expert index (rows of NaN)."""
    rng = np.random.default_rng(21)
    E, N, K, M = 6, 48, 256, 1
    w, s, b = rand_affine(rng, N, K, 64, 4, "bf16", lead=(E,))
    x = oracle.from_float(rng.standard_normal((7, M, K)).astype(np.float32), "bf16")
    rhs = np.array([0, 0, 0, 2, 2, 3, 5, 5, 5, 5, 6], np.int32)      # 6 is out of range; 1, 4 unused
    lhs = np.array([1, 3, 6, 0, 0, 2, 4, 5, 6, 1, 2], np.int32)
    got = ops.gather_qmm(from_np(x, "bf16"), words_to_torch(w), from_np(s, "bf16"),
                         from_np(b, "bf16"), torch.from_numpy(lhs).cuda(),
                         torch.from_numpy(rhs).cuda(), sorted_indices=True)
    g = as_f64(to_np(got, "bf16"), "bf16")
    assert g.shape == (11, M, N)
    for i in range(11):
        if rhs[i] >= E:
            assert np.all(np.isnan(g[i]))
            continue
        ref = oracle.qmm(x[lhs[i]], "bf16", w[rhs[i]], s[rhs[i]], b[rhs[i]], "bf16", True, 64, 4,
                         odt="f32")
        assert rel_err(g[i], ref) <= TOL["bf16"]


@pytest.mark.parametrize("xdt", ["bf16", "f16"])
@pytest.mark.parametrize("M", [1, 2])
def test_gather_qmm_sorted_few_rows(ops, M, xdt):
    """Sorted grouped gather at K = 2048 with few rows per expert: ragged
    segments (1..4 batch elements of M x rows), unused experts, an
    out-of-range expert (NaN rows) and an out-of-range lhs x index (NaN row)."""
    rng = np.random.default_rng(31 + M)
    E, N, K = 6, 130, 2048
    w, s, b = rand_affine(rng, N, K, 64, 4, xdt, lead=(E,))
    x = oracle.from_float(rng.standard_normal((7, M, K)).astype(np.float32), xdt)
    rhs = np.array([0, 0, 0, 2, 2, 3, 5, 5, 5, 5, 6], np.int32)      # 6 is out of range; 1, 4 unused
    lhs = np.array([1, 3, 6, 0, 9, 2, 4, 5, 6, 1, 2], np.int32)      # 9: x index out of range
    got = ops.gather_qmm(from_np(x, xdt), words_to_torch(w), from_np(s, xdt),
                         from_np(b, xdt), torch.from_numpy(lhs).cuda(),
                         torch.from_numpy(rhs).cuda(), sorted_indices=True)
    g = as_f64(to_np(got, xdt), xdt)
    assert g.shape == (11, M, N)
    for i in range(11):
        if rhs[i] >= E or lhs[i] >= 7:
            assert np.all(np.isnan(g[i]))
            continue
        ref = oracle.qmm(x[lhs[i]], xdt, w[rhs[i]], s[rhs[i]], b[rhs[i]], xdt, True, 64, 4,
                         odt="f32")
        assert rel_err(g[i], ref) <= TOL[xdt]


@pytest.mark.parametrize("mode", ["affine", "nvfp4"])
def test_gather_qmm_sorted_many_rows_per_expert(ops, mode):
    """More than 32 rows on one expert exercises the m-tile loop."""
    rng = np.random.default_rng(22)
    E, N, K = 3, 40, 512
    if mode == "affine":
        w, s, b = rand_affine(rng, N, K, 64, 4, "f16", lead=(E,))
        ts, tb = from_np(s, "f16"), from_np(b, "f16")
    else:
        w, s = rand_fp(rng, N, K, mode, lead=(E,))
        b = None
        ts, tb = torch.from_numpy(s).cuda(), None
    rhs = np.sort(rng.integers(0, E, 90)).astype(np.int64)
    rhs[:50] = 1
    rhs = np.sort(rhs)
    x = oracle.from_float(rng.standard_normal((90, 1, K)).astype(np.float32), "f16")
    got = ops.gather_qmm(from_np(x, "f16"), words_to_torch(w), ts, tb, None,
                         torch.from_numpy(rhs).cuda(), mode=mode, sorted_indices=True)
    g = as_f64(to_np(got, "f16"), "f16")
    for i in range(90):
        e = rhs[i]
        ref = oracle.qmm(x[i], "f16", w[e], s[e], None if b is None else b[e], "f16" if b is not None else None,
                         True, None if mode != "affine" else 64, None if mode != "affine" else 4, mode,
                         odt="f32")
        assert rel_err(g[i], ref) <= (TOL if mode == "affine" else TOL_FP)["f16"]


# ------------------------------------------------------------------ 8-bit M = 1 GEMV
@pytest.mark.parametrize("xdt", ["bf16", "f16"])
@pytest.mark.parametrize("mode,gs", [("affine", 32), ("affine", 64), ("affine", 128), ("mxfp8", 32)])
@pytest.mark.parametrize("N,K", [(300, 1024), (4100, 4096), (97, 3072), (2048, 8192), (64, 1056)])
def test_qmv_8bit_gemv(ops, xdt, mode, gs, N, K):
    """qmv_q8_kernel: affine 8-bit and mxfp8 at M = 1 (16-code half chunks per
    lane; partial last slots when K / 16 is not a multiple of 64)."""
    if K % gs:
        pytest.skip("K not a multiple of the group size")
    print(f"q8 gemv {mode} gs{gs} {xdt} N={N} K={K}", flush=True)
    rng = np.random.default_rng(N + K + gs)
    if mode == "affine":
        w, s, b = rand_affine(rng, N, K, gs, 8, xdt)
        ts, tb = from_np(s, xdt), from_np(b, xdt)
    else:
        w, s = rand_fp(rng, N, K, mode)
        ts, tb, b = torch.from_numpy(s).cuda(), None, None
    x = oracle.from_float(rng.standard_normal((1, K)).astype(np.float32), xdt)
    got = ops.quantized_matmul(from_np(x, xdt), words_to_torch(w), ts, tb, True,
                               gs if mode == "affine" else None, 8 if mode == "affine" else None, mode)
    ref = oracle.qmm(x, xdt, w, s, b, xdt if mode == "affine" else "f32", True,
                     gs if mode == "affine" else None, 8 if mode == "affine" else None, mode)
    tol = TOL if mode == "affine" else TOL_FP
    assert rel_err(as_f64(to_np(got, xdt), xdt), as_f64(ref, xdt)) <= tol[xdt]


def test_qmv_mxfp8_nan_code(ops):
    """An e4m3 NaN code (S.1111.111) makes its row NaN, as the dequantized
    weight is NaN; other rows are unaffected."""
    rng = np.random.default_rng(3)
    N, K = 8, 2048
    w, s = rand_fp(rng, N, K, "mxfp8")
    w = w.copy()
    w[5, 100] = (w[5, 100] & ~np.uint32(0xff)) | np.uint32(0x7f)
    x = oracle.from_float(rng.standard_normal((1, K)).astype(np.float32), "bf16")
    got = ops.quantized_matmul(from_np(x, "bf16"), words_to_torch(w), torch.from_numpy(s).cuda(), None, True,
                               mode="mxfp8").float().cpu().numpy()
    assert np.isnan(got[0, 5]) and not np.isnan(np.delete(got[0], 5)).any()


def _misaligned(t):
    """a copy of t whose data pointer is 2 bytes past an 8-byte boundary"""
    flat = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)[1:]
    out = flat.view(t.shape)
    out.copy_(t)
    assert out.data_ptr() % 8 != 0
    return out


@pytest.mark.parametrize("gs", [32, 64])
def test_decode_width_and_gather_misaligned_scales(ops, gs):
    # the chunk-major decode-width, skinny and grouped-gather kernels read a block's
    # group scales / biases as one 4- / 8-byte word; scale arrays that are not
    # 8-byte aligned take the per-group kernels and give the same results
    # within the matmul tolerance
    rng = np.random.default_rng(gs)
    # factored kernel (8200 rows) and split-K skinny kernel (200 rows)
    for N, K, M in ((8200, 1152, 16), (200, 512, 8)):
        w, s, b = rand_affine(rng, N, K, gs, 4, "bf16")
        tw, ts, tb = words_to_torch(w), from_np(s, "bf16"), from_np(b, "bf16")
        x = from_np(oracle.from_float(rng.standard_normal((M, K)).astype(np.float32), "bf16"), "bf16")
        got = ops.quantized_matmul(x, tw, _misaligned(ts), _misaligned(tb), True, gs, 4)
        ref = ops.quantized_matmul(x, tw, ts, tb, True, gs, 4)
        assert rel_err(as_f64(to_np(got, "bf16"), "bf16"), as_f64(to_np(ref, "bf16"), "bf16")) <= TOL["bf16"]
    # grouped gather: 4 experts, 40 rows each
    E, n, k2 = 4, 256, 1024
    ws = [rand_affine(rng, n, k2, gs, 4, "bf16") for _ in range(E)]
    tw2 = torch.stack([words_to_torch(u[0]) for u in ws])
    ts2 = torch.stack([from_np(u[1], "bf16") for u in ws])
    tb2 = torch.stack([from_np(u[2], "bf16") for u in ws])
    xg = from_np(oracle.from_float(rng.standard_normal((E * 40, 1, k2)).astype(np.float32), "bf16"), "bf16")
    rhs = torch.arange(E, device="cuda", dtype=torch.int32).repeat_interleave(40)
    g1 = ops.gather_qmm(xg, tw2, _misaligned(ts2), _misaligned(tb2), None, rhs, True, gs, 4, "affine", True)
    g0 = ops.gather_qmm(xg, tw2, ts2, tb2, None, rhs, True, gs, 4, "affine", True)
    assert rel_err(as_f64(to_np(g1, "bf16"), "bf16"), as_f64(to_np(g0, "bf16"), "bf16")) <= TOL["bf16"]


# ------------------------------------------------------------------ mixed dtypes
@pytest.mark.parametrize("xdt,sdt", [("f32", "bf16"), ("f32", "f16"), ("f16", "bf16"), ("bf16", "f16"),
                                     ("bf16", "f32")])
@pytest.mark.parametrize("M", [1, 5, 70])
def test_mixed_dtype_promotes_to_f32(ops, xdt, sdt, M):
    """MLX casts x, scales and biases to their promoted type (float32 for any
    mixed pair) before the product (mlx/src/nn/linear.rs:51-63 passes x in
    whatever type the model produces).  The result is float32 and equals the
    oracle's float32 product of the exactly upcast operands."""
    print(f"mixed x={xdt} scales={sdt} M={M}", flush=True)
    rng = np.random.default_rng(M + len(xdt) * 7 + len(sdt))
    N, K = 96, 512
    w, s, b = rand_affine(rng, N, K, 64, 4, sdt)
    x = oracle.from_float(rng.standard_normal((M, K)).astype(np.float32), xdt)
    got = ops.quantized_matmul(from_np(x, xdt), words_to_torch(w), from_np(s, sdt), from_np(b, sdt),
                               True, 64, 4)
    assert got.dtype == torch.float32
    up = lambda a, dt: oracle.to_float(a, dt).astype(np.float32)  # noqa: E731
    ref = oracle.qmm(up(x, xdt), "f32", w, up(s, sdt), up(b, sdt), "f32", True, 64, 4, odt="f32")
    assert rel_err(got.cpu().numpy(), ref) <= 1e-5


def test_mixed_dtype_gather_and_swiglu(ops):
    """gather_qmm and the fused SwiGLU follow the same promotion."""
    rng = np.random.default_rng(5)
    E, N, K, T = 4, 64, 256, 6
    w, s, b = rand_affine(rng, N * E, K, 64, 4, "bf16")
    wt, st, bt = (words_to_torch(w).view(E, N, -1), from_np(s, "bf16").view(E, N, -1),
                  from_np(b, "bf16").view(E, N, -1))
    x = rng.standard_normal((T, 1, K)).astype(np.float32)
    idx = torch.tensor([3, 0, 1, 1, 2, 0], dtype=torch.int32, device="cuda")
    got = ops.gather_qmm(torch.from_numpy(x).cuda(), wt, st, bt, None, idx)
    assert got.dtype == torch.float32
    up = lambda a: oracle.to_float(a, "bf16").astype(np.float32)  # noqa: E731
    wn, sn, bn = w.reshape(E, N, -1), s.reshape(E, N, -1), b.reshape(E, N, -1)
    for i, e in enumerate(idx.tolist()):
        ref = oracle.qmm(x[i], "f32", wn[e], up(sn[e]), up(bn[e]), "f32", True, 64, 4, odt="f32")
        assert rel_err(got[i].cpu().numpy(), ref) <= 1e-5
    # SwiGLU over [2I, K]: f32 x with bf16 scales gives float32 silu(gate) * up
    gu = ops.quantized_swiglu(torch.from_numpy(x[:, 0]).cuda(), words_to_torch(w[:2 * N]),
                              from_np(s[:2 * N], "bf16"), from_np(b[:2 * N], "bf16"), 64, 4)
    assert gu.dtype == torch.float32
    prod = oracle.qmm(x[:, 0], "f32", w[:2 * N], up(s[:2 * N]), up(b[:2 * N]), "f32", True, 64, 4, odt="f32")
    ref = oracle.swiglu(prod, "f32").astype(np.float64)
    assert rel_err(gu.cpu().numpy(), ref) <= 1e-5
