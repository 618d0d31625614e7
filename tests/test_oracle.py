"""Pins the CPU oracle (oracle/iqmm_oracle.c) before it is trusted as the
parity checker.  Every check here uses an independent implementation or a
closed form: numpy/torch float decoders and encoders, numpy's little-endian
packbits, float64 matmul of the dequantized weight, hand-derived known
answers, and invariants of the quantizer.  No GPU needed.

Reference surface: mlx/src/ops.rs:653-727 (dequantize, quantized_matmul).
The reference holds no golden vectors for this path (no test touches the
quantized ops), so the committed fixtures in tests/golden/ are the
known-answer vectors written by tests/golden/make_golden.py.
"""
import json
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ----------------------------------------------------------------- conversions
def test_half_decode_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = oracle.to_float(bits.view(np.float16), "f16")
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _float_probe(n=20000, seed=0):
    rng = np.random.default_rng(seed)
    v = np.concatenate([
        rng.standard_normal(n).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, n),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, 2 ** -24, 2 ** -25,
                  3 * 2 ** -26, 2 ** -14, 6.1e-5, np.inf, -np.inf, 1.0009765625,
                  1 + 2 ** -11, 1 + 3 * 2 ** -11, 448, 464, 3.3895e38], np.float32),
    ])
    # ties in the fp16 / bf16 grids: midpoints between neighbouring values
    h = rng.integers(0, 0x7bff, 2000).astype(np.uint16).view(np.float16).astype(np.float64)
    h2 = np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    v = np.concatenate([v, ((h + h2) / 2).astype(np.float32)])
    b = rng.integers(0, 0x7f7f, 2000).astype(np.uint32) << 16
    v = np.concatenate([v, (b | 0x8000).view(np.float32), (b | 0x18000).view(np.float32)])
    return v


def test_half_encode_rne():
    v = _float_probe()
    got = oracle.from_float(v, "f16").view(np.uint16)
    with np.errstate(over="ignore"):  # the probe holds values past fp16's range (-> inf)
        ref = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_roundtrip_vs_torch():
    v = _float_probe(seed=1)
    got = oracle.from_float(v, "bf16")
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    dec = oracle.to_float(allbits, "bf16")
    tdec = torch.from_numpy(allbits.view(np.int16)).view(torch.bfloat16).float().numpy()
    nan = np.isnan(tdec)
    assert np.array_equal(np.isnan(dec), nan)
    assert np.array_equal(dec[~nan], tdec[~nan])


def test_e4m3_decode_all_codes_vs_torch():
    L = oracle.lib()
    codes = np.arange(256, dtype=np.uint8)
    got = np.array([L.iqo_e4m3_to_float(int(c)) for c in codes], np.float32)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert nan.sum() == 2 and np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], ref[~nan])
    assert got[0x7e] == 448.0 and got[1] == 2.0 ** -9


def test_e4m3_encode_vs_torch_in_range():
    L = oracle.lib()
    rng = np.random.default_rng(2)
    v = (rng.standard_normal(20000) * 10.0 ** rng.integers(-3, 3, 20000)).astype(np.float32)
    v = v[np.abs(v) <= 448]
    grid = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    mids = ((grid[:126].astype(np.float64) + grid[1:127]) / 2).astype(np.float32)
    v = np.concatenate([v, mids, -mids])
    got = np.array([L.iqo_float_to_e4m3(float(x)) for x in v], np.uint8)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    # torch encodes tiny negatives that round to zero as -0 (0x80); the oracle
    # writes +0 for every zero result.  Same value; compare decoded values.
    gv = torch.from_numpy(got).view(torch.float8_e4m3fn).float().numpy()
    rv = torch.from_numpy(ref).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(gv, rv)
    # saturation (the oracle's choice: clamp to +-448)
    assert L.iqo_float_to_e4m3(1000.0) == 0x7E and L.iqo_float_to_e4m3(-1e30) == 0xFE


E2M1 = [0, 0.5, 1, 1.5, 2, 3, 4, 6]   # OCP MX v1.0, table of FP4 E2M1 values


def test_e2m1_table_and_rne():
    L = oracle.lib()
    for c in range(16):
        ref = E2M1[c & 7] * (-1 if c & 8 else 1)
        assert L.iqo_e2m1_to_float(c) == ref
    # midpoint ties go to the even code, beyond-max saturates
    cases = {0.25: 0, 0.75: 2, 1.25: 2, 1.75: 4, 2.5: 4, 3.5: 6, 5.0: 6, 7.0: 7, 100.0: 7,
             -0.75: 0xA, -5.0: 0xE, 0.26: 1, 0.2: 0}
    for v, c in cases.items():
        assert L.iqo_float_to_e2m1(v) == c, v


def test_e8m0_all_codes():
    L = oracle.lib()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e8m0fnu).float().numpy()
    for c in range(256):
        g = L.iqo_e8m0_to_float(c)
        if c == 255:
            assert np.isnan(g) and np.isnan(ref[c])
        else:
            assert g == 2.0 ** (c - 127) == ref[c]


# ----------------------------------------------------------------- packing
def _packbits_ref(codes, bits):
    """Independent little-endian bit-stream builder via numpy.packbits."""
    rows, K = codes.shape
    b = ((codes[..., None] >> np.arange(bits)) & 1).astype(np.uint8).reshape(rows, K * bits)
    by = np.packbits(b, axis=1, bitorder="little")
    return by.view("<u4")


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_pack_vs_packbits_and_roundtrip(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, (7, 256)).astype(np.uint32)
    w = oracle.pack(codes, bits)
    assert np.array_equal(w, _packbits_ref(codes, bits))
    assert np.array_equal(oracle.unpack(w, 256, bits), codes)


def test_pack_known_answers():
    assert oracle.pack(np.arange(8).reshape(1, 8), 4)[0, 0] == 0x76543210
    assert oracle.pack(np.array([[1, 2, 3, 4]]), 8)[0, 0] == 0x04030201
    assert oracle.pack(np.array([[3, 2, 1, 0] * 4]), 2)[0, 0] == 0x1B1B1B1B
    # 3-bit: codes 0..7 repeated -> 24-bit pattern 0xFAC688 every 3 bytes
    w = oracle.pack(np.tile(np.arange(8), 4).reshape(1, 32), 3)
    assert list(w[0]) == [0x88FAC688, 0xC688FAC6, 0xFAC688FA]


# ----------------------------------------------------------------- dequantize
def _rand_affine(rows, K, gs, bits, sdt, seed):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 1 << bits, (rows, K)).astype(np.uint32)
    s = (rng.standard_normal((rows, K // gs)) * 0.01).astype(np.float32)
    b = (rng.standard_normal((rows, K // gs)) * 0.05).astype(np.float32)
    return codes, oracle.from_float(s, sdt), oracle.from_float(b, sdt)


@pytest.mark.parametrize("sdt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("bits,gs", [(2, 32), (3, 64), (4, 64), (5, 128), (6, 32), (8, 128)])
def test_dequantize_affine_closed_form(bits, gs, sdt):
    rows, K = 5, 256
    codes, s, b = _rand_affine(rows, K, gs, bits, sdt, bits * 7 + gs)
    w = oracle.pack(codes, bits)
    got = oracle.dequantize(w, s, b, sdt, gs, bits)
    s64 = np.repeat(oracle.to_float(s, sdt).astype(np.float64), gs, axis=1)
    b64 = np.repeat(oracle.to_float(b, sdt).astype(np.float64), gs, axis=1)
    # fp32(s*q) then fp32(+b) then the output dtype
    ref32 = ((s64 * codes).astype(np.float32).astype(np.float64) + b64).astype(np.float32)
    ref = ref32 if sdt == "f32" else oracle.from_float(ref32, sdt)
    assert np.array_equal(np.asarray(got).view(np.uint8), np.asarray(ref).view(np.uint8))


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8", "nvfp4"])
def test_dequantize_fp_closed_form(mode):
    gs, bits = oracle.defaults(mode)
    rng = np.random.default_rng(5)
    rows, K = 4, 256
    ncode = 256 if bits == 8 else 16
    codes = rng.integers(0, ncode, (rows, K)).astype(np.uint32)
    if mode == "mxfp8":
        codes[(codes & 0x7F) == 0x7F] = 0   # keep NaN codes out of the product test
    sc = rng.integers(100, 150, (rows, K // gs)).astype(np.uint8)
    w = oracle.pack(codes, bits)
    got = oracle.dequantize(w, sc, None, None, gs, bits, mode, odt="f32")
    if mode == "mxfp8":
        elem = torch.from_numpy(codes.astype(np.uint8)).view(torch.float8_e4m3fn).float().numpy()
    else:
        elem = np.array([E2M1[c & 7] * (-1 if c & 8 else 1) for c in codes.reshape(-1)],
                        np.float64).reshape(rows, K)
    if mode == "nvfp4":
        scale = torch.from_numpy(sc).view(torch.float8_e4m3fn).float().numpy()
    else:
        scale = 2.0 ** (sc.astype(np.float64) - 127)
    ref = (elem * np.repeat(scale, gs, axis=1)).astype(np.float32)
    assert np.array_equal(got, ref)
    # default output dtype of the fp modes is bf16, exact for these products
    got_bf = oracle.dequantize(w, sc, None, None, gs, bits, mode)
    assert np.array_equal(oracle.to_float(got_bf, "bf16"), ref)


# ----------------------------------------------------------------- matmul
@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("mode,bits,gs", [("affine", 4, 64), ("affine", 3, 32),
                                          ("affine", 8, 128), ("mxfp8", 8, 32),
                                          ("nvfp4", 4, 16), ("mxfp4", 4, 32)])
def test_qmm_vs_float64_matmul(mode, bits, gs, transpose):
    rng = np.random.default_rng(11)
    M, K, N = 3, 256, 96
    rows, cols = (N, K) if transpose else (K, N)
    if mode == "affine":
        codes, s, b = _rand_affine(rows, cols, gs, bits, "f32", 3)
        sdt = "f32"
    else:
        codes = rng.integers(0, 1 << bits, (rows, cols)).astype(np.uint32)
        if mode == "mxfp8":
            codes[(codes & 0x7F) == 0x7F] = 0
        lo, hi = (0x30, 0x50) if mode == "nvfp4" else (120, 130)   # no NaN scale codes
        s = rng.integers(lo, hi, (rows, cols // gs)).astype(np.uint8)
        b, sdt = None, None
    w = oracle.pack(codes, bits)
    x = rng.standard_normal((M, K)).astype(np.float32)
    wd = oracle.dequantize(w, s, b, sdt or "f32", gs, bits, mode, odt="f32").astype(np.float64)
    ref = x.astype(np.float64) @ (wd.T if transpose else wd)
    got = oracle.qmm(x, "f32", w, s, b, sdt or "f32", transpose, gs, bits, mode)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_qmm_special_cases():
    rng = np.random.default_rng(12)
    N, K = 40, 128
    # bits=8, s=1, b=0 is an integer GEMM
    codes = rng.integers(0, 256, (N, K)).astype(np.uint32)
    w = oracle.pack(codes, 8)
    ones = np.ones((N, K // 64), np.float32)
    zeros = np.zeros_like(ones)
    xi = rng.integers(-5, 6, (2, K)).astype(np.float32)
    got = oracle.qmm(xi, "f32", w, ones, zeros, "f32", True, 64, 8)
    assert np.array_equal(got, (xi.astype(np.int64) @ codes.T.astype(np.int64)).astype(np.float32))
    # one-hot x selects a dequantized column of w^T (a row of w)
    codes4, s, b = _rand_affine(N, K, 32, 4, "f16", 9)
    w4 = oracle.pack(codes4, 4)
    x = np.zeros((1, K), np.float32)
    x[0, 77] = 1.0
    got = oracle.qmm(x, "f32", w4, s, b, "f16", True, 32, 4)
    deq = oracle.dequantize(w4, s, b, "f16", 32, 4, odt="f32")
    assert np.array_equal(got[0], deq[:, 77])
    # qmv streaming form agrees with the dequantize-then-dot form
    x16 = oracle.from_float(rng.standard_normal((2, K)).astype(np.float32), "f16")
    a = oracle.qmm(x16, "f16", w4, s, b, "f16", True, 32, 4, odt="f32")
    c = oracle.qmv_affine(x16, "f16", w4, s, b, "f16", 32, 4, odt="f32")
    assert np.max(np.abs(a - c)) <= 1e-5 * np.max(np.abs(a))


def test_gather_qmm_is_loop_of_qmm():
    rng = np.random.default_rng(13)
    E, N, K, M = 4, 32, 128, 2
    ws, ss, bs = [], [], []
    for e in range(E):
        c, s, b = _rand_affine(N, K, 64, 4, "bf16", 20 + e)
        ws.append(oracle.pack(c, 4)); ss.append(s); bs.append(b)
    w, s, b = np.stack(ws), np.stack(ss), np.stack(bs)
    x = oracle.from_float(rng.standard_normal((3, M, K)).astype(np.float32), "bf16")
    lhs = np.array([[0, 2], [1, 1]])
    rhs = np.array([[3, 0], [2, 3]])
    out = oracle.gather_qmm(x, "bf16", w, s, b, "bf16", lhs, rhs, odt="f32")
    assert out.shape == (2, 2, M, N)
    xf = oracle.to_float(x, "bf16").astype(np.float64)
    for i in range(2):
        for j in range(2):
            wd = oracle.dequantize(w[rhs[i, j]], s[rhs[i, j]], b[rhs[i, j]], "bf16", 64, 4,
                                   odt="f32").astype(np.float64)
            ref = xf[lhs[i, j]] @ wd.T
            assert np.max(np.abs(out[i, j] - ref)) <= 1e-5 * np.max(np.abs(ref))


# ----------------------------------------------------------------- quantize
def test_affine_quantize_known_answer():
    # 32 values on [-1, 2]: |min| < |max| so the scale is negative and the
    # edge is max=2: scale = -(3/15) -> q0 = rint(2/-0.2) = -10 -> scale =
    # 2/-10 = -0.2, bias = 2; q = rint((w-2)/-0.2)
    w = np.linspace(-1, 2, 32).astype(np.float32).reshape(1, 32)
    wq, s, b = oracle.affine_quantize(w, "f32", 32, 4)
    assert s[0, 0] == np.float32(2.0) / np.float32(-10.0) and b[0, 0] == 2.0
    exp = [int(np.rint(float((Fraction(float(v)) - 2) / Fraction(-1, 5)))) for v in w[0]]
    assert list(oracle.unpack(wq, 32, 4)[0]) == [min(max(e, 0), 15) for e in exp]


@pytest.mark.parametrize("bits,gs", [(2, 32), (3, 64), (4, 64), (6, 128), (8, 32)])
def test_affine_quantize_invariants(bits, gs):
    rng = np.random.default_rng(bits + gs)
    w = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
    wq, s, b = oracle.affine_quantize(w, "f32", gs, bits)
    codes = oracle.unpack(wq, 512, bits)
    assert codes.max() <= (1 << bits) - 1
    deq = oracle.dequantize(wq, s, b, "f32", gs, bits)
    err = np.abs(deq - w)
    step = np.repeat(np.abs(s), gs, axis=1)
    # interior codes are the nearest grid point; the edge snap (scale=edge/q0)
    # can leave the far extreme up to one more half step outside the grid,
    # where the code clips to 0 or 2^bits-1
    interior = (codes > 0) & (codes < (1 << bits) - 1)
    assert np.all(err[interior] <= step[interior] * 0.5 * (1 + 1e-5) + 1e-9)
    assert np.all(err <= step * (1 + 1e-5) + 1e-9)
    # the larger-magnitude edge of each group is reproduced exactly (q=0 -> bias)
    wg = w.reshape(16, -1, gs)
    edge = np.where(np.abs(wg.min(-1)) > np.abs(wg.max(-1)), wg.min(-1), wg.max(-1))
    assert np.array_equal(b, edge)


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8", "nvfp4"])
def test_fp_quantize_invariants(mode):
    gs, bits = oracle.defaults(mode)
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((8, 256)) * 0.02).astype(np.float32)
    wq, sc = oracle.fp_quantize(w, "f32", mode)
    deq = oracle.dequantize(wq, sc, None, None, gs, bits, mode, odt="f32")
    amax = np.abs(w.reshape(8, -1, gs)).max(-1)
    if mode == "nvfp4":
        scale = torch.from_numpy(sc).view(torch.float8_e4m3fn).float().numpy()
        # e4m3 block scale is amax/6 rounded to nearest
        assert np.all(np.abs(scale - amax / 6) <= 2.0 ** -4 * amax / 6 + 2 ** -9)
    else:
        scale = 2.0 ** (sc.astype(np.float64) - 127)
        emax = 8 if mode == "mxfp8" else 2
        assert np.array_equal(np.floor(np.log2(amax)) - emax, sc.astype(np.int64) - 127)
    # every element is the nearest point of the signed element grid (values
    # beyond the grid saturate to its end): brute force over the grid
    if mode == "mxfp8":
        grid = torch.arange(127, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    else:
        grid = np.array(E2M1, np.float64)
    grid = np.concatenate([grid, -grid])
    v = w.astype(np.float64) / np.repeat(scale, gs, axis=1)
    best = np.abs(v[..., None] - grid).min(-1)
    got = np.abs(v - deq / np.repeat(scale, gs, axis=1))
    assert np.allclose(got, best, rtol=0, atol=1e-6)


def test_golden_fixtures_match_oracle():
    """Known-answer vectors committed under tests/golden (written by
    tests/golden/make_golden.py from closed forms, not from the oracle)."""
    path = os.path.join(GOLDEN, "known_answers.json")
    with open(path) as f:
        g = json.load(f)
    for case in g["pack"]:
        codes = np.array(case["codes"], np.uint32).reshape(1, -1)
        assert [int(v) for v in oracle.pack(codes, case["bits"])[0]] == case["words"]
    for case in g["dequant_affine"]:
        w = np.array(case["words"], np.uint32).reshape(1, -1)
        s = np.array(case["scales_f16_bits"], np.uint16).view(np.float16).reshape(1, -1)
        b = np.array(case["biases_f16_bits"], np.uint16).view(np.float16).reshape(1, -1)
        out = oracle.dequantize(w, s, b, "f16", case["group_size"], case["bits"])
        assert [int(v) for v in out.view(np.uint16)[0]] == case["out_f16_bits"]
    for case in g["qmm"]:
        x = np.array(case["x"], np.float32).reshape(case["M"], -1)
        w = np.array(case["words"], np.uint32).reshape(case["N"], -1)
        s = np.array(case["scales"], np.float32).reshape(case["N"], -1)
        b = np.array(case["biases"], np.float32).reshape(case["N"], -1)
        out = oracle.qmm(x, "f32", w, s, b, "f32", True, case["group_size"], case["bits"])
        assert np.allclose(out, np.array(case["out"], np.float32).reshape(out.shape),
                           rtol=1e-6, atol=1e-6)
