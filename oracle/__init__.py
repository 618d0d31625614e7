"""CPU oracle for the quantized-matmul path — TEST INFRASTRUCTURE ONLY.

Python face of ``oracle/iqmm_oracle.c`` (the C restatement of MLX's
quantize / dequantize / quantized_matmul semantics; see that file's header for
the rules and the reference call sites it follows:
``mlx/src/ops.rs:653-727``, ``mlx/src/nn/moe.rs:55-183``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
package; the product (``ironmlx_amd``) never does.

Arrays are numpy.  Floating arrays carry a dtype tag: ``"f32"`` (float32),
``"f16"`` (float16) or ``"bf16"`` (raw bfloat16 bits held in uint16).

Parity status of each function (how it is pinned, see tests/test_oracle.py):
  * conversions (fp16/bf16/e4m3/e2m1/e8m0): pinned exhaustively against
    numpy/torch decoders and encoders (an independent implementation).
  * pack / unpack: pinned by hand-written known-answer words and by numpy's
    little-endian ``packbits`` (independent bit-stream builder).
  * dequantize: pinned by closed forms (s*q+b per element, e4m3*2^k tables)
    computed in float64 with numpy.
  * qmm / qmv: pinned by float64 numpy matmul of the dequantized weight and
    by special cases (one-hot x selects a row, bits=8 s=1 b=0 is an integer
    GEMM, constant scale factors out).
  * affine_quantize: pinned by a hand-derived known answer (sign/edge-snap
    rule) and invariants (code range, reconstruction error <= |scale|/2 for
    interior codes, exact larger-magnitude group edge).
  * fp_quantize: pinned by invariants (OCP shared-exponent rule, nvfp4
    block scale = RNE(amax/6), each element the nearest grid point by brute
    force).  MLX's own tie/eps/scale-selection choices for quantize are not
    verifiable without MLX: "parity unpinned" against MLX itself.
  * expf: pinned against float64 exp (<= 2 ulp over the float range) and
    exact points (exp(0) = 1, overflow / underflow edges).
  * swiglu: pinned by closed forms (g = 0 gives 0, saturated sigmoid gives
    rn(g * u), large negative g gives 0) and float64 silu(g)*u within the
    rounding of its three steps.  MLX's own sigmoid rounding: "parity
    unpinned" against MLX itself.
  * moe_route: pinned by float64 softmax + numpy stable argsort on
    well-separated logits (exact ids), tie cases (lower id first) and
    normalised scores summing to 1.
  * moe_sort: pinned by numpy stable argsort of the expert ids.
  * moe_combine: pinned by float64 weighted sums and the k = 1 identity.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libiqmm_oracle.so")

DT = {"f32": 0, "f16": 1, "bf16": 2}
MODES = {"affine": 0, "mxfp4": 1, "mxfp8": 2, "nvfp4": 3}
NP_STORAGE = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16}

_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with gcc (oracle/Makefile)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        L.iqo_bf16_to_float.restype = ctypes.c_float
        L.iqo_bf16_to_float.argtypes = [ctypes.c_uint16]
        L.iqo_float_to_bf16.restype = ctypes.c_uint16
        L.iqo_float_to_bf16.argtypes = [ctypes.c_float]
        L.iqo_half_to_float.restype = ctypes.c_float
        L.iqo_half_to_float.argtypes = [ctypes.c_uint16]
        L.iqo_float_to_half.restype = ctypes.c_uint16
        L.iqo_float_to_half.argtypes = [ctypes.c_float]
        for n in ("iqo_e4m3_to_float", "iqo_e2m1_to_float", "iqo_e8m0_to_float"):
            getattr(L, n).restype = ctypes.c_float
            getattr(L, n).argtypes = [ctypes.c_uint8]
        for n in ("iqo_float_to_e4m3", "iqo_float_to_e2m1"):
            getattr(L, n).restype = ctypes.c_uint8
            getattr(L, n).argtypes = [ctypes.c_float]
        L.iqo_pack.argtypes = [vp, i64, i64, i32, vp]
        L.iqo_unpack.argtypes = [vp, i64, i64, i32, vp]
        L.iqo_dequantize.argtypes = [vp, vp, vp, i32, i64, i64, i32, i32, i32, vp, i32]
        L.iqo_qmm.argtypes = [vp, i32, i64, i64, vp, vp, vp, i32, i64, i32, i32, i32, i32,
                              vp, i32, i32]
        L.iqo_qmv_affine.argtypes = [vp, i32, i64, i64, vp, vp, vp, i32, i64, i32, i32, vp,
                                     i32, i32]
        L.iqo_affine_quantize.argtypes = [vp, i32, i64, i64, i32, i32, vp, vp, vp, i32]
        L.iqo_fp_quantize.argtypes = [vp, i32, i64, i64, i32, vp, vp]
        L.iqo_from_float_array.argtypes = [vp, i64, i32, vp]
        L.iqo_to_float_array.argtypes = [vp, i64, i32, vp]
        L.iqo_expf.restype = ctypes.c_float
        L.iqo_expf.argtypes = [ctypes.c_float]
        L.iqo_swiglu.argtypes = [vp, i32, i64, i64, vp]
        L.iqo_moe_route.argtypes = [vp, i32, i64, i64, i32, i32, vp, vp]
        L.iqo_moe_sort.argtypes = [vp, i64, i32, i32, vp, vp, vp, vp]
        L.iqo_moe_combine.argtypes = [vp, i32, i64, vp, vp, vp, i64, i32, i32, vp]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ----------------------------------------------------------------- conversions
def to_float(a: np.ndarray, dt: str) -> np.ndarray:
    """Decode a tagged float array to float32 (via the oracle's decoder)."""
    if dt == "f32":
        return np.asarray(a, np.float32)
    src = np.ascontiguousarray(a).view(np.uint16)
    out = np.empty(src.shape, np.float32)
    lib().iqo_to_float_array(_p(src), src.size, DT[dt], _p(out))
    return out


def from_float(a: np.ndarray, dt: str) -> np.ndarray:
    """Round float32 values to a tagged float array (RNE, via the oracle)."""
    src = np.ascontiguousarray(a, np.float32)
    if dt == "f32":
        return src.copy()
    out = np.empty(src.shape, np.uint16)
    lib().iqo_from_float_array(_p(src), src.size, DT[dt], _p(out))
    return out.view(np.float16) if dt == "f16" else out


# ----------------------------------------------------------------- packing
def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    codes = _c(codes, np.uint32)
    rows, K = codes.shape
    out = np.zeros((rows, K * bits // 32), np.uint32)
    lib().iqo_pack(_p(codes), rows, K, bits, _p(out))
    return out


def unpack(w: np.ndarray, K: int, bits: int) -> np.ndarray:
    w = _c(w, np.uint32)
    rows = w.shape[0]
    out = np.zeros((rows, K), np.uint32)
    lib().iqo_unpack(_p(w), rows, K, bits, _p(out))
    return out


def defaults(mode: str, group_size=None, bits=None):
    """MLX's per-mode defaults (affine: gs64/4-bit; mxfp4: 32/4; mxfp8: 32/8;
    nvfp4: 16/4)."""
    d = {"affine": (64, 4), "mxfp4": (32, 4), "mxfp8": (32, 8), "nvfp4": (16, 4)}[mode]
    return (group_size or d[0], bits or d[1])


# ----------------------------------------------------------------- dequantize
def dequantize(w, scales, biases, sdt: str, group_size, bits, mode="affine", odt=None):
    """w [rows, K*bits/32] -> [rows, K] in odt (default: scales dtype for
    affine, bf16 for the fp modes)."""
    gs, bits = defaults(mode, group_size, bits)
    odt = odt or (sdt if mode == "affine" else "bf16")
    w = _c(w, np.uint32)
    rows = w.shape[0]
    K = w.shape[1] * 32 // bits
    sc = _c(scales, NP_STORAGE[sdt] if mode == "affine" else np.uint8)
    bi = _c(biases, NP_STORAGE[sdt]) if mode == "affine" else sc
    out = np.zeros((rows, K), NP_STORAGE[odt])
    lib().iqo_dequantize(_p(w), _p(sc), _p(bi), DT.get(sdt, 0), rows, K, gs, bits,
                         MODES[mode], _p(out), DT[odt])
    return out


# ----------------------------------------------------------------- matmul
def qmm(x, xdt, w, scales, biases, sdt, transpose=True, group_size=None, bits=None,
        mode="affine", odt=None, nthreads=0):
    """2-D quantized matmul; x [M,K] (tagged xdt) -> [M,N] in odt (default xdt)."""
    gs, bits = defaults(mode, group_size, bits)
    odt = odt or xdt
    x = _c(x, NP_STORAGE[xdt])
    M, K = x.shape
    w = _c(w, np.uint32)
    N = w.shape[0] if transpose else w.shape[1] * 32 // bits
    sc = _c(scales, NP_STORAGE[sdt] if mode == "affine" else np.uint8)
    bi = _c(biases, NP_STORAGE[sdt]) if mode == "affine" else sc
    out = np.zeros((M, N), NP_STORAGE[odt])
    rc = lib().iqo_qmm(_p(x), DT[xdt], M, K, _p(w), _p(sc), _p(bi), DT.get(sdt, 0), N,
                       int(transpose), gs, bits, MODES[mode], _p(out), DT[odt], nthreads)
    assert rc == 0
    return out


def qmv_affine(x, xdt, w, scales, biases, sdt, group_size, bits, odt=None, nthreads=0):
    """Streaming (no dequantized copy) affine GEMV/GEMM, transpose=True."""
    odt = odt or xdt
    x = _c(x, NP_STORAGE[xdt])
    M, K = x.shape
    w = _c(w, np.uint32)
    N = w.shape[0]
    out = np.zeros((M, N), NP_STORAGE[odt])
    sc, bi = _c(scales, NP_STORAGE[sdt]), _c(biases, NP_STORAGE[sdt])
    lib().iqo_qmv_affine(_p(x), DT[xdt], M, K, _p(w), _p(sc), _p(bi), DT[sdt], N, group_size,
                         bits, _p(out), DT[odt], nthreads)
    return out


def gather_qmm(x, xdt, w, scales, biases, sdt, lhs_indices, rhs_indices, transpose=True,
               group_size=None, bits=None, mode="affine", odt=None):
    """Brute-force gather_qmm: x [Bx, M, K], w [E, ...]; for each flat index
    pair i: out[i] = qmm(x[lhs[i]], w[rhs[i]]).  Indices are already
    broadcast to one shape; out has shape indices.shape + [M, N]."""
    lhs = np.asarray(lhs_indices).reshape(-1)
    rhs = np.asarray(rhs_indices).reshape(-1)
    outs = []
    for li, ri in zip(lhs, rhs):
        outs.append(qmm(x[li], xdt, w[ri], scales[ri], None if biases is None else biases[ri],
                        sdt, transpose, group_size, bits, mode, odt))
    out = np.stack(outs) if outs else np.zeros((0,) + x.shape[-2:-1] + (0,))
    return out.reshape(np.shape(lhs_indices) + out.shape[-2:])


# ----------------------------------------------------------------- quantize
def affine_quantize(w, wdt, group_size=64, bits=4, sdt=None):
    """w [rows, K] -> (wq u32 [rows, K*bits/32], scales, biases) in sdt
    (default: w's dtype)."""
    sdt = sdt or wdt
    w = _c(w, NP_STORAGE[wdt])
    rows, K = w.shape
    wq = np.zeros((rows, K * bits // 32), np.uint32)
    sc = np.zeros((rows, K // group_size), NP_STORAGE[sdt])
    bi = np.zeros_like(sc)
    lib().iqo_affine_quantize(_p(w), DT[wdt], rows, K, group_size, bits, _p(wq), _p(sc),
                              _p(bi), DT[sdt])
    return wq, sc, bi


def fp_quantize(w, wdt, mode):
    """w [rows, K] -> (wq u32, scales u8) for mode in mxfp4/mxfp8/nvfp4."""
    gs, bits = defaults(mode)
    w = _c(w, NP_STORAGE[wdt])
    rows, K = w.shape
    wq = np.zeros((rows, K * bits // 32), np.uint32)
    sc = np.zeros((rows, K // gs), np.uint8)
    lib().iqo_fp_quantize(_p(w), DT[wdt], rows, K, MODES[mode], _p(wq), _p(sc))
    return wq, sc


# ----------------------------------------------------------------- SwiGLU / MoE routing
def expf(x) -> np.ndarray:
    """The library's exp restated (Cody-Waite + degree-7 Taylor, float32)."""
    x = _c(x, np.float32)
    L = lib()
    return np.array([L.iqo_expf(float(v)) for v in x.ravel()], np.float32).reshape(x.shape)


def swiglu(gu, dt: str) -> np.ndarray:
    """gu [rows, 2I] (gate | up, tagged dt) -> silu(gate) * up [rows, I], each
    elementwise step rounded to dt (mlx/src/nn/mlp.rs:27-33)."""
    gu = _c(gu, NP_STORAGE[dt])
    rows, two_i = gu.shape
    out = np.zeros((rows, two_i // 2), NP_STORAGE[dt])
    lib().iqo_swiglu(_p(gu), DT[dt], rows, two_i // 2, _p(out))
    return out


def moe_route(logits, dt: str, k: int, norm: bool = True):
    """logits [T, E] -> (scores f32 [T, k], experts i32 [T, k]) (moe.rs:67-82)."""
    lg = _c(logits, NP_STORAGE[dt])
    T, E = lg.shape
    scores = np.zeros((T, k), np.float32)
    experts = np.zeros((T, k), np.int32)
    lib().iqo_moe_route(_p(lg), DT[dt], T, E, k, int(norm), _p(scores), _p(experts))
    return scores, experts


def moe_sort(experts, num_experts: int):
    """experts [T, k] i32 -> (tokens, sorted, inverse, offsets), stable by expert."""
    ex = _c(experts, np.int32)
    n, k = ex.size, ex.shape[1]
    tokens, srt, inv = (np.zeros(n, np.int32) for _ in range(3))
    offs = np.zeros(num_experts + 1, np.int32)
    lib().iqo_moe_sort(_p(ex), n, k, num_experts, _p(tokens), _p(srt), _p(inv), _p(offs))
    return tokens, srt, inv, offs


def moe_combine(y, dt: str, inverse, experts, scores, num_experts: int) -> np.ndarray:
    """y [n, D] sorted expert rows -> float32 [T, D] (moe.rs:146-168)."""
    y = _c(y, NP_STORAGE[dt])
    D = y.shape[-1]
    ex = _c(experts, np.int32)
    T, k = ex.shape
    out = np.zeros((T, D), np.float32)
    lib().iqo_moe_combine(_p(y), DT[dt], D, _p(_c(inverse, np.int32)), _p(ex),
                          _p(_c(scores, np.float32)), T, k, num_experts, _p(out))
    return out
