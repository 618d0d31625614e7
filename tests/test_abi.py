"""C-ABI checks that need no GPU: the library loads, exports exactly what
include/iqmm.h declares, infers result shapes/dtypes (query calls launch
nothing) and rejects bad arguments with mlx-style messages instead of
crashing (mlx/src/error.rs:27-35; survey of ops.rs:653-727)."""
import ctypes
import os
import re

import pytest

from ironmlx_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    with open(os.path.join(ROOT, "include", "iqmm.h")) as f:
        src = f.read()
    return sorted(set(re.findall(r"^\S.*?\b(iqmm_[a-z_]+)\(", src, re.M)))


def test_exports_match_header():
    L = _lib.load()
    decl = _declared()
    assert set(decl) == set(_lib.EXPORTS)
    for name in decl:
        assert hasattr(L, name), name
    assert L.iqmm_version().decode().startswith("iqmm")


def A(shape, dtype, data=None):
    a = _lib.IqmmArray()
    a.data = data
    for i, s in enumerate(shape):
        a.shape[i] = s
    a.ndim = len(shape)
    a.dtype = dtype
    return a


F16, BF16, F32, U32, U8, I32 = (_lib.FLOAT16, _lib.BFLOAT16, _lib.FLOAT32, _lib.UINT32,
                                _lib.UINT8, _lib.INT32)
NONE = _lib.IqmmArray()


def qmm_query(x, w, s, b, transpose=True, gs=None, bits=None, mode=b"affine"):
    L = _lib.load()
    res = _lib.IqmmArray()
    rc = L.iqmm_quantized_matmul(ctypes.byref(res), x, w, s, b, transpose, _lib.opt_int(gs),
                                 _lib.opt_int(bits), mode, None)
    err = L.iqmm_last_error().decode()
    return rc, res, err


def shape_of(res):
    return tuple(res.shape[i] for i in range(res.ndim))


def test_infer_shapes_affine():
    rc, res, err = qmm_query(A((2, 7, 4096), F16), A((11008, 512), U32), A((11008, 64), F16),
                             A((11008, 64), F16))
    assert rc == 0, err
    assert shape_of(res) == (2, 7, 11008) and res.dtype == F16
    # 1-D x
    rc, res, _ = qmm_query(A((4096,), BF16), A((14336, 512), U32), A((14336, 64), BF16),
                           A((14336, 64), BF16))
    assert rc == 0 and shape_of(res) == (14336,)
    # batched w broadcasts against x batch
    rc, res, err = qmm_query(A((3, 1, 5, 256), BF16), A((4, 64, 32), U32), A((4, 64, 4), BF16),
                             A((4, 64, 4), BF16))
    assert rc == 0, err
    assert shape_of(res) == (3, 4, 5, 64)
    # transpose=false: w [K, N*bits/32]
    rc, res, err = qmm_query(A((8, 256), F32), A((256, 16), U32), A((256, 2), F32),
                             A((256, 2), F32), transpose=False)
    assert rc == 0, err
    assert shape_of(res) == (8, 128)


def test_infer_shapes_fp_modes():
    rc, res, err = qmm_query(A((4, 4096), BF16), A((4096, 1024), U32), A((4096, 128), U8), NONE,
                             mode=b"mxfp8")
    assert rc == 0, err
    assert shape_of(res) == (4, 4096)
    rc, res, err = qmm_query(A((4, 4096), BF16), A((4096, 512), U32), A((4096, 256), U8), NONE,
                             mode=b"nvfp4")
    assert rc == 0, err


@pytest.mark.parametrize("args,msg", [
    (dict(mode=b"int3"), "Invalid quantization mode"),
    (dict(bits=7), "number of bits 7 is not supported"),
    (dict(gs=48), "group size 48 is not supported"),
    (dict(mode=b"mxfp8", bits=4), "requires bits 8"),
])
def test_rejects_params(args, msg):
    rc, _, err = qmm_query(A((1, 4096), F16), A((64, 512), U32), A((64, 64), F16),
                           A((64, 64), F16), **args)
    assert rc != 0 and msg in err


def test_rejects_shapes_and_dtypes():
    w, s, b = A((64, 512), U32), A((64, 64), F16), A((64, 64), F16)
    rc, _, err = qmm_query(A((1, 4000), F16), w, s, b)
    assert rc != 0 and "must be equal to the unpacked last dimension" in err
    rc, _, err = qmm_query(A((1, 4096), F16), w, A((64, 32), F16), b)
    assert rc != 0 and "expected number of groups" in err
    rc, _, err = qmm_query(A((1, 4096), F16), w, s, NONE)
    assert rc != 0 and "Biases must be provided" in err
    rc, _, err = qmm_query(A((1, 4096), F16), A((64, 512), F32), s, b)
    assert rc != 0 and "uint32" in err
    rc, _, err = qmm_query(A((1, 4096), BF16), A((64, 1024), U32), A((64, 128), U8),
                           A((64, 128), U8), mode=b"mxfp8")
    assert rc != 0 and "Biases must not be provided" in err
    rc, _, err = qmm_query(A((2, 1, 64), F16), A((3, 8, 8), U32), A((3, 8, 1), F16),
                           A((3, 8, 1), F16), gs=64)
    assert rc != 0 and "broadcast" in err


@pytest.mark.parametrize("xdt,sdt,odt", [(BF16, F16, F32), (F16, BF16, F32), (F32, BF16, F32),
                                         (F32, F16, F32), (BF16, F32, F32), (BF16, BF16, BF16),
                                         (F16, F16, F16), (F32, F32, F32)])
def test_mixed_dtype_promotion(xdt, sdt, odt):
    """x and affine scales of different types promote as MLX promotes them
    (equal types stay; float32 wins; float16 with bfloat16 gives float32)."""
    w, s, b = A((64, 512), U32), A((64, 64), sdt), A((64, 64), sdt)
    rc, res, err = qmm_query(A((3, 4096), xdt), w, s, b)
    assert rc == 0, err
    assert res.dtype == odt and shape_of(res) == (3, 64)
    # fp modes keep x's type (uint8 scales)
    rc, res, err = qmm_query(A((1, 4096), F32), A((64, 1024), U32), A((64, 128), U8), NONE, mode=b"mxfp8")
    assert rc == 0 and res.dtype == F32


def test_result_buffer_mismatch_is_rejected():
    L = _lib.load()
    res = A((1, 63), F16, data=1234)       # wrong N; never dereferenced
    rc = L.iqmm_quantized_matmul(ctypes.byref(res), A((1, 4096), F16), A((64, 512), U32),
                                 A((64, 64), F16), A((64, 64), F16), True, _lib.opt_int(None),
                                 _lib.opt_int(None), b"affine", None)
    assert rc != 0 and "result buffer" in L.iqmm_last_error().decode()


def test_dequantize_and_quantize_queries():
    L = _lib.load()
    res = _lib.IqmmArray()
    rc = L.iqmm_dequantize(ctypes.byref(res), A((10, 3, 96), U32), A((10, 3, 16), BF16),
                           A((10, 3, 16), BF16), _lib.opt_int(64), _lib.opt_int(3), b"affine",
                           _lib.OptionalDtype(0, False), None)
    assert rc == 0, L.iqmm_last_error()
    assert shape_of(res) == (10, 3, 1024) and res.dtype == BF16
    res = _lib.IqmmArray()
    rc = L.iqmm_dequantize(ctypes.byref(res), A((8, 64), U32), A((8, 32), U8), NONE,
                           _lib.opt_int(None), _lib.opt_int(None), b"nvfp4",
                           _lib.OptionalDtype(F32, True), None)
    assert rc == 0 and shape_of(res) == (8, 512) and res.dtype == F32
    rw, rs, rb = _lib.IqmmArray(), _lib.IqmmArray(), _lib.IqmmArray()
    rc = L.iqmm_quantize(ctypes.byref(rw), ctypes.byref(rs), ctypes.byref(rb),
                         A((5, 256), F16), _lib.opt_int(32), _lib.opt_int(6), b"affine", None)
    assert rc == 0
    assert shape_of(rw) == (5, 48) and shape_of(rs) == (5, 8) and rs.dtype == F16
    rc = L.iqmm_quantize(ctypes.byref(rw), ctypes.byref(rs), ctypes.byref(rb),
                         A((5, 100), F16), _lib.opt_int(32), _lib.opt_int(4), b"affine", None)
    assert rc != 0 and "divisible" in L.iqmm_last_error().decode()


def test_gather_qmm_query():
    L = _lib.load()
    res = _lib.IqmmArray()
    rc = L.iqmm_gather_qmm(ctypes.byref(res), A((64, 1, 1, 2048), BF16), A((256, 512, 256), U32),
                           A((256, 512, 32), BF16), A((256, 512, 32), BF16), NONE,
                           A((64, 8), I32), True, _lib.opt_int(None), _lib.opt_int(None),
                           b"affine", False, None)
    assert rc == 0, L.iqmm_last_error()
    assert shape_of(res) == (64, 8, 1, 512)
    rc = L.iqmm_gather_qmm(ctypes.byref(res), A((64, 1, 2048), BF16), A((256, 512, 256), U32),
                           A((256, 512, 32), BF16), A((256, 512, 32), BF16), NONE,
                           A((64, 8), F32), True, _lib.opt_int(None), _lib.opt_int(None),
                           b"affine", False, None)
    assert rc != 0 and "integers" in L.iqmm_last_error().decode()


# ------------------------------------------------------------------ fused / routing entry points
def test_swiglu_infer_and_errors():
    L = _lib.load()
    res = _lib.IqmmArray()
    rc = L.iqmm_quantized_swiglu(ctypes.byref(res), A((1, 4096), BF16), A((28672, 512), U32),
                                 A((28672, 64), BF16), A((28672, 64), BF16), _lib.opt_int(None),
                                 _lib.opt_int(None), b"affine", None)
    assert rc == 0, L.iqmm_last_error().decode()
    assert shape_of(res) == (1, 14336) and res.dtype == BF16
    res = _lib.IqmmArray()
    rc = L.iqmm_quantized_swiglu(ctypes.byref(res), A((1, 4096), BF16), A((301, 512), U32),
                                 A((301, 64), BF16), A((301, 64), BF16), _lib.opt_int(None),
                                 _lib.opt_int(None), b"affine", None)
    assert rc != 0 and "even number of rows" in L.iqmm_last_error().decode()
    res = _lib.IqmmArray()
    rc = L.iqmm_gather_qmm_swiglu(ctypes.byref(res), A((64, 1, 2048), BF16), A((256, 1024, 256), U32),
                                  A((256, 1024, 32), BF16), A((256, 1024, 32), BF16), A((512,), I32),
                                  A((512,), I32), _lib.opt_int(None), _lib.opt_int(None), b"affine", True,
                                  None)
    assert rc == 0, L.iqmm_last_error().decode()
    assert shape_of(res) == (512, 1, 512)


def test_dequantize_rows_infer_and_errors():
    L = _lib.load()
    od = _lib.OptionalDtype(0, False)
    res = _lib.IqmmArray()
    rc = L.iqmm_dequantize_rows(ctypes.byref(res), A((128256, 512), U32), A((128256, 64), BF16),
                                A((128256, 64), BF16), A((2, 7), I32), _lib.opt_int(None),
                                _lib.opt_int(None), b"affine", od, None)
    assert rc == 0, L.iqmm_last_error().decode()
    assert shape_of(res) == (2, 7, 4096) and res.dtype == BF16
    res = _lib.IqmmArray()
    rc = L.iqmm_dequantize_rows(ctypes.byref(res), A((100, 512), U32), A((100, 64), BF16),
                                A((100, 64), BF16), A((3,), F32), _lib.opt_int(None),
                                _lib.opt_int(None), b"affine", od, None)
    assert rc != 0 and "indices must be an integer array" in L.iqmm_last_error().decode()


def test_moe_entry_points_infer_and_errors():
    L = _lib.load()
    rs, re_ = _lib.IqmmArray(), _lib.IqmmArray()
    rc = L.iqmm_moe_route(ctypes.byref(rs), ctypes.byref(re_), A((512, 256), BF16), 8, True, None)
    assert rc == 0, L.iqmm_last_error().decode()
    assert shape_of(rs) == (512, 8) and rs.dtype == F32 and re_.dtype == I32
    rs, re_ = _lib.IqmmArray(), _lib.IqmmArray()
    assert L.iqmm_moe_route(ctypes.byref(rs), ctypes.byref(re_), A((4, 16), BF16), 17, True, None) != 0
    assert "k must be" in L.iqmm_last_error().decode()
    outs = [_lib.IqmmArray() for _ in range(4)]
    rc = L.iqmm_moe_sort(*[ctypes.byref(o) for o in outs], A((512, 8), I32), 256, None)
    assert rc == 0, L.iqmm_last_error().decode()
    assert [shape_of(o) for o in outs] == [(4096,), (4096,), (4096,), (257,)]
    outs = [_lib.IqmmArray() for _ in range(4)]
    assert L.iqmm_moe_sort(*[ctypes.byref(o) for o in outs], A((5000, 8), I32), 256, None) != 0
    assert "32768" in L.iqmm_last_error().decode()
    res = _lib.IqmmArray()
    rc = L.iqmm_moe_combine(ctypes.byref(res), A((4096, 1, 2048), BF16), A((4096,), I32), A((512, 8), I32),
                            A((512, 8), F32), 256, None)
    assert rc == 0, L.iqmm_last_error().decode()
    assert shape_of(res) == (512, 2048) and res.dtype == F32
