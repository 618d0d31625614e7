"""Host-side mirror of ironmlx's quantized ops over the C ABI.

Same names, argument order, argument meaning, defaults and error behaviour as
the Rust wrappers in ``mlx/src/ops.rs``:

* ``dequantize(w, scales, biases, group_size, bits, mode, stream)``
  -- ``mlx/src/ops.rs:653-686``
* ``quantized_matmul(x, w, scales, biases, transpose, group_size, bits, mode,
  stream)`` -- ``mlx/src/ops.rs:695-727``
* ``gather_qmm(...)`` -- mlx-c's ``mlx_gather_qmm`` (ironmlx has no wrapper;
  its MoE loop ``mlx/src/nn/moe.rs:84-170`` is what it replaces)
* ``quantize(w, group_size, bits, mode)`` -- mlx-c's ``mlx_quantize``

Arrays are torch tensors on a ROCm device (torch only provides device memory
and the stream); every computation runs in the HIP library libiqmm.so.
Failures raise :class:`IqmmError` with the library's message, as the Rust
wrappers return ``Err(Error::Mlx(msg))``.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import IqmmError

_TORCH_TO_DT = {
    torch.float32: _lib.FLOAT32, torch.float16: _lib.FLOAT16, torch.bfloat16: _lib.BFLOAT16,
    torch.uint32: _lib.UINT32, torch.int32: _lib.INT32, torch.uint8: _lib.UINT8,
    torch.int64: _lib.INT64,
}
_DT_TO_TORCH = {_lib.FLOAT32: torch.float32, _lib.FLOAT16: torch.float16,
                _lib.BFLOAT16: torch.bfloat16, _lib.UINT32: torch.uint32,
                _lib.UINT8: torch.uint8, _lib.INT32: torch.int32, _lib.INT64: torch.int64}


def _device_of(*ts) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise IqmmError("iqmm ops run on the GPU only; got a tensor on "
                            f"{t.device} (there is no CPU path)")
        if dev is not None and t.device != dev:
            raise IqmmError(f"tensors on different devices: {dev} and {t.device}")
        dev = t.device
    return dev


def _arr(t: Optional[torch.Tensor], packed: bool = False) -> _lib.IqmmArray:
    a = _lib.IqmmArray()
    if t is None:
        return a
    if not t.is_contiguous():
        raise IqmmError("iqmm ops take C-contiguous arrays")
    if t.dim() > _lib.MAX_NDIM:
        raise IqmmError(f"too many dimensions ({t.dim()})")
    a.data = t.data_ptr() if t.numel() > 0 else (t.data_ptr() or 1)
    for i, s in enumerate(t.shape):
        a.shape[i] = s
    a.ndim = t.dim()
    dt = _TORCH_TO_DT.get(t.dtype)
    if dt is None:
        raise IqmmError(f"unsupported dtype {t.dtype}")
    # packed weights may arrive as int32 views of the uint32 words
    a.dtype = _lib.UINT32 if (packed and dt == _lib.INT32) else dt
    return a


def _stream(dev: torch.device, stream) -> ctypes.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream(dev)
    return ctypes.c_void_p(stream.cuda_stream)


def _alloc(res: _lib.IqmmArray, dev) -> torch.Tensor:
    shape = tuple(res.shape[i] for i in range(res.ndim))
    dt = _DT_TO_TORCH[res.dtype]
    if dt == torch.uint32:
        return torch.empty(shape, dtype=torch.int32, device=dev).view(torch.uint32)
    return torch.empty(shape, dtype=dt, device=dev)


def _run(fn, res: _lib.IqmmArray, dev, args) -> torch.Tensor:
    _lib.check(fn(ctypes.byref(res), *args))          # shape/dtype inference
    out = _alloc(res, dev)
    res.data = out.data_ptr() if out.numel() > 0 else 1
    _lib.check(fn(ctypes.byref(res), *args))
    return out


def _mode(mode: str) -> bytes:
    return (mode or "affine").encode()


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: Optional[torch.Tensor] = None, transpose: bool = True,
                     group_size: Optional[int] = None, bits: Optional[int] = None,
                     mode: str = "affine", stream=None) -> torch.Tensor:
    """``x @ dequantize(w, scales, biases)^T`` (``transpose``) or ``x @
    dequantize(w)``; mirrors ``ops::quantized_matmul`` (mlx/src/ops.rs:695-727)."""
    L = _lib.load()
    dev = _device_of(x, w, scales, biases)
    args = (_arr(x), _arr(w, True), _arr(scales), _arr(biases), bool(transpose),
            _lib.opt_int(group_size), _lib.opt_int(bits), _mode(mode), _stream(dev, stream))
    return _run(L.iqmm_quantized_matmul, _lib.IqmmArray(), dev, args)


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: Optional[torch.Tensor] = None,
               group_size: Optional[int] = None, bits: Optional[int] = None,
               mode: str = "affine", stream=None,
               dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Unpack and rescale; mirrors ``ops::dequantize`` (mlx/src/ops.rs:653-686).
    ``dtype`` is mlx-c's optional output dtype (ironmlx always passes none)."""
    L = _lib.load()
    dev = _device_of(w, scales, biases)
    od = _lib.OptionalDtype(0, False) if dtype is None else \
        _lib.OptionalDtype(_TORCH_TO_DT[dtype], True)
    args = (_arr(w, True), _arr(scales), _arr(biases), _lib.opt_int(group_size),
            _lib.opt_int(bits), _mode(mode), od, _stream(dev, stream))
    return _run(L.iqmm_dequantize, _lib.IqmmArray(), dev, args)


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
               biases: Optional[torch.Tensor] = None,
               lhs_indices: Optional[torch.Tensor] = None,
               rhs_indices: Optional[torch.Tensor] = None, transpose: bool = True,
               group_size: Optional[int] = None, bits: Optional[int] = None,
               mode: str = "affine", sorted_indices: bool = False, stream=None) -> torch.Tensor:
    """``out[i] = x[lhs[i]] @ dequantize(w[rhs[i]])^T`` over the broadcast index
    shape; mirrors mlx-c ``mlx_gather_qmm``."""
    L = _lib.load()
    dev = _device_of(x, w, scales, biases, lhs_indices, rhs_indices)
    args = (_arr(x), _arr(w, True), _arr(scales), _arr(biases), _arr(lhs_indices),
            _arr(rhs_indices), bool(transpose), _lib.opt_int(group_size), _lib.opt_int(bits),
            _mode(mode), bool(sorted_indices), _stream(dev, stream))
    return _run(L.iqmm_gather_qmm, _lib.IqmmArray(), dev, args)


def quantized_swiglu(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: Optional[torch.Tensor] = None, group_size: Optional[int] = None,
                     bits: Optional[int] = None, mode: str = "affine", stream=None) -> torch.Tensor:
    """``silu(x @ gate^T) * (x @ up^T)`` over a fused gate_up weight (gate rows
    first, then up rows): the gate / up / silu / multiply of
    ``MLP::forward_with_stream`` (mlx/src/nn/mlp.rs:27-33) in one call."""
    L = _lib.load()
    dev = _device_of(x, w, scales, biases)
    args = (_arr(x), _arr(w, True), _arr(scales), _arr(biases), _lib.opt_int(group_size),
            _lib.opt_int(bits), _mode(mode), _stream(dev, stream))
    return _run(L.iqmm_quantized_swiglu, _lib.IqmmArray(), dev, args)


def gather_qmm_swiglu(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                      biases: Optional[torch.Tensor] = None,
                      lhs_indices: Optional[torch.Tensor] = None,
                      rhs_indices: Optional[torch.Tensor] = None,
                      group_size: Optional[int] = None, bits: Optional[int] = None,
                      mode: str = "affine", sorted_indices: bool = False,
                      stream=None) -> torch.Tensor:
    """:func:`gather_qmm` over stacked gate_up experts [E, 2I, .] followed by
    the SwiGLU of :func:`quantized_swiglu` (each Expert of mlx/src/nn/moe.rs:10-33)."""
    L = _lib.load()
    dev = _device_of(x, w, scales, biases, lhs_indices, rhs_indices)
    args = (_arr(x), _arr(w, True), _arr(scales), _arr(biases), _arr(lhs_indices),
            _arr(rhs_indices), _lib.opt_int(group_size), _lib.opt_int(bits), _mode(mode),
            bool(sorted_indices), _stream(dev, stream))
    return _run(L.iqmm_gather_qmm_swiglu, _lib.IqmmArray(), dev, args)


def dequantize_rows(w: torch.Tensor, scales: torch.Tensor, biases: Optional[torch.Tensor],
                    indices: torch.Tensor, group_size: Optional[int] = None,
                    bits: Optional[int] = None, mode: str = "affine", stream=None,
                    dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``dequantize(w)[indices]`` without dequantizing the table (the lookup of
    ``QuantizedEmbedding::forward``, mlx/src/nn/embedding.rs:62-72)."""
    L = _lib.load()
    dev = _device_of(w, scales, biases, indices)
    od = _lib.OptionalDtype(0, False) if dtype is None else \
        _lib.OptionalDtype(_TORCH_TO_DT[dtype], True)
    args = (_arr(w, True), _arr(scales), _arr(biases), _arr(indices), _lib.opt_int(group_size),
            _lib.opt_int(bits), _mode(mode), od, _stream(dev, stream))
    return _run(L.iqmm_dequantize_rows, _lib.IqmmArray(), dev, args)


def _run_multi(fn, n_out: int, dev, args, optional_last: bool = False):
    res = [_lib.IqmmArray() for _ in range(n_out)]
    refs = [ctypes.byref(r) for r in res]
    _lib.check(fn(*refs, *args))
    outs = [_alloc(r, dev) for r in res]
    for r, t in zip(res, outs):
        r.data = t.data_ptr() or 1
    _lib.check(fn(*refs, *args))
    return outs


def moe_route(logits: torch.Tensor, k: int, norm_topk_prob: bool = True,
              stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Softmax over experts, top-k (stable descending), optional normalisation
    (mlx/src/nn/moe.rs:67-82).  Returns (scores float32 [T, k], experts int32 [T, k])."""
    L = _lib.load()
    dev = _device_of(logits)
    args = (_arr(logits), int(k), bool(norm_topk_prob), _stream(dev, stream))
    scores, experts = _run_multi(L.iqmm_moe_route, 2, dev, args)
    return scores, experts


def moe_sort(experts: torch.Tensor, num_experts: int, stream=None):
    """Stable sort of the (token, slot) rows by expert (mlx/src/nn/moe.rs:92-104).
    Returns (tokens, sorted_experts, inverse, offsets), all int32."""
    L = _lib.load()
    dev = _device_of(experts)
    args = (_arr(experts), int(num_experts), _stream(dev, stream))
    return tuple(_run_multi(L.iqmm_moe_sort, 4, dev, args))


def moe_combine(y: torch.Tensor, inverse: torch.Tensor, experts: torch.Tensor,
                scores: torch.Tensor, num_experts: int, stream=None) -> torch.Tensor:
    """Per token, the sorted expert rows times their scores summed in float32 in
    ascending expert order (mlx/src/nn/moe.rs:146-168).  Returns float32 [T, D]."""
    L = _lib.load()
    dev = _device_of(y, inverse, experts, scores)
    args = (_arr(y), _arr(inverse), _arr(experts), _arr(scores), int(num_experts),
            _stream(dev, stream))
    return _run(L.iqmm_moe_combine, _lib.IqmmArray(), dev, args)


def moe_token(logits: torch.Tensor, x: torch.Tensor, gate_up, down, k: int,
              norm_topk_prob: bool = True, group_size: int = 64, bits: int = 4,
              stream=None) -> torch.Tensor:
    """One token's routed experts (route, fused gate_up SwiGLU, down, ordered
    combine; mlx/src/nn/moe.rs:55-183 for T = 1) in two launches.  ``gate_up``
    and ``down`` are (weight, scales, biases) of the stacked affine 4-bit
    experts.  Returns float32 [1, D]."""
    L = _lib.load()
    (gw, gs, gb), (dw, ds, db) = gate_up, down
    dev = _device_of(logits, x, gw, gs, gb, dw, ds, db)
    args = (_arr(logits), _arr(x), _arr(gw, True), _arr(gs), _arr(gb), _arr(dw, True), _arr(ds),
            _arr(db), int(k), bool(norm_topk_prob), int(group_size), int(bits), _stream(dev, stream))
    return _run(L.iqmm_moe_token, _lib.IqmmArray(), dev, args)


def quantize(w: torch.Tensor, group_size: Optional[int] = None, bits: Optional[int] = None,
             mode: str = "affine", stream=None
             ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Quantize along the last axis; returns (w_q uint32, scales, biases|None);
    mirrors mlx-c ``mlx_quantize``."""
    L = _lib.load()
    dev = _device_of(w)
    rw, rs, rb = _lib.IqmmArray(), _lib.IqmmArray(), _lib.IqmmArray()
    args = (_arr(w), _lib.opt_int(group_size), _lib.opt_int(bits), _mode(mode),
            _stream(dev, stream))
    _lib.check(L.iqmm_quantize(ctypes.byref(rw), ctypes.byref(rs), ctypes.byref(rb), *args))
    tw, ts = _alloc(rw, dev), _alloc(rs, dev)
    tb = _alloc(rb, dev) if rb.ndim > 0 else None
    rw.data, rs.data = tw.data_ptr() or 1, ts.data_ptr() or 1
    if tb is not None:
        rb.data = tb.data_ptr() or 1
    _lib.check(L.iqmm_quantize(ctypes.byref(rw), ctypes.byref(rs),
                               ctypes.byref(rb) if tb is not None else None, *args))
    return tw, ts, tb


__all__ = ["quantized_matmul", "dequantize", "gather_qmm", "quantize", "quantized_swiglu",
           "gather_qmm_swiglu", "dequantize_rows", "moe_route", "moe_sort", "moe_combine",
           "IqmmError"]


def workspace_reserve(nbytes: int, stream=None, device=None) -> None:
    """Grow every library workspace of ``stream`` (default: the current stream)
    to at least ``nbytes`` so that calls later captured into a HIP graph on that
    stream allocate nothing (the library never allocates while capturing)."""
    L = _lib.load()
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    _lib.check(L.iqmm_workspace_reserve(_stream(dev, stream), int(nbytes)))
