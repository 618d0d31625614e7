"""Shared helpers for the GPU parity tests: seeded input builders and
torch <-> oracle conversions.  The oracle (oracle/) is the checker only."""
import numpy as np
import torch

import oracle

TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def to_np(t: torch.Tensor, dt: str) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if dt == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    if dt == "f16":
        return t.numpy()
    return t.numpy()


def from_np(a: np.ndarray, dt: str, dev="cuda") -> torch.Tensor:
    if dt == "bf16":
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def words_to_torch(w: np.ndarray, dev="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(w).view(np.int32)).to(dev).view(torch.uint32)


def words_to_np(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int32).cpu().numpy().view(np.uint32)


def rand_affine(rng, rows, K, gs, bits, sdt, lead=()):
    """Random codes with scale ~ 0.02/2^bits and bias ~ N(0, 0.02): the scale of
    a quantized N(0, 0.02) weight."""
    shape = lead + (rows, K)
    codes = rng.integers(0, 1 << bits, shape).astype(np.uint32)
    s = (rng.standard_normal(lead + (rows, K // gs)) * 0.08 / (1 << bits)).astype(np.float32)
    b = (rng.standard_normal(lead + (rows, K // gs)) * 0.02).astype(np.float32)
    w = oracle.pack(codes.reshape(-1, K), bits).reshape(lead + (rows, K * bits // 32))
    return w, oracle.from_float(s, sdt), oracle.from_float(b, sdt)


def rand_fp(rng, rows, K, mode, lead=()):
    gs, bits = oracle.defaults(mode)
    shape = lead + (rows, K)
    codes = rng.integers(0, 1 << bits, shape).astype(np.uint32)
    if mode == "mxfp8":
        codes[(codes & 0x7F) == 0x7F] = 0x7E          # no NaN elements
        sc = rng.integers(118, 122, lead + (rows, K // gs)).astype(np.uint8)
    elif mode == "nvfp4":
        sc = rng.integers(0x20, 0x38, lead + (rows, K // gs)).astype(np.uint8)
    else:
        sc = rng.integers(118, 124, lead + (rows, K // gs)).astype(np.uint8)
    w = oracle.pack(codes.reshape(-1, K), bits).reshape(lead + (rows, K * bits // 32))
    return w, sc


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| in float64 (the tolerance metric)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref)) if ref.size else 1.0
    return float(np.max(np.abs(got - ref)) / max(den, 1e-30)) if ref.size else 0.0


def as_f64(a: np.ndarray, dt: str) -> np.ndarray:
    return oracle.to_float(a, dt).astype(np.float64) if dt != "f32" else a.astype(np.float64)
