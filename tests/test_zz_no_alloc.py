"""iqmm_moe_sort_noalloc (the sort with its bucket counts in a fixed
per-device array) against iqmm_moe_sort, through the C ABI: bit-identical
tokens / experts / inverse / offsets on two calls in a row, the second
smaller, then a routing past the fixed array (bitonic path, no scratch)."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _arr(t):
    from ironmlx_amd import _lib
    a = _lib.IqmmArray()
    a.data = t.data_ptr()
    for i, s in enumerate(t.shape):
        a.shape[i] = s
    a.ndim = t.dim()
    a.dtype = _lib.INT32
    return a


def _sort(fn_name, experts, E):
    from ironmlx_amd import _lib
    L = _lib.load()
    n = experts.numel()
    outs = [torch.full((n,), -7, dtype=torch.int32, device="cuda") for _ in range(3)]
    outs.append(torch.full((E + 1,), -7, dtype=torch.int32, device="cuda"))
    res = [_arr(o) for o in outs]
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = getattr(L, fn_name)(*[ctypes.byref(r) for r in res], _arr(experts), E, st)
    _lib.check(rc)
    torch.cuda.synchronize()
    return [o.cpu() for o in outs]


def _routing(T, k, E, seed):
    g = torch.Generator().manual_seed(seed)
    ex = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    ex[0, 0] = E + 3          # an invalid id sorts last
    return ex.contiguous().cuda()


@pytest.mark.parametrize("T,k,E", [(512, 8, 256), (64, 8, 256), (512, 8, 2048)])
def test_noalloc_sort_matches_sort(T, k, E):
    """512 x 8 over 256 experts (counts fill 4112 ints of the fixed array),
    then 64 x 8 (514 ints: the array keeps the first call's tail), then
    512 x 8 over 2048 experts (past the array: bitonic, no scratch)."""
    assert torch.cuda.is_available()
    print(f"noalloc sort T={T} k={k} E={E}", flush=True)
    ex = _routing(T, k, E, seed=T + E)
    ref = _sort("iqmm_moe_sort", ex, E)
    got = _sort("iqmm_moe_sort_noalloc", ex, E)
    for r, o in zip(ref, got):
        assert torch.equal(r, o)


def test_noalloc_sort_two_calls_in_a_row():
    """two noalloc calls back to back without a sync, the second smaller, each
    equal to iqmm_moe_sort's result"""
    from ironmlx_amd import _lib
    L = _lib.load()
    print("noalloc sort: two calls in a row", flush=True)
    cases = [(_routing(400, 8, 128, 1), 128), (_routing(33, 4, 60, 2), 60)]
    refs = [_sort("iqmm_moe_sort", ex, E) for ex, E in cases]
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    for ex, E in cases:
        n = ex.numel()
        o = [torch.full((n,), -7, dtype=torch.int32, device="cuda") for _ in range(3)]
        o.append(torch.full((E + 1,), -7, dtype=torch.int32, device="cuda"))
        _lib.check(L.iqmm_moe_sort_noalloc(*[ctypes.byref(_arr(t)) for t in o], _arr(ex), E, st))
        outs.append(o)
    torch.cuda.synchronize()
    for ref, o in zip(refs, outs):
        for r, t in zip(ref, o):
            assert torch.equal(r, t.cpu())


def test_noalloc_sort_rejects_too_many_rows():
    from ironmlx_amd import _lib
    ex = torch.zeros((4097, 8), dtype=torch.int32, device="cuda")
    with pytest.raises(_lib.IqmmError, match="at most 32768"):
        _sort("iqmm_moe_sort_noalloc", ex, 16)
