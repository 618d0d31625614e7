"""Oracle parity at the exact shapes of BASELINE.json's configs, so that every
tile, split-K and kernel choice the library makes for them runs against the
CPU restatement of MLX's arithmetic (oracle/):

* C3 Llama-3-8B decode, M in {4, 8, 16, 32}: q/o 4096->4096, k/v 4096->1024,
  fused qkv 4096->6144, gate/up 4096->14336, down 14336->4096
  (mlx/src/model/llama.rs:117-140 through QuantizedLinear,
  mlx/src/nn/linear.rs:51-63);
* the fused SwiGLU at those widths, I = 14336, against the oracle's own
  gate / up products and its SwiGLU (mlx/src/nn/mlp.rs:27-33);
* C4 MoE down projection 512 -> 2048 over 256 experts, T in {64, 512};
* C5 K = N = 4096, M in {1, 256}: affine bits {2, 3, 6, 8} x gs {32, 64,
  128}, mxfp4, mxfp8, nvfp4.

The metric is max |got - ref| / max |ref| (fp32 oracle output), bounded by
1e-2 for bf16 / fp16 outputs and 2e-2 for the fp8 / fp4 modes."""
import os

import numpy as np
import pytest
import torch

import oracle
from helpers import as_f64, rel_err, to_np

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)
TOL_AFFINE = 1e-2
TOL_FP = 2e-2


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available()
    from ironmlx_amd import ops as _ops
    return _ops


def _words(t):
    return t.view(torch.int32).cpu().numpy().view(np.uint32)


def _weight(ops, N, K, seed, gs=64, bits=4, mode="affine", dt=torch.bfloat16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    W = (torch.randn((N, K), generator=g, device="cuda") * 0.02).to(dt)
    if mode == "affine":
        return ops.quantize(W, gs, bits)
    return ops.quantize(W, mode=mode)


def _x(M, K, seed, dt=torch.bfloat16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn((M, K), generator=g, device="cuda").to(dt)


C3_SHAPES = [(4096, 4096), (1024, 4096), (6144, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("M", [2, 3, 4, 8, 16, 32])
@pytest.mark.parametrize("N,K", C3_SHAPES)
def test_llama_decode_widths_vs_oracle(ops, M, N, K):
    print(f"C3 qmm M={M} N={N} K={K}", flush=True)
    wq, s, b = _weight(ops, N, K, seed=100 + N + K)
    x = _x(M, K, seed=M)
    got = ops.quantized_matmul(x, wq, s, b, True, 64, 4)
    ref = oracle.qmv_affine(to_np(x, "bf16"), "bf16", _words(wq), to_np(s, "bf16"),
                            to_np(b, "bf16"), "bf16", 64, 4, odt="f32", nthreads=NT)
    assert rel_err(as_f64(to_np(got, "bf16"), "bf16"), ref) <= TOL_AFFINE


@pytest.mark.parametrize("M", [1, 2, 3, 4, 16, 32])
def test_fused_swiglu_llama_vs_oracle(ops, M):
    """silu(x @ gate^T) * (x @ up^T) over the stacked [2I, K] gate_up weight,
    I = 14336: the oracle computes both products from the packed words,
    rounds them to bf16 and applies its SwiGLU (each step rounded to bf16)."""
    I, K = 14336, 4096
    print(f"SwiGLU M={M} I={I}", flush=True)
    wq, s, b = _weight(ops, 2 * I, K, seed=7)
    x = _x(M, K, seed=70 + M)
    got = ops.quantized_swiglu(x, wq, s, b, 64, 4)
    gu = oracle.qmv_affine(to_np(x, "bf16"), "bf16", _words(wq), to_np(s, "bf16"),
                           to_np(b, "bf16"), "bf16", 64, 4, odt="bf16", nthreads=NT)
    ref = as_f64(oracle.swiglu(gu, "bf16"), "bf16")
    assert rel_err(as_f64(to_np(got, "bf16"), "bf16"), ref) <= TOL_AFFINE


@pytest.mark.parametrize("T", [64, 512])
def test_moe_down_projection_vs_oracle(ops, T):
    """Qwen3.5-MoE down projection (512 -> 2048, 256 experts, top-8 of a
    softmax over N(0,1) logits), sorted grouped form, against the oracle's
    per-expert products over the same rows."""
    E, H, I, k = 256, 2048, 512, 8
    print(f"C4 down T={T}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(31)
    W = (torch.randn((E * H, I), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    wq, s, b = ops.quantize(W, 64, 4)
    logits = torch.randn((T, E), generator=g, device="cuda")
    idx = torch.topk(torch.softmax(logits, -1), k, dim=-1).indices.to(torch.int32).view(-1)
    order = torch.argsort(idx, stable=True)
    se = idx[order].contiguous()
    h = torch.randn((T * k, 1, I), generator=g, device="cuda").to(torch.bfloat16)
    got = ops.gather_qmm(h, wq.view(E, H, -1), s.view(E, H, -1), b.view(E, H, -1), None, se,
                         sorted_indices=True)[:, 0]
    got = as_f64(to_np(got, "bf16"), "bf16")
    wn, sn, bn = _words(wq).reshape(E, H, -1), to_np(s, "bf16").reshape(E, H, -1), \
        to_np(b, "bf16").reshape(E, H, -1)
    hn = to_np(h[:, 0], "bf16")
    sen = se.cpu().numpy()
    ref = np.zeros((T * k, H))
    for e in np.unique(sen):
        rows = np.nonzero(sen == e)[0]
        ref[rows] = oracle.qmv_affine(hn[rows], "bf16", wn[e], sn[e], bn[e], "bf16", 64, 4,
                                      odt="f32", nthreads=NT)
    assert rel_err(got, ref) <= TOL_AFFINE


C5_AFFINE = [(bits, gs) for bits in (2, 3, 6, 8) for gs in (32, 64, 128)]


@pytest.mark.parametrize("M", [1, 256])
@pytest.mark.parametrize("bits,gs", C5_AFFINE)
def test_mode_sweep_affine_vs_oracle(ops, M, bits, gs):
    print(f"C5 affine bits={bits} gs={gs} M={M}", flush=True)
    wq, s, b = _weight(ops, 4096, 4096, seed=400 + bits * 10 + gs, gs=gs, bits=bits)
    x = _x(M, 4096, seed=4)
    got = ops.quantized_matmul(x, wq, s, b, True, gs, bits)
    ref = oracle.qmm(to_np(x, "bf16"), "bf16", _words(wq), to_np(s, "bf16"), to_np(b, "bf16"),
                     "bf16", True, gs, bits, "affine", odt="f32", nthreads=NT)
    assert rel_err(as_f64(to_np(got, "bf16"), "bf16"), ref) <= TOL_AFFINE


@pytest.mark.parametrize("M", [1, 256])
@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8", "nvfp4"])
def test_mode_sweep_fp_vs_oracle(ops, M, mode):
    print(f"C5 {mode} M={M}", flush=True)
    wq, s, _ = _weight(ops, 4096, 4096, seed=500 + len(mode), mode=mode)
    x = _x(M, 4096, seed=5)
    got = ops.quantized_matmul(x, wq, s, None, True, mode=mode)
    ref = oracle.qmm(to_np(x, "bf16"), "bf16", _words(wq), s.cpu().numpy(), None, "bf16", True,
                     mode=mode, odt="f32", nthreads=NT)
    assert rel_err(as_f64(to_np(got, "bf16"), "bf16"), ref) <= TOL_FP


def test_tied_lm_head_gemv_vs_oracle(ops):
    """The tied lm_head of Llama-3-8B (LinearLayer::from_weights on
    model.embed_tokens, mlx/src/model/llama.rs:158-162): N = 128256, K = 4096,
    M = 1 GEMV over the quantized embedding table."""
    N, K = 128256, 4096
    print("lm_head N=128256 K=4096 M=1", flush=True)
    wq, s, b = _weight(ops, N, K, seed=9)
    x = _x(1, K, seed=9)
    got = ops.quantized_matmul(x, wq, s, b, True, 64, 4)
    ref = oracle.qmv_affine(to_np(x, "bf16"), "bf16", _words(wq), to_np(s, "bf16"),
                            to_np(b, "bf16"), "bf16", 64, 4, odt="f32", nthreads=NT)
    assert rel_err(as_f64(to_np(got, "bf16"), "bf16"), ref) <= TOL_AFFINE


@pytest.mark.parametrize("N,M", [(128256, 8), (65536, 20)])
def test_wide_matrix_decode_widths_vs_oracle(ops, N, M):
    """Wide matrices at decode widths (the tied lm_head at batched decode,
    llama.rs:158-162): the streaming kernel, one and two m tiles."""
    K = 4096
    print(f"wide qmm M={M} N={N} K={K}", flush=True)
    wq, s, b = _weight(ops, N, K, seed=N + M)
    x = _x(M, K, seed=M + 1)
    got = ops.quantized_matmul(x, wq, s, b, True, 64, 4)
    ref = oracle.qmv_affine(to_np(x, "bf16"), "bf16", _words(wq), to_np(s, "bf16"),
                            to_np(b, "bf16"), "bf16", 64, 4, odt="f32", nthreads=NT)
    assert rel_err(as_f64(to_np(got, "bf16"), "bf16"), ref) <= TOL_AFFINE


@pytest.mark.parametrize("gs,M,dt", [(32, 8, "bf16"), (64, 12, "f16"), (32, 3, "f16")])
def test_fused_swiglu_group_sizes_vs_oracle(ops, gs, M, dt):
    """The streaming SwiGLU kernel at gs 32 and in fp16, I = 14336."""
    I, K = 14336, 4096
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    print(f"SwiGLU gs={gs} M={M} {dt}", flush=True)
    wq, s, b = _weight(ops, 2 * I, K, seed=11 + gs, gs=gs, dt=tdt)
    x = _x(M, K, seed=80 + M, dt=tdt)
    got = ops.quantized_swiglu(x, wq, s, b, gs, 4)
    gu = oracle.qmv_affine(to_np(x, dt), dt, _words(wq), to_np(s, dt), to_np(b, dt), dt, gs, 4,
                           odt=dt, nthreads=NT)
    ref = as_f64(oracle.swiglu(gu, dt), dt)
    assert rel_err(as_f64(to_np(got, dt), dt), ref) <= TOL_AFFINE


@pytest.mark.parametrize("bits", [2, 3, 6])
@pytest.mark.parametrize("N,K,gs,dt", [(1000, 1024, 32, "bf16"), (4097, 6144, 64, "f16"),
                                       (4096, 14336, 128, "bf16"), (2047, 4096, 64, "f16")])
def test_low_bit_gemv_widths_vs_oracle(ops, bits, N, K, gs, dt):
    """The affine 2 / 3 / 6-bit one-row GEMV: one and two rows per wave (N
    below / from 4096, with a ragged last pair), one to seven chunks per
    lane, bf16 and fp16."""
    print(f"low-bit GEMV bits={bits} N={N} K={K} gs={gs} {dt}", flush=True)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    wq, s, b = _weight(ops, N, K, seed=900 + bits + K, gs=gs, bits=bits, dt=tdt)
    x = _x(1, K, seed=9, dt=tdt)
    got = ops.quantized_matmul(x, wq, s, b, True, gs, bits)
    ref = oracle.qmm(to_np(x, dt), dt, _words(wq), to_np(s, dt), to_np(b, dt),
                     dt, True, gs, bits, "affine", odt="f32", nthreads=NT)
    assert rel_err(as_f64(to_np(got, dt), dt), ref) <= TOL_AFFINE


@pytest.mark.parametrize("bits", [2, 3, 5, 6])
@pytest.mark.parametrize("M,N,K,gs,dt", [(130, 1000, 1024, 32, "f16"), (300, 4096, 2048, 128, "bf16")])
def test_widened_code_gemm_vs_oracle(ops, bits, M, N, K, gs, dt):
    """M > 64 with 2 / 3 / 5 / 6-bit codes: the codes are widened to 4 or 8
    bits in the stream's workspace and run through the register-B GEMM."""
    print(f"widened GEMM bits={bits} M={M} N={N} K={K} gs={gs} {dt}", flush=True)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    wq, s, b = _weight(ops, N, K, seed=950 + bits + M, gs=gs, bits=bits, dt=tdt)
    x = _x(M, K, seed=11, dt=tdt)
    got = ops.quantized_matmul(x, wq, s, b, True, gs, bits)
    ref = oracle.qmm(to_np(x, dt), dt, _words(wq), to_np(s, dt), to_np(b, dt),
                     dt, True, gs, bits, "affine", odt="f32", nthreads=NT)
    assert rel_err(as_f64(to_np(got, dt), dt), ref) <= TOL_AFFINE


@pytest.mark.parametrize("N,M,gs,dt", [(10240, 12, 32, "f16"), (6144, 5, 64, "bf16"), (8000, 12, 64, "bf16"),
                                       (6150, 9, 32, "bf16"), (10250, 2, 32, "f16"), (6144, 3, 64, "f16")])
def test_streaming_decode_widths_vs_oracle(ops, N, M, gs, dt):
    """The streaming kernel at 6144 .. 14336 rows (K = 4096): gs 32 / 64,
    fp16, a ragged last tile, M not a multiple of 4."""
    print(f"stream decode N={N} M={M} gs={gs} {dt}", flush=True)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    wq, s, b = _weight(ops, N, 4096, seed=970 + M, gs=gs, dt=tdt)
    x = _x(M, 4096, seed=12, dt=tdt)
    got = ops.quantized_matmul(x, wq, s, b, True, gs, 4)
    ref = oracle.qmm(to_np(x, dt), dt, _words(wq), to_np(s, dt), to_np(b, dt),
                     dt, True, gs, 4, "affine", odt="f32", nthreads=NT)
    assert rel_err(as_f64(to_np(got, dt), dt), ref) <= TOL_AFFINE


@pytest.mark.parametrize("N,K,dt", [(10250, 4096, "f16"), (20482, 4096, "bf16"), (12000, 3072, "bf16"),
                                    (28672, 4096, "bf16"), (16384, 2048, "bf16"), (10240, 8192, "f16")])
def test_shared_x_gemv_vs_oracle(ops, N, K, dt):
    """The one-row GEMV with four waves sharing x through LDS (from 10240
    rows): a ragged last workgroup (rows past N) and a K that leaves some
    lanes' chunks masked."""
    print(f"shared-x GEMV N={N} K={K} {dt}", flush=True)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    wq, s, b = _weight(ops, N, K, seed=990 + N % 97, gs=64, dt=tdt)
    x = _x(1, K, seed=13, dt=tdt)
    got = ops.quantized_matmul(x, wq, s, b, True, 64, 4)
    ref = oracle.qmv_affine(to_np(x, dt), dt, _words(wq), to_np(s, dt), to_np(b, dt), dt, 64, 4,
                            odt="f32", nthreads=NT)
    assert rel_err(as_f64(to_np(got, dt), dt), ref) <= TOL_AFFINE


@pytest.mark.parametrize("I,dt", [(6144, "bf16"), (5203, "f16")])
def test_shared_x_swiglu_rows_vs_oracle(ops, I, dt):
    """The M = 1 fused SwiGLU with four gate / up wave pairs sharing x
    (10240 <= 2I < 24576 rows), including a ragged last workgroup."""
    K = 4096
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    print(f"shared-x SwiGLU I={I} {dt}", flush=True)
    wq, s, b = _weight(ops, 2 * I, K, seed=31 + I % 13, gs=64, dt=tdt)
    x = _x(1, K, seed=90, dt=tdt)
    got = ops.quantized_swiglu(x, wq, s, b, 64, 4)
    gu = oracle.qmv_affine(to_np(x, dt), dt, _words(wq), to_np(s, dt), to_np(b, dt), dt, 64, 4,
                           odt=dt, nthreads=NT)
    ref = as_f64(oracle.swiglu(gu, dt), dt)
    assert rel_err(as_f64(to_np(got, dt), dt), ref) <= TOL_AFFINE
