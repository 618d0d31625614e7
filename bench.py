"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline (BASELINE.json metric "4-bit qmatmul: decode GEMV HBM GB/s (%peak);
prefill TFLOP/s (%MFMA peak)"):

* value    = decode GEMV HBM GB/s: affine 4-bit gs64, K=4096, N=14336, M=1,
             bf16 x/scales/biases.  A "step" is one GEMV over each of a pool
             of distinct weight sets (> 2x the 256 MB Infinity Cache, so every
             launch streams from HBM), replayed from a HIP graph.
* prefill  = the prefill GEMM (M=2048, K=4096, N=14336, bf16) in TFLOP/s.
* roofline = the GEMV kernel's algorithmic bytes per launch / its average
             launch duration (HIP events around each launch on the stream the
             kernel runs on) against 8 TB/s; prefill likewise against the
             2.5 PFLOP/s bf16 dense MFMA peak.
* cpu_baseline = the CPU restatement of the same GEMV (oracle/, OpenMP)
             timed on this host on a bounded sample.

Inputs are synthetic (seeded), resident in HBM before timing starts.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s


def gemv_bytes(M, N, K, bits=4, gs=64, xbytes=2, sbytes=2):
    """Algorithmic bytes of one quantized GEMV: packed weight + scales + biases
    + x + out."""
    return N * K * bits // 8 + 2 * N * (K // gs) * sbytes + M * K * xbytes + M * N * xbytes


def make_weight(ops, N, K, gen, dt=torch.bfloat16, gs=64, bits=4):
    """Random packed codes + scales/biases at the scale of a quantized N(0,0.02)
    weight (quantize() of a full fp matrix per set would dominate set-up)."""
    words = torch.randint(-2**31, 2**31 - 1, (N, K * bits // 32), generator=gen, device="cuda",
                          dtype=torch.int32).view(torch.uint32)
    s = (torch.rand((N, K // gs), generator=gen, device="cuda") * 0.004 + 0.002).to(dt)
    b = (torch.randn((N, K // gs), generator=gen, device="cuda") * 0.02).to(dt)
    return words, s, b


def time_launches(fn, n, stream):
    """Average device duration of `fn` over n launches: HIP events bracket each
    launch on `stream` (the stream the kernel is enqueued on).  A spin kernel
    queued first keeps the GPU busy while the host enqueues all n launches,
    so host-side call overhead never sits between an event pair."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n)]
    torch.cuda._sleep(int(2.0e6 + 1.5e5 * n))
    for a, b in evs:
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in evs) / n * 1e-3


def bench_gemv(ops, steps, warmup, M=1, N=14336, K=4096, pool_bytes=640 << 20, dt=torch.bfloat16):
    gen = torch.Generator(device="cuda").manual_seed(0)
    per = gemv_bytes(M, N, K)
    P = max(2, int(np.ceil(pool_bytes / per)))
    pool = [make_weight(ops, N, K, gen, dt=dt) for _ in range(P)]
    x = torch.randn((M, K), generator=gen, device="cuda").to(dt)
    stream = torch.cuda.current_stream()
    outs = [None] * P

    def one_pass():
        for i, (w, s, b) in enumerate(pool):
            outs[i] = ops.quantized_matmul(x, w, s, b, True, 64, 4, "affine")

    one_pass()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        one_pass()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        g.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    total_s = t0.elapsed_time(t1) * 1e-3
    # The kernel is a few microseconds long, so an event pair around each
    # launch would time the event records too; the average launch duration is
    # the timed replays (HIP events on the launch stream) over the launches
    # they contain.  rocprofv3's kernel trace of `bench.py --only gemv` agrees.
    avg_launch_s = total_s / (steps * P)
    res = {
        "gbs": per * P * steps / total_s / 1e9,
        "ms_per_step": total_s / steps * 1e3,
        "bytes_per_launch": per,
        "pool_sets": P,
        "avg_launch_us": avg_launch_s * 1e6,
        "kernel_gbs": per / avg_launch_s / 1e9,
    }
    del pool, outs, g
    torch.cuda.empty_cache()
    return res


def bench_prefill(ops, steps, warmup, M=2048, N=14336, K=4096):
    """Average device time per prefill GEMM: n launches captured in one HIP
    graph and replayed, HIP events on the launch stream around the replays.
    The graph removes host launch overhead; what remains between kernels is
    the GPU's own dispatch gap, so the figure is within a few percent of
    rocprofv3's per-kernel average."""
    gen = torch.Generator(device="cuda").manual_seed(1)
    w, s, b = make_weight(ops, N, K, gen)
    x = torch.randn((M, K), generator=gen, device="cuda").to(torch.bfloat16)
    stream = torch.cuda.current_stream()
    n = max(3, steps)
    outs = [None] * n

    def run():
        for i in range(n):
            outs[i] = ops.quantized_matmul(x, w, s, b, True, 64, 4, "affine")

    run()
    # split-K shapes keep fp32 partials in the capture stream's workspace,
    # sized by an eager pass on it (nothing is allocated while capturing)
    _warm_on_capture_stream(run)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=_capture_stream()):
        run()
    for _ in range(max(1, warmup)):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    g.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    avg = t0.elapsed_time(t1) * 1e-3 / n
    flops = 2.0 * M * N * K
    del g, outs
    # isolated kernel duration: HIP events around each launch on the launch
    # stream (the kernels queue behind a spin kernel, so no host gap is timed);
    # this is what rocprofv3's per-kernel average measures
    iso = time_launches(lambda: ops.quantized_matmul(x, w, s, b, True, 64, 4, "affine"), n, stream)
    torch.cuda.empty_cache()
    return {"tflops": flops / avg / 1e12, "avg_launch_us": avg * 1e6, "flops_per_launch": flops,
            "kernel_us": iso * 1e6, "kernel_tflops": flops / iso / 1e12}


def bench_moe(ops, Ts=(1, 64, 512), reps=10):
    """Qwen3.5-MoE-style gather_qmm: 256 experts, top-8 of softmax(N(0,1)
    logits); gate (and up) 2048 -> 512 and down 512 -> 2048, q4 gs64, bf16.
    GB/s counts the bytes of the experts the sampled routing touches (plus x
    and out)."""
    E, H, I, k = 256, 2048, 512, 8
    gen = torch.Generator(device="cuda").manual_seed(3)

    def stack(n, kk):
        w = torch.randint(-2**31, 2**31 - 1, (E, n, kk // 8), generator=gen, device="cuda",
                          dtype=torch.int32).view(torch.uint32)
        s = (torch.rand((E, n, kk // 64), generator=gen, device="cuda") * 0.004 + 0.002).to(torch.bfloat16)
        b = (torch.randn((E, n, kk // 64), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
        return w, s, b

    gate, down = stack(I, H), stack(H, I)
    per_expert = I * H // 2 + 2 * I * (H // 64) * 2   # one projection's bytes
    stream = torch.cuda.current_stream()
    out = {}
    for T in Ts:
        logits = torch.randn((T, E), generator=gen, device="cuda")
        idx = torch.topk(torch.softmax(logits, -1), k, dim=-1).indices.to(torch.int32)
        x = torch.randn((T, H), generator=gen, device="cuda").to(torch.bfloat16)
        h = torch.randn((T * k, 1, I), generator=gen, device="cuda").to(torch.bfloat16)
        uniq = int(torch.unique(idx).numel())
        if T == 1:
            xin, hin, rhs, srt = x.view(T, 1, 1, H), h.view(T, k, 1, I), idx, False
        else:
            flat = idx.view(-1)
            order = torch.argsort(flat, stable=True)
            xin, hin = x[order // k].view(T * k, 1, H).contiguous(), h
            rhs, srt = flat[order].contiguous(), True
        res = {"unique_experts": uniq, "path": "sorted grouped" if srt else "per-token"}
        for name, (w, s, b), inp, n_out, kk in (("gate", gate, xin, I, H), ("down", down, hin, H, I)):
            fn = lambda: ops.gather_qmm(inp, w, s, b, None, rhs, True, 64, 4, "affine", srt)  # noqa: E731
            fn()
            torch.cuda.synchronize()
            dt = time_launches(fn, reps, stream)
            nbytes = uniq * per_expert + T * k * (kk + n_out) * 2
            res[name] = {"us": round(dt * 1e6, 2), "gbs": round(nbytes / dt / 1e9, 1),
                         "tflops": round(2.0 * T * k * n_out * kk / dt / 1e12, 2)}
        out[str(T)] = res
    return out


_CAPTURE_STREAM = None


def _capture_stream():
    """One stream for every capture, warmed up before capturing: the library
    keeps its per-stream workspaces (split-K partials, fused-SwiGLU product,
    grouped-gather offsets), so captured calls reuse them instead of adding
    allocation nodes to the graph."""
    global _CAPTURE_STREAM
    if _CAPTURE_STREAM is None:
        _CAPTURE_STREAM = torch.cuda.Stream()
    return _CAPTURE_STREAM


def _warm_on_capture_stream(fn):
    s = _capture_stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    s.synchronize()


def graph_time(fn, n):
    """Average device time of fn() over n calls captured in one HIP graph."""
    fn()
    _warm_on_capture_stream(fn)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=_capture_stream()):
        for _ in range(n):
            fn()
    g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1e-3 / n


def bench_decode_widths(ops, shapes=((14336, 4096), (6144, 4096), (4096, 14336), (4096, 4096)),
                        Ms=(2, 4, 8, 16, 24, 32), steps=10, warmup=2):
    """Decode batch widths of the 4-bit gs64 path on the Llama-3-8B projection
    shapes (gate/up, fused q/k/v, down, o): per-launch time over a rotating
    weight pool (graph replay, as the M = 1 headline), weight GB/s and
    TFLOP/s."""
    out = {}
    for N, K in shapes:
        row = {}
        for M in Ms:
            r = bench_gemv(ops, steps, warmup, M=M, N=N, K=K)
            row[str(M)] = {"us": round(r["avg_launch_us"], 2), "gbs": round(r["kernel_gbs"], 1),
                           "tflops": round(2.0 * M * N * K / (r["avg_launch_us"] * 1e-6) / 1e12, 1)}
        out[f"N{N}_K{K}"] = row
    return out


def bench_mode_sweep(ops, K=4096, N=4096, Ms=(1, 256), n=20):
    """Mode / bit-width sweep at K = N = 4096: weights ~N(0, 0.02) quantized by
    the library's own quantize for each mode, bf16 x; M = 1 reports weight GB/s,
    M = 256 TFLOP/s."""
    gen = torch.Generator(device="cuda").manual_seed(5)
    wf = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    cases = [("affine", b, g) for b in (2, 3, 4, 6, 8) for g in (32, 64, 128)]
    cases += [("mxfp4", 4, 32), ("mxfp8", 8, 32), ("nvfp4", 4, 16)]
    out = {}
    for mode, bits, gs in cases:
        aff = mode == "affine"
        wq, sq, bq = ops.quantize(wf, gs if aff else None, bits if aff else None, mode)
        wbytes = wq.numel() * 4 + sq.numel() * sq.element_size() * (2 if aff else 1)
        row = {}
        for M in Ms:
            x = torch.randn((M, K), generator=gen, device="cuda").to(torch.bfloat16)
            fn = lambda: ops.quantized_matmul(x, wq, sq, bq, True, gs if aff else None,  # noqa: E731
                                              bits if aff else None, mode)
            dt = graph_time(fn, n)
            row[str(M)] = ({"us": round(dt * 1e6, 2), "gbs": round(wbytes / dt / 1e9, 1)} if M == 1
                           else {"us": round(dt * 1e6, 2), "tflops": round(2.0 * M * N * K / dt / 1e12, 1)})
        out[f"{mode}{bits}" + (f"_gs{gs}" if aff else "")] = row
    return out


def bench_llama_decode(ops, Ms=(1, 4, 8, 16, 32), steps=5):
    """Llama-3-8B-shaped decode step: 32 layers x {q,k,v,o,gate,up,down} of
    distinct 4-bit gs64 weights; tokens/s = M / step time.  gate and up are
    the two row halves of one stacked [2 x 14336, 4096] weight, so the same
    bytes also run the fused-MLP step (q, k, v, o, quantized_swiglu(gate_up),
    down: six calls per layer instead of seven plus silu * up), and with q, k,
    v stacked into one weight the fused-QKV-and-MLP step (four calls)."""
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (2 * 14336, 4096), (4096, 14336)]
    gen = torch.Generator(device="cuda").manual_seed(2)
    layers = [[make_weight(ops, N, K, gen) for (N, K) in shapes] for _ in range(32)]
    wbytes = sum(w.numel() * 4 + s.numel() * 2 * 2 for L in layers for (w, s, b) in L)
    I = 14336
    # the fused-QKV variant reads the same bytes from one stacked weight per layer
    qkv = [tuple(torch.cat([L[i][j] for i in range(3)], dim=0) for j in range(3)) for L in layers]
    out = {}
    stream = torch.cuda.current_stream()
    for M in Ms:
        xs = {K: torch.randn((M, K), generator=gen, device="cuda").to(torch.bfloat16)
              for K in (4096, 14336)}
        h = torch.randn((M, I), generator=gen, device="cuda").to(torch.bfloat16)

        def step_unfused():
            for L in layers:
                for (w, s, b) in L[:4]:
                    ops.quantized_matmul(xs[4096], w, s, b, True, 64, 4, "affine")
                w, s, b = L[4]
                ops.quantized_matmul(xs[4096], w[:I], s[:I], b[:I], True, 64, 4, "affine")
                ops.quantized_matmul(xs[4096], w[I:], s[I:], b[I:], True, 64, 4, "affine")
                w, s, b = L[5]
                ops.quantized_matmul(xs[14336], w, s, b, True, 64, 4, "affine")

        def step_fused():
            for L in layers:
                for (w, s, b) in L[:4]:
                    ops.quantized_matmul(xs[4096], w, s, b, True, 64, 4, "affine")
                w, s, b = L[4]
                ops.quantized_swiglu(xs[4096], w, s, b, 64, 4)
                w, s, b = L[5]
                ops.quantized_matmul(h, w, s, b, True, 64, 4, "affine")

        def step_fused_qkv():
            # q, k, v stacked row-wise (one [6144, 4096] weight per layer: the
            # first three weights of a layer are contiguous row blocks of it)
            for L, QKV in zip(layers, qkv):
                ops.quantized_matmul(xs[4096], *QKV, True, 64, 4, "affine")
                w, s, b = L[3]
                ops.quantized_matmul(xs[4096], w, s, b, True, 64, 4, "affine")
                w, s, b = L[4]
                ops.quantized_swiglu(xs[4096], w, s, b, 64, 4)
                w, s, b = L[5]
                ops.quantized_matmul(h, w, s, b, True, 64, 4, "affine")

        row = {}
        for name, step in (("", step_unfused), ("fused_mlp_", step_fused), ("fused_qkv_mlp_", step_fused_qkv)):
            step()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step()
            g.replay()
            torch.cuda.synchronize()
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record(stream)
            for _ in range(steps):
                g.replay()
            t1.record(stream)
            torch.cuda.synchronize()
            dt = t0.elapsed_time(t1) * 1e-3 / steps
            row[name + "ms_per_step"] = dt * 1e3
            row[name + "tokens_per_s"] = M / dt
            row[name + "weight_gbs"] = wbytes / dt / 1e9
            del g
        out[str(M)] = row
    del layers, qkv
    torch.cuda.empty_cache()
    return out


def _graph_layers(fns, reps=5, inner=1):
    """Average device time of one pass over fns: `inner` passes are captured in
    one graph (so the graph's own launch cost, ~10 us, is spread over them)
    and the graph is replayed `reps` times."""
    def step():
        for _ in range(inner):
            for f in fns:
                f()
    step()
    _warm_on_capture_stream(step)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=_capture_stream()):
        step()
    g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    del g
    return t0.elapsed_time(t1) * 1e-3 / (reps * inner)


def bench_fused(ops, Ms=(1, 4, 16), layers=32):
    """The caller-side paths around the quantized ops, each against the
    composition it replaces:
    * Llama-3-8B MLP gate + up (4096 -> 2 x 14336, q4 gs64): two
      quantized_matmul + silu * up (mlx/src/nn/mlp.rs:27-33) vs one fused
      quantized_swiglu, over `layers` distinct weights (HIP-graph replay);
    * Qwen3.5-MoE expert block (E=256, top-8, 2048 -> 2 x 512 -> 2048):
      routing + sort + fused gate_up gather + down gather + combine, all on
      the device, vs the same with torch softmax / topk / argsort / index_add
      and split gate / up gathers;
    * quantized embedding (vocab 128256 x 4096): row gather vs full-table
      dequantize + index_select (mlx/src/nn/embedding.rs:62-72)."""
    import torch.nn.functional as F
    from ironmlx_amd import nn
    gen = torch.Generator(device="cuda").manual_seed(6)
    out = {}
    H, I = 4096, 14336
    gu = [make_weight(ops, 2 * I, H, gen) for _ in range(layers)]
    wbytes = gu[0][0].numel() * 4 + gu[0][1].numel() * 4
    mlp = {}
    for M in Ms:
        x = torch.randn((M, H), generator=gen, device="cuda").to(torch.bfloat16)
        def unfused():
            fs = []
            for (wq, sq, bq) in gu:
                def f(wq=wq, sq=sq, bq=bq):
                    g = ops.quantized_matmul(x, wq[:I], sq[:I], bq[:I], True, 64, 4)
                    u = ops.quantized_matmul(x, wq[I:], sq[I:], bq[I:], True, 64, 4)
                    return F.silu(g) * u
                fs.append(f)
            return fs
        fused = [lambda wq=wq, sq=sq, bq=bq: ops.quantized_swiglu(x, wq, sq, bq, 64, 4) for (wq, sq, bq) in gu]
        tu = _graph_layers(unfused()) / layers
        tf = _graph_layers(fused) / layers
        mlp[str(M)] = {"unfused_us": round(tu * 1e6, 2), "fused_us": round(tf * 1e6, 2),
                       "fused_weight_gbs": round(wbytes / tf / 1e9, 1)}
    out["llama_gate_up_swiglu"] = mlp
    del gu
    torch.cuda.empty_cache()

    E, Hm, Im, k = 256, 2048, 512, 8
    def stack(n, kk):
        w = torch.randint(-2**31, 2**31 - 1, (E, n, kk // 8), generator=gen, device="cuda",
                          dtype=torch.int32).view(torch.uint32)
        sc = (torch.rand((E, n, kk // 64), generator=gen, device="cuda") * 0.004 + 0.002).to(torch.bfloat16)
        bi = (torch.randn((E, n, kk // 64), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
        return w, sc, bi
    gu_w, down_w = stack(2 * Im, Hm), stack(Hm, Im)
    fused_ex = {"gate_up": nn.StackedExperts(*gu_w), "down": nn.StackedExperts(*down_w)}
    split_ex = {"gate": nn.StackedExperts(gu_w[0][:, :Im].contiguous(), gu_w[1][:, :Im].contiguous(),
                                          gu_w[2][:, :Im].contiguous()),
                "up": nn.StackedExperts(gu_w[0][:, Im:].contiguous(), gu_w[1][:, Im:].contiguous(),
                                        gu_w[2][:, Im:].contiguous()),
                "down": nn.StackedExperts(*down_w)}
    moe = {}
    for T in (1, 64, 512):
        logits = torch.randn((T, E), generator=gen, device="cuda").to(torch.bfloat16)
        x = torch.randn((T, Hm), generator=gen, device="cuda").to(torch.bfloat16)
        dev = nn.MoEMLP(None, fused_ex, None, None, k, True)

        def on_device():
            sc, ex = ops.moe_route(logits, k, True)
            return dev.experts_forward(x, sc, ex)

        def torch_routing():
            p = torch.softmax(logits.float(), -1)
            sc, ex = torch.topk(p, k, -1)
            sc = sc / sc.sum(-1, keepdim=True)
            flat = ex.reshape(-1)
            order = torch.argsort(flat, stable=True)
            rhs = flat[order].to(torch.int32)
            xs = x[order // k].reshape(T * k, 1, Hm)
            g = ops.gather_qmm(xs, split_ex["gate"].weight, split_ex["gate"].scales, split_ex["gate"].biases,
                               None, rhs, True, 64, 4, "affine", True)
            u = ops.gather_qmm(xs, split_ex["up"].weight, split_ex["up"].scales, split_ex["up"].biases,
                               None, rhs, True, 64, 4, "affine", True)
            h = (F.silu(g) * u).contiguous()
            y = ops.gather_qmm(h, split_ex["down"].weight, split_ex["down"].scales, split_ex["down"].biases,
                               None, rhs, True, 64, 4, "affine", True).reshape(T * k, -1)
            o = torch.zeros((T, Hm), dtype=torch.float32, device="cuda")
            o.index_add_(0, order // k, y.float() * sc.reshape(-1)[order].unsqueeze(-1))
            return o

        td = _graph_layers([on_device], reps=10, inner=16 if T == 1 else 4)
        tt = _graph_layers([torch_routing], reps=10, inner=16 if T == 1 else 4)
        moe[str(T)] = {"device_routing_fused_us": round(td * 1e6, 2), "torch_routing_split_us": round(tt * 1e6, 2)}
        if T == 1:
            # route + experts + combine of one token in two launches (ops.moe_token)
            tk = _graph_layers([lambda: dev.token_forward(x, logits)], reps=10, inner=16)
            moe[str(T)]["one_token_kernels_us"] = round(tk * 1e6, 2)
    out["qwen_moe_expert_block"] = moe
    del gu_w, down_w, fused_ex, split_ex
    torch.cuda.empty_cache()

    V, Hd = 128256, 4096
    ew, es, eb = make_weight(ops, V, Hd, gen)
    emb = {}
    for T in (1, 512):
        tok = torch.randint(0, V, (T,), generator=gen, device="cuda")
        tg = _graph_layers([lambda: ops.dequantize_rows(ew, es, eb, tok, 64, 4)], reps=10, inner=16)
        tf = _graph_layers([lambda: ops.dequantize(ew, es, eb, 64, 4).index_select(0, tok)], reps=3)
        emb[str(T)] = {"row_gather_us": round(tg * 1e6, 2), "full_table_dequant_us": round(tf * 1e6, 2)}
    # dequantize alone: packed codes + scales / biases in, bf16 out
    td = _graph_layers([lambda: ops.dequantize(ew, es, eb, 64, 4)], reps=5)
    dbytes = V * Hd // 2 + V * (Hd // 64) * 4 + V * Hd * 2
    emb["dequantize_table"] = {"us": round(td * 1e6, 2), "gbs": round(dbytes / td / 1e9, 1),
                               "hbm_frac": round(dbytes / td / 1e9 / HBM_PEAK_GBS, 3)}
    out["embedding_lookup_vocab128256_h4096"] = emb
    del ew, es, eb
    torch.cuda.empty_cache()
    return out


def _time_cpu_gemv(oracle, args, threads, seconds):
    for _ in range(2):
        oracle.qmv_affine(*args, nthreads=threads)
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 5 or time.perf_counter() < t_end:
        t = time.perf_counter()
        oracle.qmv_affine(*args, nthreads=threads)
        times.append(time.perf_counter() - t)
        if len(times) >= 400:
            break
    return float(np.median(times)), len(times)


def cpu_baseline(seconds=10.0, N=14336, K=4096):
    """The oracle's streaming GEMV (oracle/iqmm_oracle.c iqo_qmv_affine) on the
    host, same shape as the headline, timed at one thread and at the host
    threads this process may use (the CPU share a GPU box grants a one-GPU
    job: OMP_NUM_THREADS, at most the CPUs in the affinity mask); a bounded
    sample of about `seconds` each, median of the timed calls."""
    import oracle
    host_cpus = os.cpu_count() or 1
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host_cpus
    threads = max(1, min(avail, int(os.environ.get("OMP_NUM_THREADS", "0") or avail)))
    rng = np.random.default_rng(0)
    w = rng.integers(0, 2**32, (N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = oracle.from_float((rng.random((N, K // 64)) * 0.004 + 0.002).astype(np.float32), "bf16")
    b = oracle.from_float((rng.standard_normal((N, K // 64)) * 0.02).astype(np.float32), "bf16")
    x = oracle.from_float(rng.standard_normal((1, K)).astype(np.float32), "bf16")
    args = (x, "bf16", w, s, b, "bf16", 64, 4)
    nbytes = gemv_bytes(1, N, K)
    med1, n1 = _time_cpu_gemv(oracle, args, 1, seconds)
    medn, nn = _time_cpu_gemv(oracle, args, threads, seconds)
    return {"value": nbytes / medn / 1e9, "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{nn} GEMVs K={K} N={N} M=1 q4 gs64 bf16 at {threads} threads (median "
                      f"{medn * 1e3:.2f} ms), by the oracle's OpenMP streaming qmv "
                      "(MLX-CPU-semantics restatement)",
            "single_thread": {"value": nbytes / med1 / 1e9, "unit": "GB/s", "cores": 1,
                              "sample": f"{n1} GEMVs, median {med1 * 1e3:.2f} ms"},
            "host_cpus": host_cpus, "affinity_cpus": avail}


def run_only(ops, args):
    """Single-workload mode for profiler passes.  "copy" moves a known number
    of bytes with a plain device copy, the calibration point for the HBM
    FETCH_SIZE / WRITE_SIZE counters."""
    if args.only == "gemv":
        r = bench_gemv(ops, args.steps, args.warmup)
        return {"only": "gemv", **{k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}}
    if args.only == "prefill":
        r = bench_prefill(ops, args.steps, args.warmup)
        return {"only": "prefill", **{k: round(v, 3) for k, v in r.items()}}
    if args.only == "moe":
        return {"only": "moe", **bench_moe(ops)}
    if args.only == "sweep":
        return {"only": "sweep", **bench_mode_sweep(ops)}
    if args.only == "fused":
        return {"only": "fused", **bench_fused(ops)}
    if args.only == "llama":
        return {"only": "llama", **bench_llama_decode(ops)}
    if args.only == "widths":
        return {"only": "widths", **bench_decode_widths(ops)}
    if args.only == "decode":
        # the decode-width kernel at the Llama-3-8B gate/up and down shapes
        res = {}
        for (N, K, M) in ((14336, 4096, 16), (14336, 4096, 32), (4096, 14336, 16)):
            r = bench_gemv(ops, args.steps, args.warmup, M=M, N=N, K=K)
            res[f"M{M}_N{N}_K{K}"] = {"us": round(r["avg_launch_us"], 2), "gbs": round(r["kernel_gbs"], 1),
                                      "bytes_per_launch": r["bytes_per_launch"]}
        return {"only": "decode", **res}
    if args.only == "moe512":
        return {"only": "moe512", **bench_moe(ops, Ts=(512,))}
    nbytes = 256 << 20
    a = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(max(1, args.steps)):
        b.copy_(a)
    torch.cuda.synchronize()
    return {"only": "copy", "bytes_read_per_copy": nbytes, "bytes_written_per_copy": nbytes,
            "copies": max(1, args.steps)}


def load_traffic():
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return {}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-llama", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-widths", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", choices=["gemv", "prefill", "moe", "sweep", "fused", "llama", "widths", "decode", "moe512", "copy"], default=None,
                    help="run one workload (for rocprofv3 kernel-trace / counter passes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("RANK", "0")) != 0:
        return
    from ironmlx_amd import ops, _lib
    _lib.load()
    torch.cuda.set_device(0)
    if args.only is not None:
        print(json.dumps(run_only(ops, args)), flush=True)
        return

    gemv = bench_gemv(ops, args.steps, args.warmup)
    prefill = bench_prefill(ops, args.steps, args.warmup)
    prefill_down = bench_prefill(ops, args.steps, args.warmup, N=4096, K=14336)
    moe = bench_moe(ops)
    sweep = None if args.no_sweep else bench_mode_sweep(ops)
    widths = None if args.no_widths else bench_decode_widths(ops)
    llama = None if args.no_llama else bench_llama_decode(ops)
    fused = bench_fused(ops)
    # tied lm_head of Llama-3-8B (LinearLayer::from_weights on model.embed_tokens,
    # mlx/src/model/llama.rs:158-162): the largest GEMV of a decode step
    lmh = bench_gemv(ops, max(3, args.steps // 4), args.warmup, M=1, N=128256, K=4096)
    # configs[0]'s shape on the GPU (the reference's own CPU case): fp16 x and
    # scales, N = 11008
    c1 = bench_gemv(ops, args.steps, args.warmup, M=1, N=11008, K=4096, dt=torch.float16)
    tr = load_traffic()
    traffic = tr.get("gemv_q4_gs64_k4096_n14336_m1", {}).get("traffic_bytes")
    traffic_pf = tr.get("prefill_q4_gs64_m2048_k4096_n14336", {}).get("traffic_bytes")
    line = {
        "metric": "4-bit qmatmul: decode GEMV HBM GB/s (%peak); prefill TFLOP/s (%MFMA peak)",
        "value": round(gemv["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gemv["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random 4-bit codes, bf16 scales/biases, x~N(0,1))",
        "config": {"workload": "decode GEMV affine q4 gs64 K=4096 N=14336 M=1 bf16, "
                               f"{gemv['pool_sets']} distinct weight sets per step "
                               "(HIP-graph replay)",
                   "K": 4096, "N": 14336, "M": 1, "group_size": 64, "bits": 4,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gemv["kernel_gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gemv["kernel_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "bytes_per_launch": gemv["bytes_per_launch"],
                     "avg_launch_us": round(gemv["avg_launch_us"], 3)},
        "prefill": {"workload": "prefill GEMM affine q4 gs64 M=2048 K=4096 N=14336 bf16",
                    "value": round(prefill["kernel_tflops"], 2), "unit": "TFLOP/s",
                    "avg_launch_us": round(prefill["kernel_us"], 2),
                    "graph_replay_avg_launch_us": round(prefill["avg_launch_us"], 2),
                    "roofline": {"bound": "mfma", "achieved": round(prefill["kernel_tflops"], 2),
                                 "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(prefill["kernel_tflops"] / BF16_PEAK_TFLOPS, 4),
                                 "avg_launch_us": round(prefill["kernel_us"], 2),
                                 "traffic": traffic_pf},
                    "down_proj_K14336_N4096_tflops": round(prefill_down["kernel_tflops"], 2),
                    "down_proj_avg_launch_us": round(prefill_down["kernel_us"], 2)},
        "moe_gather_qmm": moe,
        "lm_head_gemv_n128256_k4096_m1": {"us": round(lmh["avg_launch_us"], 2),
                                          "gbs": round(lmh["kernel_gbs"], 1),
                                          "hbm_frac": round(lmh["kernel_gbs"] / HBM_PEAK_GBS, 4),
                                          "bytes_per_launch": lmh["bytes_per_launch"]},
        "c1_gemv_fp16_n11008_k4096_m1": {"us": round(c1["avg_launch_us"], 2),
                                         "gbs": round(c1["kernel_gbs"], 1),
                                         "hbm_frac": round(c1["kernel_gbs"] / HBM_PEAK_GBS, 4),
                                         "bytes_per_launch": c1["bytes_per_launch"]},
        "fused_paths": fused,
    }
    if sweep is not None:
        line["mode_sweep_k4096_n4096"] = sweep
    if widths is not None:
        line["decode_widths_q4_gs64"] = widths
    if llama is not None:
        line["llama3_8b_decode"] = llama
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
