"""HIP-graph capture of the library's calls in the way bench.py and a serving
loop capture them: every call first runs once on the capture stream (which
sizes that stream's workspaces: split-K partials, fused-SwiGLU product,
grouped-gather offsets), then the calls are captured on the same stream, so
the graph holds kernel nodes only.  Each replay must equal the eager result
bit for bit.  Shapes are the bench's: the K = N = 4096 mode-sweep GEMM at
M = 256 (split K), the Llama gate_up SwiGLU at M = 1 / 4 / 16 and the
256-expert MoE block at T = 64."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from ironmlx_amd import ops as _ops
    from ironmlx_amd import _lib
    _lib.load()
    return _ops


@pytest.fixture(scope="module")
def cap_stream():
    return torch.cuda.Stream()


def _codes(gen, *shape):
    return torch.randint(-2**31, 2**31 - 1, shape, generator=gen, device="cuda",
                         dtype=torch.int32).view(torch.uint32)


def _weight(gen, lead, n, k):
    w = _codes(gen, *lead, n, k // 8)
    s = (torch.rand((*lead, n, k // 64), generator=gen, device="cuda") * 0.004 + 0.002).to(torch.bfloat16)
    b = (torch.randn((*lead, n, k // 64), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    return w, s, b


def _bits(t):
    return t.view(torch.uint16) if t.dtype in (torch.bfloat16, torch.float16) else t


def _check_warm_graph(fn, stream, reps=3):
    ref = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        outs = fn()
    for r in range(reps):
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, ref)):
            assert torch.equal(_bits(o), _bits(e)), f"replay {r}, output {i}"


def test_graph_split_k_gemm(ops, cap_stream):
    gen = torch.Generator(device="cuda").manual_seed(21)
    w, s, b = _weight(gen, (), 4096, 4096)
    x = torch.randn((256, 4096), generator=gen, device="cuda").to(torch.bfloat16)
    print("graph: split-K GEMM M=256 K=N=4096", flush=True)
    _check_warm_graph(lambda: (ops.quantized_matmul(x, w, s, b, True, 64, 4),), cap_stream)


def test_graph_fused_swiglu(ops, cap_stream):
    gen = torch.Generator(device="cuda").manual_seed(22)
    gu = _weight(gen, (), 2 * 14336, 4096)
    xs = [torch.randn((m, 4096), generator=gen, device="cuda").to(torch.bfloat16) for m in (1, 4, 16)]
    print("graph: fused SwiGLU 4096 -> 2x14336, M = 1/4/16", flush=True)
    _check_warm_graph(lambda: tuple(ops.quantized_swiglu(x, *gu, 64, 4) for x in xs), cap_stream)


def test_graph_moe_block(ops, cap_stream):
    from ironmlx_amd import nn
    gen = torch.Generator(device="cuda").manual_seed(23)
    E, H, I, k, T = 256, 2048, 512, 8, 64
    experts = {"gate_up": nn.StackedExperts(*_weight(gen, (E,), 2 * I, H)),
               "down": nn.StackedExperts(*_weight(gen, (E,), H, I))}
    moe = nn.MoEMLP(None, experts, None, None, k, True)
    logits = torch.randn((T, E), generator=gen, device="cuda").to(torch.bfloat16)
    x = torch.randn((T, H), generator=gen, device="cuda").to(torch.bfloat16)

    def block():
        sc, ex = ops.moe_route(logits, k, True)
        return (moe.experts_forward(x, sc, ex), sc, ex)

    print("graph: MoE block E=256 H=2048 I=512 k=8 T=64", flush=True)
    _check_warm_graph(block, cap_stream)


def test_graph_moe_token_and_wide_decode(ops, cap_stream):
    """The one-token MoE block (two launches, per-stream workspace for the
    SwiGLU rows and the routing) and the streaming wide-matrix kernel
    (N = 65536, M = 8) replayed from one graph."""
    from ironmlx_amd import nn
    gen = torch.Generator(device="cuda").manual_seed(26)
    E, H, I, k = 256, 2048, 512, 8
    experts = {"gate_up": nn.StackedExperts(*_weight(gen, (E,), 2 * I, H)),
               "down": nn.StackedExperts(*_weight(gen, (E,), H, I))}
    moe = nn.MoEMLP(None, experts, None, None, k, True)
    logits = torch.randn((1, E), generator=gen, device="cuda").to(torch.bfloat16)
    x1 = torch.randn((1, H), generator=gen, device="cuda").to(torch.bfloat16)
    w, s, b = _weight(gen, (), 65536, 4096)
    x8 = torch.randn((8, 4096), generator=gen, device="cuda").to(torch.bfloat16)
    print("graph: one-token MoE block + wide decode N=65536 M=8", flush=True)
    _check_warm_graph(lambda: (moe.token_forward(x1, logits), ops.quantized_matmul(x8, w, s, b, True, 64, 4)),
                      cap_stream)


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")  # the refused call enqueues nothing
def test_capture_on_unsized_stream_raises(ops):
    """Nothing is allocated during capture: on a stream whose split-K
    workspace was never sized, the captured call fails with a message (the
    request is refused before any kernel is enqueued)."""
    from ironmlx_amd._lib import IqmmError
    gen = torch.Generator(device="cuda").manual_seed(24)
    w, s, b = _weight(gen, (), 4096, 4096)
    x = torch.randn((256, 4096), generator=gen, device="cuda").to(torch.bfloat16)
    fresh = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("graph: split-K GEMM captured on an unsized stream (must raise)", flush=True)
    with pytest.raises(IqmmError, match="during graph capture"):
        with torch.cuda.graph(g, stream=fresh):
            ops.quantized_matmul(x, w, s, b, True, 64, 4)
    torch.cuda.synchronize()


def test_reserved_stream_capture_with_eager_work_between_replays(ops):
    """iqmm_workspace_reserve sizes a fresh stream's workspaces, so the calls
    captured on it hold kernel nodes only; eager allocation and
    synchronisation between replays leave every replay bit-identical."""
    from ironmlx_amd import nn
    gen = torch.Generator(device="cuda").manual_seed(25)
    w, s, b = _weight(gen, (), 4096, 4096)
    x = torch.randn((256, 4096), generator=gen, device="cuda").to(torch.bfloat16)
    gu = _weight(gen, (), 2 * 14336, 4096)
    x4 = torch.randn((4, 4096), generator=gen, device="cuda").to(torch.bfloat16)
    E, H, I, k, T = 256, 2048, 512, 8, 64
    experts = {"gate_up": nn.StackedExperts(*_weight(gen, (E,), 2 * I, H)),
               "down": nn.StackedExperts(*_weight(gen, (E,), H, I))}
    moe = nn.MoEMLP(None, experts, None, None, k, True)
    logits = torch.randn((T, E), generator=gen, device="cuda").to(torch.bfloat16)
    xm = torch.randn((T, H), generator=gen, device="cuda").to(torch.bfloat16)

    def fn():
        sc, ex = ops.moe_route(logits, k, True)
        return (ops.quantized_matmul(x, w, s, b, True, 64, 4),
                ops.quantized_swiglu(x4, *gu, 64, 4),
                moe.experts_forward(xm, sc, ex), sc, ex)

    ref = [t.clone() for t in fn()]
    stream = torch.cuda.Stream()
    ops.workspace_reserve(64 << 20, stream=stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("graph: reserved stream, split-K GEMM + SwiGLU M=4 + MoE block T=64", flush=True)
    with torch.cuda.graph(g, stream=stream):
        outs = fn()
    for r in range(3):
        junk = torch.randn(1 << 20, device="cuda") * float(r + 1)
        junk.sum().item()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, ref)):
            assert torch.equal(_bits(o), _bits(e)), f"replay {r}, output {i}"
