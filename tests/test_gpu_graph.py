"""HIP graph capture of the operators: each call is captured once into a
torch.cuda.CUDAGraph (stream capture of the library's launches on the current
torch stream) and the graph is replayed several times.  Before each replay the
graph's output buffer is filled with NaN by eager work on the same stream, and
after it the output must equal the eager call's output bit for bit: the kernels are
deterministic, and the library records no memset, copy or allocation of its own
(flags and counters are cleared by its own kernels), so a replay repeats exactly
what the eager call did.  The SwiGLU shape takes the tail/down launch, whose flags
and parked sums are reused by every replay; causal GQA takes the persistent
schedule; AdamW updates its buffers in place, replay after replay, against the
same number of eager steps."""
import pytest
import torch

from kda import ops

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
F32 = torch.float32
REPLAYS = 3


def _capture(fn):
    """fn() once on a side stream (one-time set-up outside the capture), then fn()
    captured into a graph; returns (graph, the output tensor the graph writes)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def _check_replays(name, fn):
    want = fn()
    torch.cuda.synchronize()
    g, out = _capture(fn)
    for r in range(REPLAYS):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        same = torch.equal(out, want)
        print(f"{name} replay {r}: equal={same}", flush=True)
        assert same, f"{name}: replay {r} differs from the eager call"
    del g


def _randn(shape, dtype, dev, gen, scale=1.0):
    return (torch.randn(shape, generator=gen, device=dev, dtype=F32) * scale).to(dtype).contiguous()


@pytest.fixture
def gen(dev):
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    return g


def test_graph_silu(dev, gen):
    x = _randn((2048, 8192), F32, dev, gen)
    _check_replays("silu", lambda: ops.silu(x))


def test_graph_rmsnorm_matmul_bf16(dev, gen):
    x = _randn((4096, 4096), BF, dev, gen)
    gamma = (1.0 + 0.1 * _randn((4096,), F32, dev, gen)).to(BF)
    w = _randn((4096, 11008), BF, dev, gen, 0.02)
    _check_replays("rmsnorm_matmul", lambda: ops.rmsnorm_matmul(x, w, gamma, 1e-6))


def test_graph_swiglu_bf16_tail_down_launch(dev, gen):
    x = _randn((2048, 4096), BF, dev, gen)
    w_up = _randn((4096, 14336), BF, dev, gen, 0.02)
    w_gate = _randn((4096, 14336), BF, dev, gen, 0.02)
    w_down = _randn((14336, 4096), BF, dev, gen, 0.02)
    _check_replays("swiglu", lambda: ops.swiglu(x, w_up, w_down, w_gate))


def test_graph_gqa_causal_persistent(dev, gen):
    q = _randn((4, 4096, 32, 128), BF, dev, gen, 128 ** -0.5)
    k = _randn((4, 4096, 8, 128), BF, dev, gen, 128 ** -0.5)
    v = _randn((4, 4096, 8, 128), BF, dev, gen, 128 ** -0.5)
    _check_replays("gqa", lambda: ops.gqa(q, k, v, causal=True))


def test_graph_nkibench_operators(dev, gen):
    a = _randn((16, 4096, 64), F32, dev, gen)
    b = _randn((16, 64, 4096), F32, dev, gen)
    _check_replays("bmm", lambda: ops.bmm(a, b))
    _check_replays("bmm_softmax", lambda: ops.bmm_softmax(a[:4], b[:4]))
    delta = torch.rand((256, 7168), generator=gen, device=dev) * 0.1
    u = _randn((256, 7168), F32, dev, gen)
    sa = -torch.rand((256, 16), generator=gen, device=dev)
    sb = _randn((16, 7168), F32, dev, gen)
    sc = _randn((16, 7168), F32, dev, gen)
    _check_replays("mamba", lambda: ops.mamba(delta, u, sa, sb, sc))
    qf = _randn((1, 1024, 16, 128), F32, dev, gen, 128 ** -0.5)
    kf = _randn((1, 1024, 8, 128), F32, dev, gen, 128 ** -0.5)
    vf = _randn((1, 1024, 8, 128), F32, dev, gen)
    _check_replays("gqa fp32", lambda: ops.gqa(qf, kf, vf))


def test_graph_adamw_step_in_place(dev, gen):
    """One captured in-place step, replayed: after each replay the buffers equal
    those of the same number of eager steps from the same start."""
    n = (1 << 22) + 3                      # the vector kernel and the scalar tail
    p0 = _randn((n,), F32, dev, gen)
    g = _randn((n,), F32, dev, gen, 0.01)
    m0 = _randn((n,), F32, dev, gen, 0.001)
    v0 = torch.rand((n,), generator=gen, device=dev) * 1e-4
    pe, me, ve = p0.clone(), m0.clone(), v0.clone()
    pg, mg, vg = p0.clone(), m0.clone(), v0.clone()
    step = lambda p, m, v: ops.adamw_step_(p, g, m, v, step=10)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):            # set-up call on scratch copies
        step(p0.clone(), m0.clone(), v0.clone())
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(pg, mg, vg)
    torch.cuda.synchronize()
    # capture does not run the kernels: the buffers still hold the start values
    assert torch.equal(pg, p0) and torch.equal(mg, m0) and torch.equal(vg, v0)
    for r in range(REPLAYS):
        step(pe, me, ve)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        same = torch.equal(pg, pe) and torch.equal(mg, me) and torch.equal(vg, ve)
        print(f"adamw replay {r}: equal={same}", flush=True)
        assert same, f"adamw: replay {r} differs from eager step {r + 1}"
