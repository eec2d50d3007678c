"""`torch.ops.hk_vllm.linear` on the GPU: the op vLLM's unquantized linear layers are
routed to, checked against the CPU oracle (fp32 accumulation of the same bf16 operands).

The cases of the reference's tests/hk/gpu/test_vllm_gemm.py:69-161, with this build's
table: every path the shipped routes_vllm_linear_gfx950.json names ("hk", "hk_decode",
"fallback") computes x @ W.T at Ms that land in each of its runs, and the op's counters
show which path each call took; then what a serving engine hands the op (leading batch
axes, a strided or misaligned activation, a bias, fp16) and what it does to it
(torch.compile fullgraph with a symbolic M, CUDA-graph capture and replay).

Tolerance: the path's bf16 output against the oracle's fp32, elementwise rtol = atol =
1e-2 (outputs are ~N(0, 1): weights are scaled by K^-1/2)."""

import pytest
import torch

from hk.integration import vllm_gemm as V
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
RTOL = ATOL = 1e-2


@pytest.fixture(scope="module", autouse=True)
def op():
    V.register_op()
    V.set_routes(None)          # the shipped table
    yield torch.ops.hk_vllm.linear
    V.set_routes(None)


def _xw(m, n, k, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed * 7919 + m * 31 + n + k)
    x = torch.randn(m, k, generator=g).to(dtype)
    w = (torch.randn(n, k, generator=g) * k ** -0.5).to(dtype)
    return x, w


def _took(fn):
    before = dict(V.STATS)
    out = fn()
    torch.cuda.synchronize()
    return out, {p: V.STATS[p] - before[p] for p in before}


def _check(y, x, w, bias=None):
    ref = O.gemm_fp32(x, w)
    if bias is not None:
        ref = ref + bias.float()
    O.assert_close(y.reshape(ref.shape), ref, RTOL, ATOL)


# Ms chosen to land in each run of the shipped table for these two shapes, the gaps
# between runs, and ragged counts (not a multiple of any tile).
SHAPE_MS = {
    (6144, 4096): [1, 4, 16, 17, 24, 100, 192, 256, 300, 1000],
    (4096, 12288): [1, 4, 5, 8, 64, 96, 150, 192, 256, 512, 600],
}
CASES = [(m, n, k) for (n, k), ms in SHAPE_MS.items() for m in ms]


@pytest.mark.parametrize("m,n,k", CASES)
def test_every_path_computes_x_wt(op, m, n, k):
    path = V.route_for(m, n, k)
    x, w = _xw(m, n, k)
    xd, wd = x.to(DEV), w.to(DEV)
    y, took = _took(lambda: op(xd, wd, None))
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    assert took == {p: int(p == path) for p in took}, (path, took)
    _check(y, x, w)


def test_the_cases_cover_every_path_of_the_table():
    paths = {V.route_for(m, n, k) for m, n, k in CASES}
    assert paths == {"hk", "hk_decode", "fallback"}
    # and every M up to 2048 on one shape reaches all three
    assert {V.route_for(m, 6144, 4096) for m in range(1, 2049)} == {"hk", "hk_decode", "fallback"}


def test_the_direct_call_matches_the_dispatcher(op):
    """PATCH(...) in eager code skips torch's dispatcher; both give the same bits."""
    x, w = _xw(256, 6144, 4096)
    xd, wd = x.to(DEV), w.to(DEV)
    assert torch.equal(V.PATCH(xd, wd, None), op(xd, wd, None))


def test_a_decode_batch_with_leading_axes(op):
    x, w = _xw(6, 4096, 4096)
    assert V.route_for(6, 4096, 4096) == "hk_decode"
    y, took = _took(lambda: op(x.to(DEV).view(2, 3, 4096), w.to(DEV), None))
    assert y.shape == (2, 3, 4096) and took["hk_decode"] == 1
    _check(y, x, w)


def test_a_leading_batch_axis_is_flattened_into_m(op):
    x, w = _xw(256, 6144, 4096)
    assert V.route_for(256, 6144, 4096) == "hk"
    y, took = _took(lambda: op(x.to(DEV).view(2, 128, 4096), w.to(DEV), None))
    assert y.shape == (2, 128, 6144) and took["hk"] == 1
    _check(y, x, w)


def test_a_strided_activation_is_copied_not_misread(op):
    x, w = _xw(256, 6144, 4096)
    xt = x.to(DEV).t().contiguous().t()           # the same values, column-major
    assert not xt.is_contiguous()
    y, took = _took(lambda: op(xt, w.to(DEV), None))
    assert took["hk"] == 1
    _check(y, x, w)


def test_a_misaligned_activation_is_copied(op):
    """A contiguous view that starts 2 bytes into its storage: the kernels' 16-byte loads
    would refuse it, so the op copies it first."""
    x, w = _xw(256, 6144, 4096)
    buf = torch.empty(256 * 4096 + 1, dtype=torch.bfloat16, device=DEV)
    xv = buf[1:].view(256, 4096)
    xv.copy_(x.to(DEV))
    assert xv.is_contiguous() and xv.data_ptr() % 16
    y, took = _took(lambda: op(xv, w.to(DEV), None))
    assert took["hk"] == 1
    _check(y, x, w)


def test_a_misaligned_weight_takes_the_fallback(op):
    x, w = _xw(256, 6144, 4096)
    buf = torch.empty(6144 * 4096 + 1, dtype=torch.bfloat16, device=DEV)
    wv = buf[1:].view(6144, 4096)
    wv.copy_(w.to(DEV))
    y, took = _took(lambda: op(x.to(DEV), wv, None))
    assert took["fallback"] == 1
    _check(y, x, w)


@pytest.mark.parametrize("m", [4, 256])
def test_a_bias_rides_the_fused_epilogue(op, m):
    x, w = _xw(m, 6144, 4096)
    b = (torch.randn(6144, generator=torch.Generator().manual_seed(3)) * 0.1).to(torch.bfloat16)
    path = V.route_for(m, 6144, 4096, bias=True)
    assert path in ("hk", "hk_decode")
    y, took = _took(lambda: op(x.to(DEV), w.to(DEV), b.to(DEV)))
    assert took[path] == 1
    _check(y, x, w, b)


def test_bias_takes_the_fallback_when_not_fused(op, monkeypatch):
    monkeypatch.setattr(V, "BIAS_FUSED", False)
    V.ROUTER.plans.clear()
    x, w = _xw(256, 6144, 4096)
    b = (torch.randn(6144, generator=torch.Generator().manual_seed(4)) * 0.1).to(torch.bfloat16)
    y, took = _took(lambda: op(x.to(DEV), w.to(DEV), b.to(DEV)))
    V.ROUTER.plans.clear()
    assert took["fallback"] == 1
    _check(y, x, w, b)


def test_fp16_takes_the_fallback(op):
    x, w = _xw(256, 6144, 4096, dtype=torch.float16)
    y, took = _took(lambda: op(x.to(DEV), w.to(DEV), None))
    assert took["fallback"] == 1 and y.dtype == torch.float16
    _check(y, x, w)


def test_the_patched_layer_gemm_matches_f_linear():
    class Layer:
        pass

    x, w = _xw(256, 6144, 4096)
    layer = Layer()
    y = V._layer_gemm(None, layer, x.to(DEV), w.to(DEV), None)
    assert layer._hk_route[1] == ""
    _check(y, x, w)


@pytest.mark.parametrize("m", [4, 256])
def test_it_compiles_fullgraph_with_a_symbolic_m(op, m):
    x, w = _xw(m, 6144, 4096)
    f = torch.compile(lambda a, b: op(a, b, None) * 2, fullgraph=True, dynamic=True)
    y = f(x.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    O.assert_close(y, 2 * O.gemm_fp32(x, w), RTOL, 2 * ATOL)


@pytest.mark.parametrize("m", [4, 256])
def test_it_replays_from_a_cuda_graph(op, m):
    """Captured once, replayed after the input changed (and again after eager work in
    between): each replay equals the eager result on the new input. The captured call
    counts under `captured`, not `stats`."""
    path = V.route_for(m, 6144, 4096)
    x, w = _xw(m, 6144, 4096)
    xd, wd = x.to(DEV), w.to(DEV)
    op(xd, wd, None)                              # plan and warm up before the capture
    torch.cuda.synchronize()
    cap_before = V.PATCH.captured[path]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = op(xd, wd, None)
    assert V.PATCH.captured[path] == cap_before + 1
    for seed in (1, 2):
        x2, _ = _xw(m, 6144, 4096, seed=seed)
        xd.copy_(x2.to(DEV))
        eager = op(xd, wd, None)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        _check(y, x2, w)


def test_the_graph_contract_names_the_patch():
    """Under CUDA-graph capture a graph-safe op that synchronises with the host raises
    GraphCaptureError naming it (torch's sync debug mode refuses the sync before it runs,
    so the capture itself stays valid), and a graph="never" op refuses to run at all."""
    from hk.integration import engine

    syncs = engine.Op("hk_test::syncs", "syncs(Tensor x) -> Tensor", lambda x: torch.empty_like(x),
                      paths=("a",))
    syncs.define(lambda x: x * x.sum().item())
    never = engine.Op("hk_test::never", "never(Tensor x) -> Tensor", lambda x: torch.empty_like(x),
                      paths=("a",), graph="never", why="its route reads a host-side counter")
    never.define(lambda x: x + 1)
    x = torch.ones(8, device=DEV)
    assert float(syncs(x)[0]) == 8.0 and float(never(x)[0]) == 2.0   # eager: fine
    torch.cuda.synchronize()
    for op, match in ((syncs, "hk_test::syncs synchronised"), (never, "reads a host-side")):
        g = torch.cuda.CUDAGraph()
        with pytest.raises(engine.GraphCaptureError, match=match):
            with torch.cuda.graph(g):
                op(x)
        torch.cuda.synchronize()
    assert float(syncs(x)[0]) == 8.0                                   # eager again
