"""CUDA-graph capture of the template's calls: every replay equals the eager result.

A captured graph bakes in every address its kernels touch, the split-K workspace's
included. These tests capture split-K and single-pass calls whose workspaces grow from
graph to graph, destroy the graphs and capture again (torch.cuda.graph empties the
allocator's cache before every capture), and replay each graph several times with eager
work and synchronizations in between, checking every replay against the eager output."""

import pytest
import torch

import hk

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
T = hk.templates.gemm
SPLIT = ("decode_blk", "t64k2", "t64k4", "t64k8", "t128k2")


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def test_split_k_graphs_keep_their_workspace():
    n, k = 4096, 4096
    gen = torch.Generator().manual_seed(40)
    w = (torch.randn(n, k, generator=gen) * k ** -0.5).to(torch.bfloat16).to(DEV)
    bias = torch.randn(n, generator=gen).to(torch.bfloat16).to(DEV)
    for rnd in range(2):
        for m in (1, 4, 16):
            x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(DEV)
            outs, refs, graphs = {}, {}, {}
            for sch in SPLIT:
                print(f"round {rnd} M={m} {sch}", flush=True)
                refs[sch] = T(x, w, epilogue=T.bias, bias=bias, schedule=sch).clone()
                outs[sch] = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
                graphs[sch] = _capture(lambda sch=sch: T(x, w, epilogue=T.bias, bias=bias,
                                                         out=outs[sch], schedule=sch))
            for rep in range(3):
                for sch, g in graphs.items():
                    outs[sch].fill_(7.0)
                    torch.cuda.synchronize()
                    g.replay()
                    torch.cuda.synchronize()
                    assert torch.equal(outs[sch], refs[sch]), f"{sch} M={m} replay {rep}"
            del graphs


@pytest.mark.parametrize("sched", ["t256", "t128", "t64w8", "t128n128", "decode"])
def test_single_pass_graph_replays(sched):
    m, n, k = (16, 2048, 2048) if sched == "decode" else (300, 2048, 2048)
    gen = torch.Generator().manual_seed(41)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(DEV)
    w = (torch.randn(n, k, generator=gen) * k ** -0.5).to(torch.bfloat16).to(DEV)
    bias = torch.randn(n, generator=gen).to(torch.bfloat16).to(DEV)
    ref = T(x, w, epilogue=T.bias_gelu, bias=bias, schedule=sched).clone()
    out = torch.empty_like(ref)
    g = _capture(lambda: T(x, w, epilogue=T.bias_gelu, bias=bias, out=out, schedule=sched))
    for rep in range(3):
        out.fill_(7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"


@pytest.mark.parametrize("scalar_first", [False, True])
def test_scaled_mm_with_number_scales_replays(scalar_first):
    """scaled_mm with Python-number scales under capture: the numbers become device
    tensors by a fill kernel (no host-to-device copy, which a capture refuses). Captured
    both with the scale tensors already made eagerly (scalar_first) and with the first
    sight of the numbers inside the capture; every replay equals the eager result and
    the oracle."""
    from hk.ops import gemm as G
    from oracle import gemm_oracle as O

    m, n, k = 512, 1024, 1024
    gen = torch.Generator().manual_seed(42)
    a8 = (torch.randn(m, k, generator=gen) * 4).to(torch.float8_e4m3fn)
    b8 = (torch.randn(n, k, generator=gen) * 4).to(torch.float8_e4m3fn)
    bias = (torch.randn(n, generator=gen) * 0.1).to(torch.bfloat16)
    sa, sb = 0.375 + 0.001 * scalar_first, 0.0625
    ad, bd, biasd = a8.to(DEV), b8.to(DEV), bias.to(DEV)
    G._NUMBERS.clear()
    if scalar_first:
        ref = G.scaled_mm(ad, bd, sa, sb, bias=biasd).clone()
    out = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    G.scaled_mm(ad, bd, 1.0, 1.0, bias=biasd, out=out)     # warm up with other numbers
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        G.scaled_mm(ad, bd, sa, sb, bias=biasd, out=out)
    if not scalar_first:
        assert (G._NUMBERS.keys() & {(ad.device, sa), (ad.device, sb)}) == set()
        ref = G.scaled_mm(ad, bd, sa, sb, bias=biasd).clone()
    O.assert_close(ref, O.scaled_mm(a8, b8, sa, sb, bias), rtol=3e-2, atol=1e-2)
    for rep in range(3):
        out.fill_(7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"


def test_captured_workspaces_go_with_their_graphs():
    """A split-K call captured into a graph allocates its workspace in the capture, so the
    memory belongs to the graph and goes with it: capturing and dropping graphs over and
    over (a tuner, or an engine re-capturing its batch sizes) holds no memory per captured
    call, and every replay before the drop is still right."""
    m, n, k = 16, 4096, 4096
    gen = torch.Generator().manual_seed(42)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(DEV)
    w = (torch.randn(n, k, generator=gen) * k ** -0.5).to(torch.bfloat16).to(DEV)
    ref = T(x, w, schedule="t64k8").clone()
    out = torch.empty_like(ref)

    side = torch.cuda.Stream()   # one warm-up stream: its eager workspace is cached once

    def once():
        fn = lambda: T(x, w, out=out, schedule="t64k8")  # noqa: E731
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        out.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        del g

    for _ in range(3):
        once()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    for i in range(30):
        print(f"capture {i}", flush=True)
        once()
    torch.cuda.synchronize()
    ws = 8 * m * n * 4    # one captured call's workspace: 8 fp32 shares of (M, N)
    assert torch.cuda.memory_allocated() - base < 2 * ws
