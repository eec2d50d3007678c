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
