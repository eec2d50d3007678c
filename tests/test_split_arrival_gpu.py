"""K splits finished in the kernel: each workgroup stores its fp32 share and arrives at its
block's (decode) or tile's (4-wave tile kernel) counter; the last to arrive sums the shares
in split order, applies the epilogue and resets the counter (the reference's decode split,
python/hk/ops/decode_gemm.py:155-170, 283-298, and stream-K fix-up,
python/hk/ops/gemm_cdna.py:421-496). Against the CPU oracle: back-to-back calls on the
same counters with new inputs, ragged M and N, the kernels' tile and block shapes, the
fused epilogue forms; the counters are zero after every call; the two-launch form (no
counters) gives the same values; and a captured graph replayed with new inputs uses the
counters made by the eager warm-up."""

import ctypes

import pytest
import torch

from hk import _native as nat
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _data(m, n, k, seed):
    g = torch.Generator().manual_seed(seed * 7919 + m * 31 + n + k)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    b = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    r = torch.randn(m, n, generator=g).to(torch.bfloat16)
    return a, b, bias, r


def _ep(form, bias, r):
    ep = nat.HkxEpilogue()
    ep.cmul = 1.0
    ep.col_scale = ep.row_scale = ep.row_add = ep.tile_add = -1
    if form == "none":
        ep.form = nat.EP_NONE
        return ep, []
    ep.form = nat.EP_FUSED
    ops = []
    if form in ("bias", "bias_gelu"):
        ops.append((bias, nat.ROW, 1))
        ep.row_add = 0
        if form == "bias_gelu":
            ep.act = nat.ACT_GELU_TANH
    if form == "residual":
        ops.append((r, nat.TILE, r.stride(0)))
        ep.tile_add = 0
    ep.nops = len(ops)
    for i, (t, kind, ld) in enumerate(ops):
        ep.ops[i] = nat.HkxOperand(t.data_ptr(), kind, nat.dtype_code(t.dtype), ld)
    return ep, ops


def _ref(form, a, b, bias, r):
    acc = O.gemm_fp32(a, b)
    if form == "none":
        return acc
    if form == "bias":
        return O.apply_epilogue("bias", acc, bias=bias)
    if form == "bias_gelu":
        return O.gelu_tanh(acc + bias.float())
    return acc + r.float()


def _args(a, b, c, ep, waves, rows, splits):
    return nat.gemm_args(a, b, c, kernel=nat.KERNEL_DECODE, decode_waves=waves,
                         decode_rows=rows, splits=splits, ep=ep)


def _launch(args, with_counters):
    """hkx_gemm with the workspace and, or not, the per-stream counters (nat.counters)."""
    L = nat.lib()
    need = L.hkx_gemm_workspace(ctypes.byref(args))
    ws = nat.workspace(torch.device(DEV), need)
    args.ws, args.ws_bytes = ws.data_ptr(), ws.numel() * 4
    cnt = None
    if with_counters:
        ncnt = L.hkx_gemm_counters(ctypes.byref(args))
        assert ncnt > 0
        cnt = nat.counters(torch.device(DEV), ncnt)
        assert cnt is not None, "no counters made before this capture"
        args.counters, args.counters_len = cnt.data_ptr(), cnt.numel()
    nat.check(L.hkx_gemm(ctypes.byref(args), ctypes.c_void_p(nat.stream_of(torch.device(DEV)))))
    return cnt


CASES = [  # m, n, k, waves, rows, splits
    (1, 4096, 12288, 8, 16, 4), (16, 4096, 12288, 8, 16, 4), (16, 4100, 14336, 16, 16, 7),
    (5, 1000, 4096, 4, 32, 2), (32, 2048, 8192, 8, 16, 8), (24, 520, 2048, 8, 32, 3),
    (3, 16, 1024, 8, 16, 8)]


@pytest.mark.parametrize("form", ["none", "bias", "bias_gelu", "residual"])
@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}x{c[1]}x{c[2]}w{c[3]}r{c[4]}s{c[5]}" for c in CASES])
def test_split_decode_finishes_in_the_kernel(case, form):
    m, n, k, waves, rows, splits = case
    print(f"case: arrival M={m} N={n} K={k} waves={waves} rows={rows} splits={splits} {form}",
          flush=True)
    for call in range(2):  # back to back on the same counters, new inputs
        a, b, bias, r = _data(m, n, k, seed=call)
        ad, bd, biasd, rd = a.to(DEV), b.to(DEV), bias.to(DEV), r.to(DEV)
        c = torch.full((m, n + 8), 7.0, dtype=torch.bfloat16, device=DEV)
        ep, _keep = _ep(form, biasd, rd)
        args = _args(ad, bd, c[:, :n], ep, waves, rows, splits)
        cnt = _launch(args, with_counters=True)
        torch.cuda.synchronize()
        want = _ref(form, a, b, bias, r)
        O.assert_close(c[:, :n], want, rtol=1e-2, atol=1e-2)
        assert (c[:, n:].float() == 7.0).all()
        assert int(cnt.abs().sum()) == 0, "a counter was left non-zero"
        # the two-launch form (shares, then the reduction pass) gives the same values
        c2 = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
        ep2, _keep2 = _ep(form, biasd, rd)
        _launch(_args(ad, bd, c2, ep2, waves, rows, splits), with_counters=False)
        torch.cuda.synchronize()
        assert torch.equal(c[:, :n], c2)


def test_counters_are_asked_only_for_split_unpaired_decode():
    L = nat.lib()
    a = torch.empty(16, 4096, dtype=torch.bfloat16)
    b = torch.empty(4100, 4096, dtype=torch.bfloat16)
    c = torch.empty(16, 4100, dtype=torch.bfloat16)
    args = nat.gemm_args(a, b, c, kernel=nat.KERNEL_DECODE, splits=4)
    assert L.hkx_gemm_counters(ctypes.byref(args)) == (4100 + 15) // 16
    args.decode_rows = 32
    assert L.hkx_gemm_counters(ctypes.byref(args)) == (4100 + 31) // 32
    args.splits = 1
    assert L.hkx_gemm_counters(ctypes.byref(args)) == 0


def test_captured_graph_replays_with_the_warm_up_counters():
    m, n, k, splits = 16, 4096, 12288, 4
    a, b, bias, r = _data(m, n, k, seed=5)
    ad, bd, biasd = a.to(DEV), b.to(DEV), bias.to(DEV)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    ep, _keep = _ep("bias", biasd, None)

    def call():
        nat.run(_args(ad, bd, c, ep, 8, 16, splits), torch.device(DEV))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()  # eager warm-up: makes the device's graph counters
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    gcnt = nat._CNT_GRAPH[torch.device(DEV)]
    for rep in range(3):
        a2, b2, bias2, _ = _data(m, n, k, seed=10 + rep)
        ad.copy_(a2.to(DEV))
        bd.copy_(b2.to(DEV))
        biasd.copy_(bias2.to(DEV))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        O.assert_close(c, O.apply_epilogue("bias", O.gemm_fp32(a2, b2), bias=bias2),
                       rtol=1e-2, atol=1e-2)
        assert int(gcnt.abs().sum()) == 0
        call()  # eager work between the replays
        torch.cuda.synchronize()


TILE_CASES = [  # m, n, k, tile_m, tile_n, schedule, splits
    (128, 4096, 4096, 64, 128, nat.TILE_W4, 2), (128, 1000, 4096, 64, 128, nat.TILE_W4, 8),
    (300, 2048, 3072, 128, 128, nat.TILE_W4, 3), (64, 512, 8192, 64, 256, nat.TILE_W4, 4),
    (257, 768, 2048, 128, 256, nat.TILE_RING, 2), (16, 4100, 14336, 64, 128, nat.TILE_W4, 7)]


def _tile_args(a, b, c, ep, tm, tn, sched, splits):
    return nat.gemm_args(a, b, c, kernel=nat.KERNEL_TILE, tile_m=tm, tile_n=tn,
                         schedule=sched, splits=splits, ep=ep)


@pytest.mark.parametrize("form", ["none", "bias", "bias_gelu", "residual"])
@pytest.mark.parametrize("case", TILE_CASES,
                         ids=[f"{c[0]}x{c[1]}x{c[2]}t{c[3]}x{c[4]}s{c[5]}k{c[6]}" for c in TILE_CASES])
def test_split_tiles_finish_in_the_kernel(case, form):
    m, n, k, tm, tn, sched, splits = case
    print(f"case: tile arrival M={m} N={n} K={k} tile {tm}x{tn} sched {sched} splits {splits} {form}",
          flush=True)
    for call in range(2):
        a, b, bias, r = _data(m, n, k, seed=20 + call)
        ad, bd, biasd, rd = a.to(DEV), b.to(DEV), bias.to(DEV), r.to(DEV)
        c = torch.full((m, n + 8), 7.0, dtype=torch.bfloat16, device=DEV)
        ep, _keep = _ep(form, biasd, rd)
        cnt = _launch(_tile_args(ad, bd, c[:, :n], ep, tm, tn, sched, splits), with_counters=True)
        torch.cuda.synchronize()
        O.assert_close(c[:, :n], _ref(form, a, b, bias, r), rtol=1e-2, atol=1e-2)
        assert (c[:, n:].float() == 7.0).all()
        assert int(cnt.abs().sum()) == 0, "a counter was left non-zero"
        c2 = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
        ep2, _keep2 = _ep(form, biasd, rd)
        _launch(_tile_args(ad, bd, c2, ep2, tm, tn, sched, splits), with_counters=False)
        torch.cuda.synchronize()
        assert torch.equal(c[:, :n], c2)


def test_split_tiles_fp32_and_int8_outputs():
    """The finish's store in the other output types: fp32 (unrounded) and int8 (one
    quantizer step of the oracle's)."""
    m, n, k = 128, 1024, 4096
    a, b, bias, r = _data(m, n, k, seed=30)
    ad, bd = a.to(DEV), b.to(DEV)
    acc = O.gemm_fp32(a, b)
    c32 = torch.empty((m, n), dtype=torch.float32, device=DEV)
    ep, _ = _ep("none", None, None)
    _launch(_tile_args(ad, bd, c32, ep, 64, 128, nat.TILE_W4, 4), with_counters=True)
    torch.cuda.synchronize()
    assert O.rel_to_max(c32.cpu(), acc) < 1e-5
    c8 = torch.empty((m, n), dtype=torch.int8, device=DEV)
    ep8, _ = _ep("none", None, None)
    ep8.form = nat.EP_FUSED
    ep8.cmul = 20.0
    _launch(_tile_args(ad, bd, c8, ep8, 64, 128, nat.TILE_W4, 4), with_counters=True)
    torch.cuda.synchronize()
    want = O.quantize_int8(acc * 20.0)
    assert (c8.cpu().int() - want.int()).abs().max() <= 1


def test_split_tiles_in_a_captured_graph():
    m, n, k = 128, 4096, 4096
    a, b, bias, r = _data(m, n, k, seed=40)
    ad, bd, biasd = a.to(DEV), b.to(DEV), bias.to(DEV)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    ep, _keep = _ep("bias_gelu", biasd, None)

    def call():  # hk's Python layer leaves a tile split to its reduction launch: counters by hand
        _launch(_tile_args(ad, bd, c, ep, 64, 128, nat.TILE_W4, 4), with_counters=True)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    gcnt = nat._CNT_GRAPH[torch.device(DEV)]
    for rep in range(3):
        a2, b2, bias2, _ = _data(m, n, k, seed=50 + rep)
        ad.copy_(a2.to(DEV))
        bd.copy_(b2.to(DEV))
        biasd.copy_(bias2.to(DEV))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        O.assert_close(c, O.gelu_tanh(O.gemm_fp32(a2, b2) + bias2.float()), rtol=1e-2, atol=1e-2)
        assert int(gcnt.abs().sum()) == 0
        call()
        torch.cuda.synchronize()
