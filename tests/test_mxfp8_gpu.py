"""hk.ops.mxfp8 on the GPU against the CPU oracle: the MX GEMM against the scaled fp32 product
(the reference's check and tolerance, tests/hk/gpu/test_mxfp8_gemm.py:19-34: max|err| / max|ref|
< 5e-3), ragged M and several tiles a workgroup, 32 x 32 block weight scales; the activation
quantization bit for bit against the oracle's AITER per_1x32 rule
(tests/hk/gpu/test_mxfp8_quant.py:30-45)."""

import pytest
import torch

from hk.ops import mxfp8
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _operands(m, n, k, seed, block_weight_scales=False):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(m, k, generator=g).to(torch.float8_e4m3fn)
    b = torch.randn(n, k, generator=g).to(torch.float8_e4m3fn)
    sa = torch.randint(124, 131, (m, k // 32), generator=g, dtype=torch.uint8)
    if block_weight_scales:
        sb = mxfp8.expand_block_scales(
            torch.randint(124, 131, (n // 32, k // 32), generator=g, dtype=torch.uint8))
    else:
        sb = torch.randint(124, 131, (n, k // 32), generator=g, dtype=torch.uint8)
    return a, b, sa, sb


@pytest.mark.parametrize("m,n,k,blk", [(256, 256, 512, True), (512, 384, 1280, True),
                                       (300, 512, 1152, False), (1, 256, 128, False),
                                       (2100, 2048, 2048, False), (4096, 4352, 128, False),
                                       (4096, 4352, 1152, True), (64, 512, 4224, False),
                                       (16, 1792, 5120, True)])
def test_mx_gemm_matches_the_scaled_product(m, n, k, blk):
    """Whole and partial chunks of 8 half-stages of scales (K = 1152: 18 half-stages, its last
    chunk two), the shortest K (128: a two-half-stage chunk a tile, two tiles a workgroup at
    4096 x 4352), ragged M; K split over workgroups where the tiles are few (2 splits at
    2100 x 2048 x 2048, 5 at 16 x 1792 x 5120, 4 of 9, 9, 9 and 6 k-tiles at 64 x 512 x
    4224), each split's scales read from its own first K block."""
    a, b, sa, sb = _operands(m, n, k, seed=m + n + k, block_weight_scales=blk)
    print(f"case mx_gemm {m}x{n}x{k}", flush=True)
    out = mxfp8.gemm(a.to(DEV), b.to(DEV), sa.to(DEV), sb.to(DEV))
    ref = O.mx_gemm(a, b, sa, sb)
    assert O.rel_to_max(out.cpu(), ref) < 5e-3


def test_mx_gemm_scales_reach_every_block():
    """One K block of one row of each operand scaled by 32 (its E8M0 byte + 5): exactly the
    output elements that block feeds change, by that block's share."""
    m, n, k = 256, 256, 512
    a, b, sa, sb = _operands(m, n, k, seed=3)
    base = mxfp8.gemm(a.to(DEV), b.to(DEV), sa.to(DEV), sb.to(DEV)).float().cpu()
    sa2, sb2 = sa.clone(), sb.clone()
    sa2[77, 9] += 5   # x32: large enough to show in every bf16 output it feeds
    sb2[201, 14] += 5
    out = mxfp8.gemm(a.to(DEV), b.to(DEV), sa2.to(DEV), sb2.to(DEV)).float().cpu()
    ref = O.mx_gemm(a, b, sa2, sb2)
    assert O.rel_to_max(out, ref) < 5e-3
    changed = out != base
    assert changed[77].sum() > 200 and changed[:, 201].sum() > 200
    changed[77, :] = False
    changed[:, 201] = False
    assert not changed.any()  # every other element is bit for bit the same


def _x(m, k, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(m, k, generator=g)
            * torch.exp2(torch.randint(-20, 20, (m, 1), generator=g).float())).bfloat16()


@pytest.mark.parametrize("m,k", [(64, 128), (100, 1152), (2048, 5120), (2059, 1280), (7, 32)])
def test_mx_quant_is_the_per_1x32_rule_bit_for_bit(m, k):
    x = _x(m, k, seed=m + k)
    x[0, :32] = 0.0                  # a zero block: byte clamped to 0
    if m > 1:
        x[1, :32] = 2.0 ** -130      # a tiny block: q scaled by the unclamped e
    print(f"case mx_quant {m}x{k}", flush=True)
    q, s = mxfp8.quant(x.to(DEV))
    rq, rs = O.mx_quant(x)
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s.cpu(), rs)


def test_mx_linear_is_quant_then_gemm():
    m, n, k = 300, 512, 1024
    x = _x(m, k, seed=5)
    g = torch.Generator().manual_seed(6)
    w = torch.randn(n, k, generator=g).to(torch.float8_e4m3fn)
    ws = torch.randint(120, 130, (n, k // 32), generator=g, dtype=torch.uint8)
    out = mxfp8.linear(x.to(DEV), w.to(DEV), ws.to(DEV))
    xq, xs = O.mx_quant(x)
    assert O.rel_to_max(out.cpu(), O.mx_gemm(xq, w, xs, ws)) < 5e-3


def test_vllm_mxfp8_op_takes_the_hk_path():
    """hk_vllm::mxfp8_linear's body where the route takes the shape (a table that routes it),
    on a 32 x 32 block-scaled weight: this build's quant and GEMM, right against the oracle
    (no vLLM needed on that path)."""
    from hk.integration import engine as E
    from hk.integration import vllm_mxfp8 as V

    m, n, k = 2048, 512, 1024
    V.set_routes(E.RouteTable({(n, k): {"runs": [[1, 8192, "hk"]]}}))
    try:
        _vllm_op(V, m, n, k)
    finally:
        V.set_routes(None)


def _vllm_op(V, m, n, k):
    x = _x(m, k, seed=11)
    g = torch.Generator().manual_seed(12)
    w = torch.randn(n, k, generator=g).to(torch.float8_e4m3fn)
    blocks = torch.randint(120, 130, (n // 32, k // 32), generator=g, dtype=torch.uint8)
    rows = mxfp8.expand_block_scales(blocks)
    before = V.PATCH.stats["hk"]
    out = V.mxfp8_linear(x.to(DEV), w.to(DEV), blocks.to(DEV), rows.to(DEV), torch.bfloat16)
    assert V.PATCH.stats["hk"] == before + 1
    xq, xs = O.mx_quant(x)
    assert O.rel_to_max(out.cpu(), O.mx_gemm(xq, w, xs, rows)) < 5e-3
