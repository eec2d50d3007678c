"""hk.ops.scaled_mm's whole contract on the GPU against the CPU oracle: the e5m2 operand
pairs, the fp32 out and accumulate=True (python/hk/ops/gemm.py:884-975) -- the forms past
config 5's e4m3 x e4m3 + dequant + bias, which tests/test_templates_gemm_gpu.py covers.

fp8 values are exact in fp32 (e4m3 and e5m2 alike), so the oracle is the fp32 product of
the same operands (oracle/gemm_oracle.py: scaled_mm). Checks: bf16 outputs rtol 3e-2 /
atol 1e-2 elementwise (north_star's fp8 tolerance) and the reference tests' rel-to-max
(< 8e-3); fp32 outputs rel-to-max < 1e-4 (the summation and scaling order differ; a bf16
rounding would show as ~2e-3)."""

import pytest
import torch

import hk
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
E4, E5 = torch.float8_e4m3fn, torch.float8_e5m2


def _ops(m, n, k, da, db, seed):
    g = torch.Generator().manual_seed(seed)
    a8 = (torch.randn(m, k, generator=g) * 2).to(da)
    b8 = (torch.randn(n, k, generator=g) * 2).to(db)
    sa = torch.rand(m, 1, generator=g) * 0.05 + 0.01
    sb = torch.rand(n, generator=g) * 0.05 + 0.01
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    return a8, b8, sa, sb, bias


@pytest.mark.parametrize("da,db", [(E5, E5), (E4, E5), (E5, E4), (E4, E4)])
@pytest.mark.parametrize("m,n,k", [(300, 512, 1024), (1024, 768, 2048), (5, 256, 512)])
def test_operand_pairs_with_bias(da, db, m, n, k):
    a8, b8, sa, sb, bias = _ops(m, n, k, da, db, seed=m + n)
    got = hk.ops.scaled_mm(a8.to(DEV), b8.to(DEV), sa.to(DEV), sb.to(DEV), bias=bias.to(DEV))
    ref = O.scaled_mm(a8, b8, sa, sb, bias)
    O.assert_close(got, ref, rtol=3e-2, atol=1e-2)
    got0 = hk.ops.scaled_mm(a8.to(DEV), b8.to(DEV), sa.to(DEV), sb.to(DEV))
    assert O.rel_to_max(got0.cpu(), O.scaled_mm(a8, b8, sa, sb)) < 8e-3


@pytest.mark.parametrize("da,db", [(E4, E4), (E5, E4)])
def test_fp32_out_is_the_unrounded_product(da, db):
    m, n, k = 520, 512, 1024
    a8, b8, sa, sb, _ = _ops(m, n, k, da, db, seed=11)
    out = torch.full((m, n), 7.0, device=DEV)
    got = hk.ops.scaled_mm(a8.to(DEV), b8.to(DEV), sa.to(DEV), sb.to(DEV), out=out)
    assert got is out
    assert O.rel_to_max(out.cpu(), O.scaled_mm(a8, b8, sa, sb)) < 1e-4


@pytest.mark.parametrize("da,db", [(E4, E4), (E4, E5)])
def test_accumulate_adds_into_out(da, db):
    """out += (A @ B^T) * scale_a * scale_b, twice: a weight gradient accumulated into its
    fp32 main_grad over two micro-batches."""
    m, n, k = 300, 768, 512
    a8, b8, sa, sb, _ = _ops(m, n, k, da, db, seed=12)
    r = torch.randn(m, n, generator=torch.Generator().manual_seed(13))
    out = r.to(DEV)
    for _ in range(2):
        hk.ops.scaled_mm(a8.to(DEV), b8.to(DEV), sa.to(DEV), sb.to(DEV), out=out, accumulate=True)
    ref = r + 2 * O.scaled_mm(a8, b8, sa, sb)
    assert O.rel_to_max(out.cpu(), ref) < 1e-4


def test_number_scales_with_e5m2():
    m, n, k = 64, 256, 256
    a8, b8, _, _, _ = _ops(m, n, k, E5, E5, seed=14)
    got = hk.ops.scaled_mm(a8.to(DEV), b8.to(DEV), 0.5, 0.125)
    assert O.rel_to_max(got.cpu(), O.scaled_mm(a8, b8, 0.5, 0.125)) < 8e-3


def test_e5m2_needs_the_ring_kernels_n():
    a8, b8, sa, sb, _ = _ops(64, 260, 256, E5, E5, seed=15)
    with pytest.raises(hk._native.HkxError, match="ring kernel"):
        hk.ops.scaled_mm(a8.to(DEV), b8.to(DEV), sa.to(DEV), sb.to(DEV))


@pytest.mark.parametrize("m,n,k,route", [(128, 4096, 4096, "t64x128k2"), (64, 1024, 8192, "t64x128k4"),
                                         (256, 4096, 4096, "t64x128"), (384, 2048, 8192, "t64x128k2")])
def test_mid_m_splits_over_k(m, n, k, route):
    # fp8 takes the route rule; at these shapes it runs 64 x 128 tiles, split over K where
    # each split keeps enough K (fp32 shares summed in split order, then the dequant and the
    # bias)
    from hk.ops import gemm_cdna

    assert gemm_cdna.route(m, n, k, fp8=True) == route
    a8, b8, sa, sb, bias = _ops(m, n, k, E4, E4, seed=m + k)
    got = hk.ops.scaled_mm(a8.to(DEV), b8.to(DEV), sa.to(DEV), sb.to(DEV), bias=bias.to(DEV))
    O.assert_close(got, O.scaled_mm(a8, b8, sa, sb, bias), rtol=3e-2, atol=1e-2)


@pytest.mark.parametrize("form", ["one_one", "one_vec", "vec_one", "tensor_one"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_e4m3_one_value_scales_on_the_256_tiles(form, with_bias):
    """Per-tensor scales (one value, stride 0) on the 256 x 256 tile kernels, mixed with
    per-row / per-channel ones: the quadrant kernel reads a one-value scale once and DMAs
    only the vector ones. Ragged M and N (520 x 776), two tiles a column."""
    m, n, k = 520, 776, 1024
    a8, b8, sa, sb, bias = _ops(m, n, k, E4, E4, seed=16)
    sa_d, sb_d = sa.to(DEV), sb.to(DEV)
    if form == "one_one":
        sa_x, sb_x, sa_r, sb_r = 0.03, 0.02, 0.03, 0.02
    elif form == "one_vec":
        sa_x, sb_x, sa_r, sb_r = 0.03, sb_d, 0.03, sb
    elif form == "vec_one":
        sa_x, sb_x, sa_r, sb_r = sa_d, 0.02, sa, 0.02
    else:  # 0-d device tensors
        sa_x, sb_x = torch.tensor(0.03, device=DEV), torch.tensor(0.02, device=DEV)
        sa_r, sb_r = 0.03, 0.02
    bb = bias.to(DEV) if with_bias else None
    got = hk.ops.scaled_mm(a8.to(DEV), b8.to(DEV), sa_x, sb_x, bias=bb, schedule="t256")
    ref = O.scaled_mm(a8, b8, sa_r, sb_r, bias if with_bias else None)
    O.assert_close(got, ref, rtol=3e-2, atol=1e-2)
    assert O.rel_to_max(got.cpu(), ref) < 8e-3
