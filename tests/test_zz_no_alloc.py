"""hkx_gemm_noalloc, the entry point that allocates nothing, against hkx_gemm on the GPU.

For plans that use a workspace (split-K shares summed by the reduction pass, the decode
kernel's K split, an epilogue outside the fused form run in the pass) the no-allocation
entry point must give exactly hkx_gemm's bits: the same kernels, the workspace being the
library's static per-GPU scratch instead of a caller's buffer. Two calls in a row, the
second smaller, so the second reads scratch the first left behind. A plan that needs more
scratch than the library holds is refused with HKX_ERR_WORKSPACE, and the output is
checked against the oracle as well."""

import ctypes

import pytest
import torch

import hk
from hk import _native as nat
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
T = hk.templates.gemm


def _args(a, b, c, sched_name, bias):
    from hk.ops import gemm_cdna

    m, k = a.shape
    n = c.shape[1]
    rec = gemm_cdna.resolve(gemm_cdna.CANDIDATES[sched_name], m, n, k)
    ep = T.bind(T.bias_gelu, dict(bias=bias), m, n, torch.bfloat16).struct()
    ep.ops[0].ptr, ep.ops[0].dtype, ep.ops[0].ld = bias.data_ptr(), nat.BF16, 1
    if rec["kernel"] == "tile":
        return nat.gemm_args(a, b, c, kernel=nat.KERNEL_TILE, tile_m=rec["tile_m"],
                             tile_n=rec["tile_n"], schedule=nat.SCHEDULES[rec["schedule"]],
                             variant=rec.get("variant", 0), splits=rec["splits"], ep=ep)
    return nat.gemm_args(a, b, c, kernel=nat.KERNEL_DECODE, decode_waves=rec.get("waves", 8),
                         decode_rows=rec.get("rows", 16), variant=rec.get("variant", 0),
                         splits=rec["splits"], ep=ep)


def _data(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    b = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    return a, b, bias


@pytest.mark.parametrize("sched,shapes", [
    ("t64k4", [(64, 4096, 4096), (40, 2048, 4096)]),
    ("t128k2", [(256, 4096, 2048), (130, 1024, 2048)]),
    ("decode_blk", [(16, 2048, 4096), (3, 1024, 4096)]),
])
def test_noalloc_matches_hkx_gemm_on_two_calls(sched, shapes):
    L = nat.lib()
    for i, (m, n, k) in enumerate(shapes):
        print(f"{sched} call {i}: M={m} N={n} K={k}", flush=True)
        a, b, bias = _data(m, n, k, seed=10 + i)
        ad, bd, biasd = a.to(DEV), b.to(DEV), bias.to(DEV)
        c_ref = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
        c_new = torch.full((m, n), 7.0, device=DEV, dtype=torch.bfloat16)
        args = _args(ad, bd, c_ref, sched, biasd)
        need = L.hkx_gemm_workspace(ctypes.byref(args))
        assert 0 < need <= nat.NOALLOC_SCRATCH_BYTES, need       # the plan uses scratch
        nat.run(args, ad.device)
        args2 = _args(ad, bd, c_new, sched, biasd)
        nat.run_noalloc(args2, ad.device)
        torch.cuda.synchronize()
        assert torch.equal(c_new, c_ref), f"{sched} call {i}"
        ref = O.gelu_tanh(O.gemm_fp32(a, b) + bias.float())
        O.assert_close(c_new, ref, 1e-2, 1e-2)


def test_noalloc_refuses_a_plan_beyond_its_scratch():
    m, n, k = 4096, 4096, 4096        # t64k8 shares: 8 * 4096 * 4096 * 4 bytes = 512 MiB
    a = torch.zeros(m, k, device=DEV, dtype=torch.bfloat16)
    b = torch.zeros(n, k, device=DEV, dtype=torch.bfloat16)
    bias = torch.zeros(n, device=DEV, dtype=torch.bfloat16)
    c = torch.full((m, n), 7.0, device=DEV, dtype=torch.bfloat16)
    args = _args(a, b, c, "t64k8", bias)
    assert nat.lib().hkx_gemm_workspace(ctypes.byref(args)) > nat.NOALLOC_SCRATCH_BYTES
    with pytest.raises(nat.HkxError, match="no-allocation entry point has"):
        nat.run_noalloc(args, a.device)
    torch.cuda.synchronize()
    assert bool((c == 7.0).all())          # nothing was launched
