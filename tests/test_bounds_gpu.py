"""Calls at the edge of the kernels' 32-bit addressing, against the CPU oracle.

The 256 x 256 ring kernels store C through a buffer resource with 32-bit byte offsets,
computed for every row of the last 256-row tile, the rows past M included. A call whose
C fits in 4 GiB but whose last tile, rounded up to 256 rows, does not must not take
those kernels: the rows past M would wrap round onto C's first rows and overwrite them.
Here M = 174700, N = 12288 (bf16 C: 4.2936e9 bytes < 2^32; rounded up to 174848 rows:
4.2971e9 > 2^32). The first and last rows are checked against the oracle."""

import pytest
import torch

import hk
from oracle import gemm_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
T = hk.templates.gemm


def test_c_just_under_4gib_keeps_its_first_rows():
    m, n, k = 174700, 12288, 64
    assert m * n * 2 < 2 ** 32 < ((m + 255) // 256) * 256 * n * 2
    g = torch.Generator().manual_seed(11)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    b = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    print(f"M={m} N={n} K={k} schedule t256 bias", flush=True)
    c = T(a.to(DEV), b.to(DEV), epilogue=T.bias, bias=bias.to(DEV), schedule="t256")
    torch.cuda.synchronize()
    for rows in (slice(0, 64), slice(m - 64, m)):
        ref = O.gemm_fp32(a[rows], b) + bias.float()
        O.assert_close(c[rows], ref, 1e-2, 1e-2)
    del c
    torch.cuda.empty_cache()
