"""MXFP8 GEMM on gfx950: C = (sa . A)(sb . B)^T in bf16.

The reference's contract (python/hk/ops/mxfp8.py:1-110): A (M, K) and B (N, K) fp8 e4m3,
K-contiguous (F.linear's layout); sa (M, K/32) and sb (N, K/32) their E8M0 scales, one byte
a row and 32 columns (the OCP MX layout; a 32 x 32-block weight scale is its rows repeated,
`expand_block_scales`). Here the product runs on the quadrant GEMM kernel's MX form (the
ring kernel's where K is split over workgroups): every MFMA
is gfx950's scaled one (v_mfma_scale_f32_32x32x64_f8f6f4), each lane passing the E8M0 byte
of its own fragment row and 32-K block; the scales reach LDS by the same DMA as the
operands, 16 bytes a row every 8 half-stages (whole lines: one 4-byte load a row and
half-stage doubled the L2 requests and cost 60%). K a multiple of 128, N of 8, any M.
Where the tiles fill less than half the CUs, K is split over workgroups into fp32 shares
(a cached workspace, `_native.workspace`) that a second pass sums in split order.

`quant(x)` is the activation side (python/hk/ops/mxfp8.py:605-660): bf16 x to fp8 e4m3 and
E8M0 scales by AITER's per_1x32 rule (python/hk/mx.py:17-31), in one launch, the scales in
the OCP layout `gemm` reads. The reference's packed and AITER scale layouts exist for its
own kernels' register shapes; this build's kernel reads the OCP bytes directly.
"""

from __future__ import annotations

from .. import _native as nat


def expand_block_scales(s, block_rows: int = 32):
    """32 x 32-block E8M0 scales [N/32, K/32] as one row each [N, K/32] (hk/mx.py:49-51)."""
    return s.repeat_interleave(block_rows, dim=0).contiguous()


def _scales(s, rows, k, what):
    import torch  # noqa: PLC0415

    if s.dtype not in (torch.uint8, torch.int8):
        raise TypeError(f"mxfp8: {what} holds E8M0 bytes (uint8), got {s.dtype}")
    if s.dim() != 2 or s.shape[0] != rows or s.shape[1] != k // 32:
        raise ValueError(f"mxfp8: {what} is {tuple(s.shape)}, expected ({rows}, {k // 32})")
    if s.stride(1) != 1 or s.stride(0) % 4 or s.data_ptr() % 4:
        s = s.contiguous()
    return s


def gemm(a, b, sa, sb, out=None):
    """bf16 (M, N) = (sa . a)(sb . b)^T; see the module docstring."""
    import torch  # noqa: PLC0415

    if a.dtype != torch.float8_e4m3fn or b.dtype != torch.float8_e4m3fn:
        raise TypeError(f"mxfp8.gemm: a and b are float8_e4m3fn, got {a.dtype} and {b.dtype}")
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[1]:
        raise ValueError(f"mxfp8.gemm: a (M, K) and b (N, K), got {tuple(a.shape)} and "
                         f"{tuple(b.shape)}")
    m, k = a.shape
    n = b.shape[0]
    if k % 128 or n % 8:
        raise ValueError(f"mxfp8.gemm: K={k} a multiple of 128 and N={n} of 8")
    if not a.is_cuda or b.device != a.device:
        raise ValueError("mxfp8.gemm: a and b are on one GPU")
    a = a if a.stride(1) == 1 and a.stride(0) % 16 == 0 and a.data_ptr() % 16 == 0 else a.contiguous()
    b = b if b.stride(1) == 1 and b.stride(0) % 16 == 0 and b.data_ptr() % 16 == 0 else b.contiguous()
    sa = _scales(sa, m, k, "sa")
    sb = _scales(sb, n, k, "sb")
    if out is None:
        out = torch.empty((m, n), device=a.device, dtype=torch.bfloat16)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (m, n) or out.stride(1) != 1:
        raise ValueError(f"mxfp8.gemm: out is bf16 ({m}, {n}) with unit column stride")
    L = nat.lib()
    nws = L.hkx_mx_gemm_workspace(m, n, k)
    ws = nat.workspace(a.device, nws)
    nat.check(L.hkx_mx_gemm(
        a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), sa.data_ptr(), sa.stride(0),
        sb.data_ptr(), sb.stride(0), out.data_ptr(), out.stride(0), m, n, k,
        ws.data_ptr() if ws is not None else None, nws, nat.stream_of(a.device)))
    return out


def quant(x, out=None):
    """(q, s) for bf16 x [M, K], K a multiple of 32: q float8_e4m3fn [M, K], s uint8
    [M, K/32] (OCP layout), by AITER's per_1x32 rule."""
    import torch  # noqa: PLC0415

    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise TypeError(f"mxfp8.quant: x is bf16 (M, K), got {x.dtype} {tuple(x.shape)}")
    m, k = x.shape
    if k % 32:
        raise ValueError(f"mxfp8.quant: K={k}, a multiple of 32")
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    q, s = out if out is not None else (
        torch.empty((m, k), device=x.device, dtype=torch.float8_e4m3fn),
        torch.empty((m, k // 32), device=x.device, dtype=torch.uint8))
    nat.check(nat.lib().hkx_mx_quant(x.data_ptr(), x.stride(0), q.data_ptr(), q.stride(0),
                                     s.data_ptr(), s.stride(0), m, k,
                                     nat.stream_of(x.device)))
    return q, s


def linear(x, w, ws):
    """bf16 x [M, K] @ (ws . w)^T, w fp8 [N, K] with E8M0 row scales ws [N, K/32]: the
    activation quantized (`quant`), then `gemm`."""
    xq, xs = quant(x)
    return gemm(xq, w, xs, ws)


__all__ = ["gemm", "quant", "linear", "expand_block_scales"]
