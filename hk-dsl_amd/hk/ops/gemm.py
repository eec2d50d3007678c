"""hk.ops.matmul and hk.ops.scaled_mm on gfx950.

`scaled_mm` keeps the reference's contract (python/hk/ops/gemm.py:884-975): bf16
(A @ B^T) * scale_a * scale_b (+ bias), A (M, K) and B (N, K) float8_e4m3fn, fp32
accumulate; scale_a one value or one a row of A ((M,) or (M, 1)), scale_b one value or
one a row of B ((N,) or (1, N)); bias (N,). The reference runs it on gfx1201 only (its
gfx950 fp8 GEMMs are MX block-scaled); here it is the tile kernel's fp8 form,
v_mfma_f32_32x32x64_f8f6f4 with the scales and the bias applied to the accumulators in
registers before the one bf16 store.
"""

from __future__ import annotations

import ctypes

from .. import _native as nat
from . import gemm_cdna


def matmul(a, b, out=None):
    """C = A @ B^T, bf16 (N, K)-layout B (hk.ops.gemm.matmul, gemm.py:682-699)."""
    return gemm_cdna.matmul(a, b, out=out)


#: Python-number scales as one-element fp32 device tensors, by (device, value): made once
#: by a fill kernel (no host-to-device copy per call) and reused.
_NUMBERS: dict = {}
_NUMBERS_CAP = 1024


def _number(v: float, device):
    """A scale given as a Python number, on `device`. Outside a graph capture the tensor is
    cached; while capturing it is made by a fill kernel the graph records (so a replay
    refills it) and not kept, since a tensor filled only on replay would be garbage to an
    eager call before the first replay."""
    import torch  # noqa: PLC0415

    key = (device, float(v))
    t = _NUMBERS.get(key)
    if t is not None:
        return t
    t = torch.full((1,), float(v), device=device, dtype=torch.float32)
    if not torch.cuda.is_current_stream_capturing() and len(_NUMBERS) < _NUMBERS_CAP:
        _NUMBERS[key] = t
    return t


def _vec(t, length, what, device):
    import torch  # noqa: PLC0415

    if isinstance(t, (int, float)) and not isinstance(t, bool):
        return _number(t, device), 0
    t = torch.as_tensor(t, device=device, dtype=torch.float32)
    if t.numel() == 1:
        return t.reshape(1), 0
    if t.numel() != length:
        raise ValueError(f"scaled_mm: {what} has {t.numel()} values; one, or {length}")
    return t.reshape(length).contiguous(), 1


def scaled_mm(a, b, scale_a, scale_b, *, bias=None, out=None, schedule=None):
    """bf16 (A @ B^T) * scale_a * scale_b (+ bias), fp8-e4m3 operands, fp32 accumulate."""
    import torch  # noqa: PLC0415

    if a.dtype != torch.float8_e4m3fn or b.dtype != torch.float8_e4m3fn:
        raise TypeError(f"scaled_mm: A and B float8_e4m3fn, got {a.dtype} and {b.dtype}")
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[1]:
        raise ValueError(f"scaled_mm: A (M, K) and B (N, K), got {tuple(a.shape)} and "
                         f"{tuple(b.shape)}")
    m, k = a.shape
    n = b.shape[0]
    if k % 128 or n % 4 or m < 1:
        raise ValueError(f"scaled_mm: K={k} must be a multiple of 128 and N={n} of 4; M (={m}) "
                         f"may be ragged")
    if a.stride(1) != 1 or b.stride(1) != 1:
        raise ValueError("scaled_mm: A and B need unit stride along K")
    sa, sa_ld = _vec(scale_a, m, "scale_a", a.device)
    sb, sb_ld = _vec(scale_b, n, "scale_b", a.device)
    if out is None:
        out = torch.empty(m, n, device=a.device, dtype=torch.bfloat16)
    elif tuple(out.shape) != (m, n) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError(f"scaled_mm: out is {tuple(out.shape)}/{out.dtype}, expected "
                         f"({m}, {n})/bfloat16")
    name = schedule or gemm_cdna.route(m, n, k, fp8=True)
    rec = gemm_cdna.resolve(gemm_cdna.CANDIDATES[name], m, n, k, fp8=True)
    ep = nat.HkxEpilogue()
    ep.form = nat.EP_FUSED
    ep.cmul = 1.0
    ep.col_scale, ep.row_scale, ep.row_add, ep.tile_add = 0, 1, -1, -1
    ep.ops[0] = nat.HkxOperand(sa.data_ptr(), nat.COL, nat.FP32, sa_ld)
    ep.ops[1] = nat.HkxOperand(sb.data_ptr(), nat.ROW, nat.FP32, sb_ld)
    ep.nops = 2
    keep = [sa, sb]
    if bias is not None:
        bb = bias.reshape(n).to(torch.bfloat16).contiguous()
        keep.append(bb)
        ep.ops[2] = nat.HkxOperand(bb.data_ptr(), nat.ROW, nat.BF16, 1)
        ep.row_add, ep.nops = 2, 3
    args = nat.gemm_args(a, b, out, kernel=nat.KERNEL_TILE, tile_m=rec["tile_m"],
                         tile_n=rec["tile_n"], schedule=nat.SCHEDULES[rec["schedule"]],
                         variant=rec.get("variant", 0),
                         splits=rec.get("splits", 1), ep=ep)
    nat.run(args, a.device)
    del keep
    return out


__all__ = ["matmul", "scaled_mm"]
