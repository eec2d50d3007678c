"""hk.ops.matmul and hk.ops.scaled_mm on gfx950.

`scaled_mm` keeps the reference's contract (python/hk/ops/gemm.py:884-975): bf16
(A @ B^T) * scale_a * scale_b (+ bias), A (M, K) and B (N, K) float8_e4m3fn, fp32
accumulate; scale_a one value or one a row of A ((M,) or (M, 1)), scale_b one value or
one a row of B ((N,) or (1, N)); bias (N,). The reference runs it on gfx1201 only (its
gfx950 fp8 GEMMs are MX block-scaled); here it is the tile kernels' fp8 forms (at 256 x 256
the quadrant kernel on v_mfma_f32_16x16x128_f8f6f4, smaller tiles on the 4-wave and 8-wave
kernels) with the scales and the bias applied to the accumulators in registers before the
one bf16 store.
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
    capturing = torch.device(device).type == "cuda" and torch.cuda.is_current_stream_capturing()
    if not capturing and len(_NUMBERS) < _NUMBERS_CAP:
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


def _pair_code(a, b) -> int:
    """The ab_dtype of an fp8 operand pair (include/hkx.h)."""
    import torch  # noqa: PLC0415

    e4, e5 = torch.float8_e4m3fn, torch.float8_e5m2
    codes = {(e4, e4): nat.FP8E4M3, (e5, e5): nat.FP8E5M2, (e4, e5): nat.FP8_E4M3_E5M2,
             (e5, e4): nat.FP8_E5M2_E4M3}
    code = codes.get((a.dtype, b.dtype))
    if code is None:
        raise TypeError(f"scaled_mm: A and B float8_e4m3fn or float8_e5m2, got {a.dtype} and "
                        f"{b.dtype}")
    return code


def scaled_mm(a, b, scale_a, scale_b, *, bias=None, out=None, accumulate: bool = False,
              schedule=None):
    """bf16 (A @ B^T) * scale_a * scale_b (+ bias), fp8 operands, fp32 accumulate -- the
    reference's contract (python/hk/ops/gemm.py:884-975):

    * A (M, K) and B (N, K), float8_e4m3fn or float8_e5m2, either pairing (a mixed pair is
      a training backward's gradient against a weight); e4m3 x e4m3 runs on every tile
      kernel, a pair with e5m2 on the 256 x 256 ring kernel;
    * scale_a one value or one a row of A ((M,) or (M, 1)), scale_b one value or one a row
      of B ((N,) or (1, N)); bias (N,);
    * an fp32 `out` (M, N) takes the product unrounded, and with `accumulate=True` it is
      added to: out += (A @ B^T) * scale_a * scale_b (a weight gradient into its fp32
      main_grad); no bias either way.
    """
    import torch  # noqa: PLC0415

    code = _pair_code(a, b)
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
    fp32_out = accumulate or (out is not None and out.dtype == torch.float32)
    if fp32_out:
        if bias is not None:
            raise ValueError("scaled_mm: an fp32 out takes no bias")
        if out is None or tuple(out.shape) != (m, n) or out.dtype != torch.float32 \
                or not out.is_contiguous():
            raise ValueError("scaled_mm(accumulate=True): out is the fp32 (M, N) tensor added "
                             "to, contiguous")
    elif out is None:
        out = torch.empty(m, n, device=a.device, dtype=torch.bfloat16)
    elif tuple(out.shape) != (m, n) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError(f"scaled_mm: out is {tuple(out.shape)}/{out.dtype}, expected "
                         f"({m}, {n})/bfloat16")
    sa, sa_ld = _vec(scale_a, m, "scale_a", a.device)
    sb, sb_ld = _vec(scale_b, n, "scale_b", a.device)
    if code != nat.FP8E4M3:
        name = "t256"   # a pair with e5m2: the ring kernel's generic form
    else:
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
    if accumulate:
        # the accumulator starts as out: read and written by the same lane, in place
        ep.ops[2] = nat.HkxOperand(out.data_ptr(), nat.TILE, nat.FP32, out.stride(0))
        ep.tile_add, ep.nops = 2, 3
    if bias is not None:
        bb = bias.reshape(n).to(torch.bfloat16).contiguous()
        keep.append(bb)
        ep.ops[2] = nat.HkxOperand(bb.data_ptr(), nat.ROW, nat.BF16, 1)
        ep.row_add, ep.nops = 2, 3
    args = nat.gemm_args(a, b, out, kernel=nat.KERNEL_TILE, tile_m=rec["tile_m"],
                         tile_n=rec["tile_n"], schedule=nat.SCHEDULES[rec["schedule"]],
                         variant=0 if code != nat.FP8E4M3 else rec.get("variant", 0),
                         splits=rec.get("splits", 1), ep=ep)
    args.ab_dtype = code
    nat.run(args, a.device)
    del keep
    return out


__all__ = ["matmul", "scaled_mm"]
