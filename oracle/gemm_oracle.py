"""CPU oracle for the GEMM-with-fused-epilogue path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (hk-dsl_amd/) imports this module; only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as the
checker (or the timed CPU baseline), never as the thing measured or shipped.

Every function restates, on the CPU in fp32 (float64 where stated), what the reference
computes for this path. Each cites the reference lines it follows (vivienfanghuagood/hk-dsl
0.9.24, read as text; the reference is not imported or run). How each is pinned -- against
closed forms, a float64 brute force, torch's independent implementations, and the format
definitions -- is in tests/test_oracle.py.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

# ------------------------------------------------------------------ pointwise functions

#: The reference's constants for GELU(tanh) as x * sigmoid(2u), u = sqrt(2/pi)(x + 0.044715
#: x^3), with sigmoid(2u) = 1 / (1 + 2^(x (A x^2 + B))) (templates/gemm.py:814-821).
GELU_B = -2.0 * math.log2(math.e) * math.sqrt(2.0 / math.pi)
GELU_A = GELU_B * 0.044715


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """GELU, tanh approximation, textbook form: 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3))).
    What the reference's tests compare against (`F.gelu(..., approximate="tanh")`,
    tests/hk/gpu/test_templates_gemm.py:47; bench/dx/tasks/t4_linear_bias_gelu/reference.py:23-24)."""
    x = x.float()
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x * x * x)))


def gelu_tanh_exp2(x: torch.Tensor) -> torch.Tensor:
    """The reference's instruction-level form of the same function (templates/gemm.py:824-837):
    q = 2^(x (A x^2 + B)); x * rsqrt(1 + q)^2. Equal to gelu_tanh up to rounding."""
    x = x.float()
    q = x * x * GELU_A + GELU_B
    q = torch.exp2(q * x)
    r = torch.rsqrt(q + 1.0)
    return x * r * r


def silu(x: torch.Tensor) -> torch.Tensor:
    """x * sigmoid(x) (templates/gemm.py:845-847; ops/fused.py:80-114's silu)."""
    x = x.float()
    return x / (1.0 + torch.exp(-x))


def silu_and_mul(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """silu(g) * u in fp32 with one rounding at the store (hk.ops.silu_mul,
    ops/fused.py:80-114): vLLM's SiluAndMul on the gate and up halves."""
    return silu(g) * u.float()


def relu(x: torch.Tensor) -> torch.Tensor:
    return torch.clamp_min(x.float(), 0.0)


# ------------------------------------------------------------------ the GEMM

def gemm_fp32(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """A (M, K) @ B (N, K)^T with fp32 accumulation: C = A B^T, B in F.linear's layout
    (templates/gemm.py:10-11, 775-782). Operands are exact in fp32 (bf16 and fp8 both are)."""
    return a.float() @ b.float().t()


def gemm_f64(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """The same product in float64 -- the brute-force reference the fp32 one is checked
    against on tiny shapes."""
    return a.double() @ b.double().t()


def linear_bias_gelu(x, w_kn, b) -> torch.Tensor:
    """Config 1 / the t4 task: y = gelu_tanh(x @ w + b), w given (K, N), fp32 accumulate
    (bench/dx/tasks/t4_linear_bias_gelu/reference.py:8-37)."""
    return gelu_tanh(x.float() @ w_kn.float() + b.float())


# ------------------------------------------------------------------ epilogues

def apply_epilogue(name: str, acc: torch.Tensor, **ops) -> torch.Tensor:
    """The ready-made epilogues of hk.templates.gemm on an fp32 accumulator
    (templates/gemm.py:809-888), operands converted to fp32 and broadcast against C as
    torch broadcasts them (`_kind`, :116-135)."""
    f = {k: (v.float() if isinstance(v, torch.Tensor) else v) for k, v in ops.items()}
    if name in ("none", "identity"):
        return acc
    if name == "bias":
        return acc + f["bias"]
    if name in ("gelu", "gelu_tanh"):
        return gelu_tanh(acc)
    if name == "bias_gelu":
        return gelu_tanh(acc + f["bias"])
    if name == "silu":
        return silu(acc)
    if name == "bias_silu":
        return silu(acc + f["bias"])
    if name == "relu":
        return relu(acc)
    if name == "bias_relu":
        return relu(acc + f["bias"])
    if name == "residual":
        return acc + f["residual"]
    if name == "bias_residual":
        return acc + f["bias"] + f["residual"]
    if name == "scale":
        return acc * f["scale"]
    raise KeyError(name)


def split_k(a: torch.Tensor, b: torch.Tensor, splits: int, kstep: int) -> torch.Tensor:
    """C as the reference's split-K plans form it: fp32 shares over contiguous K ranges
    (whole k-steps, ceil-divided), summed in split order, the epilogue then run once on
    the sum (gemm_cdna_dp.py:220-228, 295-324)."""
    k = a.shape[1]
    units = k // kstep
    per = -(-units // splits)
    acc = None
    for s in range(0, units, per):
        lo, hi = s * kstep, min(units, s + per) * kstep
        share = gemm_fp32(a[:, lo:hi], b[:, lo:hi])
        acc = share if acc is None else acc + share
    return acc


# ------------------------------------------------------------------ fp8 e4m3 (OCP)

def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """float8_e4m3fn bytes -> float32, from the format: sign, 4 exponent bits (bias 7),
    3 mantissa bits; exponent 0 is subnormal (m * 2^-9); 0x7f / 0xff are NaN; no inf."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> float8_e4m3fn bytes, round to nearest even, saturating at +-448 (the
    quantizing store of templates/gemm.py:883-888; torch's cast gives NaN past 448).
    Brute force over the 127 non-negative finite codes: the nearest value, ties to the
    even code."""
    x = np.asarray(x, dtype=np.float32)
    table = e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)  # 0 .. 448
    ax = np.minimum(np.abs(x.astype(np.float64)), 448.0)
    d = np.abs(ax[..., None] - table)
    best = d.min(axis=-1, keepdims=True)
    ties = d == best
    # among equally near codes, the even one (the lowest mantissa bit clear)
    idx = np.where(ties.sum(-1) > 1, np.argmax(ties & (np.arange(0x7F) % 2 == 0), axis=-1),
                   np.argmin(d, axis=-1))
    out = idx.astype(np.uint8) | np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    return np.where(np.isnan(x), np.uint8(0x7F), out).astype(np.uint8)


def quantize_int8(x: torch.Tensor) -> torch.Tensor:
    """The int8 quantizing store: round half to even, saturate to [-128, 127]
    (tests/hk/gpu/test_templates_gemm.py:131-140)."""
    return torch.clamp(torch.round(x.float()), -128, 127)


def scaled_mm(a8: torch.Tensor, b8: torch.Tensor, scale_a, scale_b, bias=None) -> torch.Tensor:
    """hk.ops.gemm.scaled_mm's product: (A B^T) * scale_a * scale_b (+ bias), fp8 operands
    exact in fp32, fp32 accumulate, one rounding to bf16 at the store (ops/gemm.py:781-787,
    884-975). scale_a one value or (M,)/(M, 1); scale_b one value or (N,)/(1, N)."""
    m, n = a8.shape[0], b8.shape[0]
    acc = gemm_fp32(a8, b8)
    sa = torch.as_tensor(scale_a, dtype=torch.float32).reshape(-1)
    sb = torch.as_tensor(scale_b, dtype=torch.float32).reshape(-1)
    sa = sa.reshape(m, 1) if sa.numel() == m and m != 1 else sa.reshape(1, -1)[:, :1]
    sb = sb.reshape(1, n) if sb.numel() == n else sb.reshape(1, 1)
    out = acc * sa * sb
    if bias is not None:
        out = out + bias.float().reshape(1, n)
    return out


def rel_to_max(got: torch.Tensor, ref: torch.Tensor) -> float:
    """max |got - ref| / max |ref|: the reference tests' error measure
    (tests/hk/gpu/test_templates_gemm.py:33-35, test_scaled_mm.py:29-32)."""
    ref = ref.float()
    return ((got.float() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def assert_close(got: torch.Tensor, ref: torch.Tensor, rtol: float, atol: float) -> None:
    """Elementwise |got - ref| <= atol + rtol |ref| (bench/dx/common.py:182-207)."""
    torch.testing.assert_close(got.float().cpu(), ref.float().cpu(), rtol=rtol, atol=atol)


__all__ = ["gelu_tanh", "gelu_tanh_exp2", "silu", "silu_and_mul", "relu", "gemm_fp32",
           "gemm_f64", "linear_bias_gelu", "apply_epilogue", "split_k", "e4m3_decode",
           "e4m3_encode", "quantize_int8", "scaled_mm", "rel_to_max", "assert_close", "F"]


# ------------------------------------------------------------------ MX (OCP microscaling) fp8


def e8m0(s: torch.Tensor) -> torch.Tensor:
    """E8M0 scale bytes as fp32: 2^(s - 127) (OCP MX v1.0 section 5.4; byte 255, NaN, unused)."""
    return torch.pow(2.0, s.to(torch.float32) - 127.0)


def mx_quant(x: torch.Tensor):
    """Rows of x to fp8 e4m3 with an E8M0 scale a 32-column block, AITER's per_1x32 rule as the
    reference states it (python/hk/mx.py:17-31): amax >= 2^-126, e = floor(log2 amax) - 8,
    + 1 where amax > 448 * 2^e (so e = ceil(log2(amax / 448))); q = clamp(x / 2^e, +-448) cast
    to e4m3 (nearest even); s = clamp(e + 127, 0, 254). Returns (q float8_e4m3fn, s uint8)."""
    m, k = x.shape
    v = x.float().reshape(m, k // 32, 32)
    amax = v.abs().amax(-1).clamp_min(2.0 ** -126)
    e = torch.floor(torch.log2(amax)) - 8
    e = e + (amax > 448.0 * torch.pow(2.0, e)).float()
    q = (v / torch.pow(2.0, e)[..., None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.reshape(m, k), (e + 127).clamp(0, 254).to(torch.uint8)


def mx_dequant(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """fp8 rows q [M, K] with E8M0 scales s [M, K/32] -> fp32 (python/hk/mx.py:33-37)."""
    return q.float() * e8m0(s).repeat_interleave(32, dim=-1)


def mx_gemm(a: torch.Tensor, b: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor) -> torch.Tensor:
    """(sa . A)(sb . B)^T in fp32 (the reference's check, tests/hk/gpu/test_mxfp8_gemm.py:27-31)."""
    return mx_dequant(a, sa) @ mx_dequant(b, sb).t()
