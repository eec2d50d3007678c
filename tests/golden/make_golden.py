"""Writes tests/golden/golden.npz: inputs and expected outputs for the GEMM-with-epilogue
path, computed here in numpy float64 from the formulas' definitions -- independently of
oracle/gemm_oracle.py, which the CPU tests then check against these vectors.

The reference holds no golden-vector files for this path (its tests compute a torch fp32
reference at run time, tests/hk/gpu/test_templates_gemm.py:26-70), so these are made from
seeded inputs of the configs' distributions:

* config 1 (bench/dx/tasks/t4_linear_bias_gelu): x bf16[256, 1024] ~N(0,1), w bf16[1024,
  1024] ~N(0, 0.02) (K, N), b bf16[1024] ~N(0, 0.1), seeds 0/1/2 -- the sha256 of each
  input's bytes and the first 16 rows of y = gelu_tanh(x @ w + b);
* tiny shapes for every ready-made epilogue, M in {1, 5, 17}, N in {128, 256},
  K in {64, 128} -- inputs and outputs whole;
* fp8 e4m3: all 256 codes' values, decoded from the format definition;
* the fp8 dequant product on a tiny shape.

    python tests/golden/make_golden.py      # rewrites golden.npz
"""

from __future__ import annotations

import hashlib
import math
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "golden.npz"


def bf16_np(t: torch.Tensor) -> np.ndarray:
    """A bf16 tensor's values as float64 (exact)."""
    return t.float().numpy().astype(np.float64)


def gelu64(x):
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def silu64(x):
    return x / (1.0 + np.exp(-x))


def e4m3_value(code: int) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 7
    if e == 15 and m == 7:
        return float("nan")
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1 + m / 8) * 2.0 ** (e - 7)


def cfg1(seed: int):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(256, 1024, generator=g).to(torch.bfloat16)
    w = (torch.randn(1024, 1024, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(1024, generator=g) * 0.1).to(torch.bfloat16)
    return x, w, b


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.view(torch.int16).numpy().tobytes()).hexdigest()


def main():
    d = {}
    for seed in (0, 1, 2):
        x, w, b = cfg1(seed)
        y = gelu64(bf16_np(x)[:16] @ bf16_np(w) + bf16_np(b))
        d[f"cfg1_s{seed}_sha"] = np.array([sha(x), sha(w), sha(b)])
        d[f"cfg1_s{seed}_y16"] = y.astype(np.float32)
    g = torch.Generator().manual_seed(1234)
    for m in (1, 5, 17):
        for n in (128, 256):
            for k in (64, 128):
                a = torch.randn(m, k, generator=g).to(torch.bfloat16)
                bb = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16)
                bias = torch.randn(n, generator=g).to(torch.bfloat16)
                res = torch.randn(m, n, generator=g).to(torch.bfloat16)
                sc = (torch.rand(m, 1, generator=g) + 0.5)
                acc = bf16_np(a) @ bf16_np(bb).T
                key = f"t_{m}_{n}_{k}"
                d[key + "_a"], d[key + "_b"] = a.view(torch.int16).numpy(), bb.view(torch.int16).numpy()
                d[key + "_bias"], d[key + "_res"] = bias.view(torch.int16).numpy(), res.view(torch.int16).numpy()
                d[key + "_scale"] = sc.numpy()
                bi, re_ = bf16_np(bias), bf16_np(res)
                d[key + "_acc"] = acc
                d[key + "_bias_gelu"] = gelu64(acc + bi)
                d[key + "_bias_silu"] = silu64(acc + bi)
                d[key + "_bias_relu"] = np.maximum(acc + bi, 0.0)
                d[key + "_bias_residual"] = acc + bi + re_
                d[key + "_scale_out"] = acc * sc.numpy().astype(np.float64)
                if n == 256:
                    d[key + "_silu_and_mul"] = silu64(acc[:, :128]) * acc[:, 128:]
    d["e4m3_values"] = np.array([e4m3_value(c) for c in range(256)], dtype=np.float64)
    g = torch.Generator().manual_seed(99)
    a8 = (torch.randn(5, 128, generator=g) * 3).to(torch.float8_e4m3fn)
    b8 = (torch.randn(64, 128, generator=g) * 3).to(torch.float8_e4m3fn)
    sa = (torch.rand(5, 1, generator=g) * 1.5 + 0.5) / 448
    sb = (torch.rand(64, generator=g) * 1.5 + 0.5) / 448
    bias = (torch.randn(64, generator=g) * 0.1).to(torch.bfloat16)
    vals = d["e4m3_values"]
    a64 = vals[a8.view(torch.uint8).numpy().astype(np.int64)]
    b64 = vals[b8.view(torch.uint8).numpy().astype(np.int64)]
    d["fp8_a"], d["fp8_b"] = a8.view(torch.uint8).numpy(), b8.view(torch.uint8).numpy()
    d["fp8_sa"], d["fp8_sb"] = sa.numpy(), sb.numpy()
    d["fp8_bias"] = bias.view(torch.int16).numpy()
    d["fp8_out"] = (a64 @ b64.T) * sa.numpy().astype(np.float64) * sb.numpy().astype(np.float64) \
        + bf16_np(bias)
    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(d)} arrays)")


if __name__ == "__main__":
    main()
