"""hk -- the GEMM-with-fused-epilogue path of hk-dsl, MI355X-native.

    import hk
    y = hk.templates.gemm(x, w, epilogue=hk.templates.gemm.bias_gelu, bias=b)

`hk.templates.gemm` (the template), `hk.ops` (matmul, scaled_mm, the route) and
`hk.integration.vllm_gemm` (the vLLM linear route) keep the reference's Python surface;
behind them every launch is a hand-written gfx950 kernel in libhkx.so, reached through
its C ABI (include/hkx.h)."""

from __future__ import annotations

import importlib

__version__ = "0.1.0"

_SUBMODULES = ("templates", "ops", "integration", "target")


def __getattr__(name):
    if name in _SUBMODULES:
        mod = importlib.import_module(f"{__name__}.{name}")
        globals()[name] = mod
        return mod
    raise AttributeError(f"module 'hk' has no attribute {name!r}")
