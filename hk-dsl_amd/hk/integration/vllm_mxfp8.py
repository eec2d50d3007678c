"""vLLM's block-scaled MXFP8 linear layers on this build's MX GEMM (gfx950).

Restates python/hk/integration/vllm_mxfp8.py (:1-225): vLLM serves 32 x 32 block-scaled
MXFP8 checkpoints on gfx950 with `RocmDotScaledMxfp8LinearKernel`, whose `apply_weights`
quantizes the activation (`mxfp8_e4m3_quantize`, AITER's per_1x32 rule) and calls
`rocm_mxfp8_block32_gemm`. The patch wraps that class's two entry points:

* `process_weights_after_loading` runs vLLM's, then lays the weight's 32 x 32 block scales
  out one row each (`mxfp8.expand_block_scales`) beside vLLM's -- the OCP layout this build's
  kernel reads;
* `apply_weights` makes one call of the opaque op `hk_vllm::mxfp8_linear`. Inside it, where
  M is a number, a call the route takes (`schedule`) quantizes the activation in one launch
  (`mxfp8.quant`, the same bits as vLLM's quantizer) and runs `mxfp8.gemm`; every other
  call runs vLLM's own quant and kernel.

The route: N a multiple of 8 and K of 128 (the kernel's), then the measured table
hk/tuned/routes_vllm_mxfp8_gfx950.json (`python -m hk.integration.tune vllm_mxfp8`; `$HK_VLLM_MXFP8_ROUTES`
overrides it): for each measured (N, K), the Ms where hk's quant + MX GEMM beat the
engine's by 3% (a shape it does not hold stays with vLLM, as the reference routes only the
shapes it measured, :33-56). Without a table, M >= MIN_M, the reference's measured bound
(:35-36). `ENABLED = False` sends every call to vLLM.
"""

from __future__ import annotations

from typing import Callable, Dict, Optional

from . import engine

#: The smallest M routed to hk.
MIN_M = 2048
#: Route hk-able calls to hk (True) or leave every call to vLLM (False).
ENABLED = True


def _fake(x, w, ws, hk_ws, out_dtype):
    return x.new_empty((x.shape[0], w.shape[0]), dtype=out_dtype)


PATCH = engine.Op("hk_vllm::mxfp8_linear",
                  "mxfp8_linear(Tensor x, Tensor w, Tensor ws, Tensor hk_ws, ScalarType out_dtype)"
                  " -> Tensor", _fake, paths=("hk", "fallback"), graph="safe")


ROUTES_ENV = "HK_VLLM_MXFP8_ROUTES"
_TABLE: list = []


def routes() -> Optional[engine.RouteTable]:
    """The measured table for this process's arch (loaded once), or None."""
    if not _TABLE:
        from ..target import current_arch  # noqa: PLC0415

        _TABLE.append(engine.shipped_table("vllm_mxfp8", current_arch(), ROUTES_ENV))
    return _TABLE[0]


def set_routes(table: Optional[engine.RouteTable]) -> None:
    """Route by `table` from now on; None reloads the shipped one."""
    _TABLE.clear()
    if table is not None:
        _TABLE.append(table)


def schedule(m: int, n: int, k: int) -> bool:
    """Whether hk takes an M x N x K call."""
    if not ENABLED or n % 8 or k % 128 or m < 1:
        return False
    t = routes()
    if t is None:
        return m >= MIN_M
    return t.lookup(m, n, k) == "hk"


class _VllmKernel:
    """vLLM's own quant and GEMM for MXFP8 linears, imported on first use."""

    quantize: Optional[Callable] = None
    gemm: Optional[Callable] = None

    @classmethod
    def load(cls):
        if cls.gemm is None:
            from vllm.model_executor.kernels.linear.mxfp8.rocm_block32_gemm import (  # noqa: PLC0415
                rocm_mxfp8_block32_gemm)
            from vllm.model_executor.layers.quantization.utils.mxfp8_utils import (  # noqa: PLC0415
                mxfp8_e4m3_quantize)

            cls.quantize, cls.gemm = mxfp8_e4m3_quantize, rocm_mxfp8_block32_gemm
        return cls


def mxfp8_linear(x, w, ws, hk_ws, out_dtype):
    """MXFP8-quantized bf16 x [M, K] @ w.T for a 32 x 32 block-scaled fp8 w [N, K]: this
    build's quant and GEMM where the route takes the call, vLLM's otherwise."""
    import torch  # noqa: PLC0415

    from ..ops import mxfp8  # noqa: PLC0415

    m, k = x.shape
    if out_dtype == torch.bfloat16 and hk_ws.numel() and schedule(m, w.shape[0], k):
        PATCH.count("hk")
        return mxfp8.linear(x, w, hk_ws)
    PATCH.count("fallback")
    v = _VllmKernel.load()
    xq, xs = v.quantize(x)
    return v.gemm(xq, xs, w, ws, out_dtype)


def _kernel_class():
    from vllm.model_executor.kernels.linear.mxfp8 import rocm_native  # noqa: PLC0415

    return rocm_native.RocmDotScaledMxfp8LinearKernel


class _MethodSwap:
    """Methods of one class replaced by ours, with the originals kept to call through and
    to put back."""

    def __init__(self):
        self.cls = None
        self.orig: Dict[str, Callable] = {}

    @property
    def active(self) -> bool:
        return self.cls is not None

    def install(self, cls, ours: Dict[str, Callable]) -> None:
        self.cls = cls
        self.orig = {name: cls.__dict__[name] if name in cls.__dict__ else getattr(cls, name)
                     for name in ours}
        for name, fn in ours.items():
            setattr(cls, name, fn)

    def restore(self) -> None:
        for name, fn in self.orig.items():
            setattr(self.cls, name, fn)
        self.cls, self.orig = None, {}


SWAP = _MethodSwap()


def process_weights_after_loading(self, layer) -> None:
    """vLLM's, then the weight's block scales one row each (the OCP layout this build's
    kernel reads), kept beside vLLM's as `layer.hk_ws`."""
    import torch  # noqa: PLC0415

    from ..ops import mxfp8  # noqa: PLC0415

    SWAP.orig["process_weights_after_loading"](self, layer)
    w, ws = layer.weight, layer.weight_scale
    n, k = w.shape
    block_scaled = ws.shape[0] != n and w.element_size() == 1
    if not block_scaled or n % 8 or k % 128:
        return
    rows = mxfp8.expand_block_scales(ws.data.view(torch.uint8))[:n]
    layer.hk_ws = torch.nn.Parameter(rows, requires_grad=False)


def apply_weights(self, layer, x, bias=None):
    """One call of the op for a layer with hk's scales; vLLM's for any other layer."""
    if not hasattr(layer, "hk_ws"):
        return SWAP.orig["apply_weights"](self, layer, x, bias)
    n = layer.weight.shape[0]
    y = PATCH(x.reshape(-1, x.shape[-1]), layer.weight, layer.weight_scale, layer.hk_ws,
              x.dtype).reshape(*x.shape[:-1], n)
    return y if bias is None else y + bias


def apply_patch() -> str:
    """Route vLLM's block-scaled MXFP8 linear layers. Returns what happened, in one line."""
    import importlib.util  # noqa: PLC0415

    if importlib.util.find_spec("vllm") is None:
        return "vllm is not importable; mxfp8 not patched"
    if SWAP.active:
        return "mxfp8: already patched"
    from ..target import current_arch  # noqa: PLC0415

    arch = current_arch()
    if arch != "gfx950":
        return f"mxfp8: not patched -- the MX GEMM is gfx950's scaled MFMA, not {arch}"
    PATCH.define(mxfp8_linear)
    SWAP.install(_kernel_class(), {"process_weights_after_loading": process_weights_after_loading,
                                   "apply_weights": apply_weights})
    cache = engine.isolate_compile_cache("mxfp8")
    t = routes()
    where = f"{t.source} measured it faster" if t is not None else f"M >= {MIN_M}"
    return f"mxfp8 -> hk where {where} (compile cache {cache})"


def revert() -> str:
    if not SWAP.active:
        return "mxfp8: not patched"
    SWAP.restore()
    return "mxfp8 -> vllm"


def status() -> str:
    return PATCH.summary() if SWAP.active else "not patched"


__all__ = ["PATCH", "schedule", "routes", "set_routes", "mxfp8_linear", "apply_patch", "revert",
           "status", "process_weights_after_loading", "apply_weights"]
