"""hk.integration: engine routes onto this build's kernels -- `vllm_gemm` (vLLM's
unquantized linear layers) and `vllm_mxfp8` (its block-scaled MXFP8 ones) over `engine`
(custom op, CUDA-graph contract, route table); `tune` measures the route tables."""

from . import engine  # noqa: F401

__all__ = ["engine", "vllm_gemm", "vllm_mxfp8", "tune"]


def __getattr__(name):
    if name in ("vllm_gemm", "vllm_mxfp8", "tune"):
        import importlib

        mod = importlib.import_module(f"{__name__}.{name}")
        globals()[name] = mod
        return mod
    raise AttributeError(name)
