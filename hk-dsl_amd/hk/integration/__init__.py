"""hk.integration: engine routes onto this build's kernels -- `vllm_gemm` (vLLM's
unquantized linear layers) over `engine` (custom op, CUDA-graph contract, route table)."""

from . import engine  # noqa: F401

__all__ = ["engine", "vllm_gemm"]


def __getattr__(name):
    if name == "vllm_gemm":
        import importlib

        mod = importlib.import_module(f"{__name__}.vllm_gemm")
        globals()[name] = mod
        return mod
    raise AttributeError(name)
