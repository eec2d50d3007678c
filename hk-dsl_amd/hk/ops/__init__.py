"""hk.ops: the GEMM entry points of this build -- `matmul` (bf16), `scaled_mm` (fp8 with
per-token x per-channel dequant), `mxfp8` (MX block-scaled fp8) and the gfx950 route
(`gemm_cdna`)."""

from . import gemm_cdna, mxfp8  # noqa: F401
from .gemm import matmul, scaled_mm  # noqa: F401

__all__ = ["matmul", "scaled_mm", "gemm_cdna", "mxfp8"]
