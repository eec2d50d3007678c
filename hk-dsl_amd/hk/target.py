"""Facts about the target, gfx950 (MI355X / CDNA4), that the plans and the roofline
reports read (the reference's python/hk/target/gfx950.py:40-91, restated)."""

from __future__ import annotations

import os
from dataclasses import dataclass


@dataclass(frozen=True)
class Target:
    name: str
    wave: int
    cus: int
    xcds: int
    lds_bytes: int
    vgprs: int          # unified VGPR + AGPR entries a lane, at one wave per SIMD
    mfma_bf16: tuple    # (M, N, K) shapes used here
    mfma_fp8: tuple


GFX950 = Target(name="gfx950", wave=64, cus=256, xcds=8, lds_bytes=160 * 1024, vgprs=512,
                mfma_bf16=((16, 16, 32), (32, 32, 16)), mfma_fp8=((16, 16, 128), (32, 32, 64)))

#: Datasheet ceilings every roofline fraction is taken against (dense, no sparsity).
CEILINGS = {"bf16_tflops": 2500.0, "fp16_tflops": 2500.0, "fp8_tflops": 5000.0,
            "hbm_gbs": 8000.0}


def current_arch() -> str:
    """The arch the plans are made for: $HK_ARCH, else gfx950 (the only one this build's
    kernels are compiled for)."""
    return os.environ.get("HK_ARCH", "gfx950")


def get_target(arch: str = "gfx950") -> Target:
    if arch != "gfx950":
        raise ValueError(f"no target {arch!r} in this build (gfx950 only)")
    return GFX950


__all__ = ["Target", "GFX950", "CEILINGS", "current_arch", "get_target"]
