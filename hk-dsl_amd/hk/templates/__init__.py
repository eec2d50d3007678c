"""hk.templates: kernels that own a schedule and take a user hook. This build carries the
GEMM template, `hk.templates.gemm` (python/hk/templates/__init__.py:18-46 binds the
reference's templates the same lazy way)."""

from __future__ import annotations

import importlib

_TEMPLATES = ("gemm",)


def __getattr__(name):
    if name in _TEMPLATES:
        mod = importlib.import_module(f"{__name__}.{name}")
        globals()[name] = mod
        return mod
    raise AttributeError(f"module 'hk.templates' has no attribute {name!r}")


__all__ = list(_TEMPLATES)
