"""forge_amd -- MI355X-native (gfx950) rebuild of Forge-LLM's quantized-linear hot path.

The W4A16 / FP8 / INT8 GEMM family behind the reference's ``forge.kernels.ops_gemm`` surface, computed only by
hand-written HIP kernels in ``libforge_mi355x.so`` (C ABI: ``include/forge_mi355x.h``).  Import the ops from
``forge_amd.ops_gemm`` and the packed formats from ``forge_amd.layouts``.
"""
from __future__ import annotations

from . import errors, layouts, ops_gemm
from .errors import ConfigError, HardwareUnsupported, NotFound

__version__ = "0.1.0"

__all__ = ["ConfigError", "HardwareUnsupported", "NotFound", "errors", "layouts", "ops_gemm"]
