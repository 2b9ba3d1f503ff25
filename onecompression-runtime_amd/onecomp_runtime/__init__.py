"""onecomp-runtime for MI355X: int4 GPTQ/RTN inference layers on hand-written
gfx950 HIP kernels, behind the reference package's API.

    from onecomp_runtime.diffusion import load_int4_model
    from onecomp_runtime.layers import FusedInt4Linear

All device work goes through ``libonecomp_hip.so`` (C ABI in
``include/onecomp_hip.h``); see :mod:`onecomp_runtime.kernels`.
"""
from __future__ import annotations

from . import backend, kernels, quant_utils
from .diffusion import load_int4_model
from .layers import (
    FusedInt4Linear,
    FusedInt4LinearAnyGroup,
    FusedInt4LinearPaddedGroups,
    GemLiteInt4Linear,
    PackedEmbedding,
    PackedGPTQLinear,
    PackedInt4Conv1d,
    PackedInt4ConvTranspose1d,
    PackedRTNLinear,
    fused_int4_gemm,
    gemlite_available,
    replace_conv_with_packed,
)

__version__ = "0.1.0"

__all__ = [
    "load_int4_model",
    "FusedInt4Linear",
    "FusedInt4LinearAnyGroup",
    "FusedInt4LinearPaddedGroups",
    "fused_int4_gemm",
    "GemLiteInt4Linear",
    "gemlite_available",
    "PackedGPTQLinear",
    "PackedRTNLinear",
    "PackedEmbedding",
    "PackedInt4Conv1d",
    "PackedInt4ConvTranspose1d",
    "replace_conv_with_packed",
    "backend",
    "kernels",
    "quant_utils",
]
