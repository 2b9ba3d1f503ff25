"""Int4 inference layers executed by the HIP library (gfx950).

- :class:`FusedInt4Linear` / :func:`fused_int4_gemm` - GPTQ groupsize-32 int4
  Linear (v1 or v2 zeros), fused dequant + GEMM.
- :class:`FusedInt4LinearPaddedGroups` - odd groupsizes re-laid into 32-row groups.
- :class:`FusedInt4LinearAnyGroup` - any groupsize.
- :class:`PackedGPTQLinear` - any groupsize, act-order ``g_idx``, 4/8-bit.
- :class:`PackedRTNLinear` / :class:`PackedEmbedding` - RTN uint8-nibble layers.
- :class:`PackedInt4Conv1d` / :class:`PackedInt4ConvTranspose1d` - RTN int4
  convolutions run as GEMMs over the packed rows.
- :class:`Dsv4PackedLinear` - DeepSeek-V4 QEP int4/int2 layers, host-resident
  experts staged to the device per call.
- :class:`GemLiteInt4Linear` / :func:`gemlite_available` - import-compatible
  names only (GemLite, a Triton library, is never available on this HIP package).
"""
from __future__ import annotations

from .fused_int4_linear import (
    FusedInt4Linear,
    FusedInt4LinearAnyGroup,
    FusedInt4LinearPaddedGroups,
    fused_int4_gemm,
)
from .dsv4_packed_linear import Dsv4PackedLinear, dequant_dsv4_packed, run_routed_experts
from .gemlite_int4_linear import GemLiteInt4Linear, gemlite_available
from .packed_gptq_linear import PackedGPTQLinear
from .packed_conv import (
    PackedInt4Conv1d,
    PackedInt4ConvTranspose1d,
    pack_int4_nibbles,
    quantize_conv_module,
    quantize_conv_weight,
    replace_conv_with_packed,
    unpack_int4_nibbles,
)
from .packed_linear import PackedEmbedding, PackedRTNLinear

__all__ = [
    "FusedInt4Linear",
    "FusedInt4LinearAnyGroup",
    "FusedInt4LinearPaddedGroups",
    "fused_int4_gemm",
    "GemLiteInt4Linear",
    "gemlite_available",
    "PackedGPTQLinear",
    "PackedRTNLinear",
    "PackedEmbedding",
    "Dsv4PackedLinear",
    "PackedInt4Conv1d",
    "PackedInt4ConvTranspose1d",
    "pack_int4_nibbles",
    "unpack_int4_nibbles",
    "quantize_conv_weight",
    "quantize_conv_module",
    "replace_conv_with_packed",
    "dequant_dsv4_packed",
    "run_routed_experts",
]
