"""GPTQ / RTN unpack and dequant helpers (API of the reference's
``onecomp_runtime.quant_utils``, quant_utils.py:12-103), executed by the HIP
library on the tensors' device.

These helpers accept tensors on a HIP device only; there is no host
implementation in the product.
"""
from __future__ import annotations

import torch

from . import kernels


def _unpack_rows(packed: torch.Tensor, num_rows: int, wbits: int) -> torch.Tensor:
    """Unpack int32-packed ``wbits`` values along dim 0 (quant_utils.py:12-28)."""
    if 32 % wbits != 0:
        raise ValueError(f"wbits must divide 32, got {wbits}")
    return kernels.unpack_rows(packed, num_rows, wbits)


def _unpack_rows_int4(packed: torch.Tensor, num_rows: int) -> torch.Tensor:
    return _unpack_rows(packed, num_rows, 4)


def unpack_int_weights(packed: torch.Tensor, wbits: int,
                       original_shape: tuple[int, int]) -> torch.Tensor:
    """Packed qweight [K/(32/wbits), N] -> int32 [N, K] (quant_utils.py:36-42)."""
    in_features = original_shape[1]
    return _unpack_rows(packed, in_features, wbits).t().contiguous()


def unpack_zeros(packed_zeros: torch.Tensor, wbits: int, out_features: int) -> torch.Tensor:
    """Packed qzeros [G, N/(32/wbits)] -> int32 [G, N] (quant_utils.py:45-47)."""
    return _unpack_rows(packed_zeros.t().contiguous(), out_features, wbits).t().contiguous()


def dequant_gptq_to_fp(
    qweight: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    g_idx: torch.Tensor,
    in_features: int,
    out_features: int,
    dtype: torch.dtype,
    v1: bool = True,
    wbits: int = 4,
) -> torch.Tensor:
    """Dequantize a GPTQ Linear to (out, in) ``dtype`` (quant_utils.py:50-69).

    Bit-exact with the reference: the fp32 product ``s * (w - z)`` (exact for
    16-bit scales) rounded to ``dtype``.
    """
    return kernels.int4_dequant(qweight, scales, qzeros, g_idx, in_features, out_features, dtype,
                                v1=v1, wbits=wbits)


def dequant_extra_u8_to_weight(
    qweight_u8: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    in_features: int,
    out_features: int,
    dtype: torch.dtype,
) -> torch.Tensor:
    """RTN uint8-nibble dequant with per-op rounding in ``dtype`` (quant_utils.py:72-103)."""
    num_groups = scales.shape[1]
    if in_features % num_groups != 0:
        raise RuntimeError(
            f"in_features={in_features} not divisible by num_groups={num_groups}"
        )
    return kernels.rtn_dequant(qweight_u8, scales, zeros, in_features, out_features, dtype)
