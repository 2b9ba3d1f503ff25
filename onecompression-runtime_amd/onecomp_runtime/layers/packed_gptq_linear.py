"""Packed GPTQ Linear for any groupsize, act-order ``g_idx`` and v1/v2 zeros.

Constructor of the reference's ``PackedGPTQLinear``
(layers/packed_gptq_linear.py:28-88). The reference dequantizes the whole
weight to ``x.dtype`` on every call and then runs ``F.linear`` (:66-74); here
4-bit layers run the fused HIP GEMM instead: act-order rows are sorted by
group once at load time (``oc_int4_plan_groups`` + ``oc_int4_prepare``)
and the kernels read the matching activation columns, so no weight is ever
materialised. The dequantized values are those of ``dequant_gptq_to_fp``
(exact fp32 product, one rounding to the activation type); only the
summation order differs. The bias is rounded to ``x.dtype`` first, as the
reference does (:73).

8-bit layers run the same way on their own tiled layout (``oc_int8_prepare``,
``oc_int8_gemm``). fp32 activations keep the reference's two-step
evaluation, on the device: a HIP dequant kernel writes the dense weight in
``x.dtype`` and ``F.linear`` multiplies it.

The module's state is the reference's: ``qweight``, ``scales``, ``qzeros``,
``g_idx`` (and ``bias``) as given.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import kernels
from .fused_int4_linear import _HipGPTQLinear


class PackedGPTQLinear(_HipGPTQLinear):
    """nn.Linear-compatible packed GPTQ layer (4- or 8-bit, any groupsize)."""

    _STATE_LAYOUT = "input"

    def __init__(
        self,
        in_features: int,
        out_features: int,
        qweight: torch.Tensor,
        scales: torch.Tensor,
        qzeros: torch.Tensor,
        g_idx: torch.Tensor | None = None,
        bias: torch.Tensor | None = None,
        groupsize: int = 128,
        wbits: int = 4,
        v1: bool = True,
    ) -> None:
        torch.nn.Module.__init__(self)
        self.wbits = int(wbits)
        if self.wbits not in (4, 8):
            raise ValueError(f"wbits must be 4 or 8, got {wbits}")
        if g_idx is None:
            g_idx = (torch.arange(in_features, device=qweight.device) // groupsize).to(torch.long)
        self._bias_cache: tuple | None = None
        # registered before the bias, as the reference does (state order)
        self.register_buffer("g_idx", g_idx.to(torch.long).contiguous())
        self._setup(in_features, out_features, qweight, scales, qzeros, bias, groupsize, g_idx, v1, "packed",
                    wbits=self.wbits)

    def _bias_as(self, dtype: torch.dtype) -> torch.Tensor | None:
        """``bias.to(x.dtype)`` (packed_gptq_linear.py:73), cached per dtype."""
        b = self.bias
        if b is None:
            return None
        c = self._bias_cache
        if c is not None and c[0] is b and c[1] == b._version and c[2] == dtype:
            return c[3]
        out = b.to(dtype)
        self._bias_cache = (b, b._version, dtype, out)
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype in (torch.float16, torch.bfloat16):
            return self._gemm(x, bias=self._bias_as(x.dtype))
        # fp32 activations: the reference's evaluation, dequantize to x.dtype
        # (exact fp32 products) then F.linear
        return F.linear(x, self.dequantize(x.dtype), self._bias_as(x.dtype))

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"wbits={self.wbits}, groupsize={self.groupsize}, packed=True, backend=hip")
