"""Packed GPTQ Linear for any groupsize, act-order ``g_idx`` and v1/v2 zeros.

Constructor of the reference's ``PackedGPTQLinear``
(layers/packed_gptq_linear.py:28-88). The reference dequantizes the whole
weight to ``x.dtype`` on every call and then runs ``F.linear`` (:66-74); here
4-bit layers run the fused HIP GEMM instead: act-order rows are sorted by
group once at load time (``oc_int4_plan_groups`` + ``oc_int4_prepare``)
and the kernels read the matching activation columns, so no weight is ever
materialised. The dequantized values are those of ``dequant_gptq_to_fp``
(exact fp32 product, one rounding to the activation type); only the
summation order differs.

fp32 activations and 8-bit layers keep the reference's two-step evaluation,
on the device: a HIP dequant kernel writes the dense weight in ``x.dtype``
and ``F.linear`` multiplies it.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import kernels
from .fused_int4_linear import _HipGPTQLinear


class PackedGPTQLinear(_HipGPTQLinear):
    """nn.Linear-compatible packed GPTQ layer (4- or 8-bit, any groupsize)."""

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
        if g_idx is None:
            g_idx = (torch.arange(in_features, device=qweight.device) // groupsize).to(torch.long)
        if self.wbits == 4:
            self._setup(in_features, out_features, qweight, scales, qzeros, bias, groupsize,
                        g_idx, v1, "packed")
            self.register_buffer("g_idx", g_idx.to(torch.long).contiguous())
        else:
            self.in_features = int(in_features)
            self.out_features = int(out_features)
            self.groupsize = int(groupsize)
            self.v1 = bool(v1)
            self.kmap = None
            self.register_buffer("qweight", qweight.contiguous())
            self.register_buffer("scales", scales.contiguous())
            self.register_buffer("qzeros", qzeros.contiguous())
            self.register_buffer("g_idx", g_idx.to(torch.long).contiguous())
            if bias is not None:
                self.register_buffer("bias", bias.contiguous())
            else:
                self.bias = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.wbits == 4:
            if x.dtype in (torch.float16, torch.bfloat16):
                return self._gemm(x)
            weight = self.dequantize(x.dtype)
        else:
            weight = kernels.int4_dequant(self.qweight, self.scales, self.qzeros, self.g_idx,
                                          self.in_features, self.out_features, x.dtype, v1=self.v1,
                                          wbits=self.wbits)
        bias = self.bias.to(x.dtype) if self.bias is not None else None
        return F.linear(x, weight, bias)

    def _apply(self, fn, recurse=True):
        if self.wbits == 4:
            return super()._apply(fn, recurse=recurse)
        qw, qz = self.qweight, self.qzeros
        result = torch.nn.Module._apply(self, fn, recurse=recurse)
        if self.qweight.dtype != torch.int32:
            self.qweight = qw.to(self.qweight.device)
        if self.qzeros.dtype != torch.int32:
            self.qzeros = qz.to(self.qzeros.device)
        return result

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"wbits={self.wbits}, groupsize={self.groupsize}, packed=True, backend=hip")
