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

fp32 activations and 8-bit layers keep the reference's two-step evaluation,
on the device: a HIP dequant kernel writes the dense weight in ``x.dtype``
and ``F.linear`` multiplies it.

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
        if self.wbits == 4:
            self._setup(in_features, out_features, qweight, scales, qzeros, bias, groupsize,
                        g_idx, v1, "packed")
        else:
            self.in_features = int(in_features)
            self.out_features = int(out_features)
            self.groupsize = int(groupsize)
            self.v1 = bool(v1)
            self._kind = "packed"
            self.kmap = None
            self.register_buffer("_q8_qweight", qweight.contiguous(), persistent=False)
            self.register_buffer("_q8_scales", scales.contiguous(), persistent=False)
            self.register_buffer("_q8_qzeros", qzeros.contiguous(), persistent=False)
            if bias is not None:
                self.register_buffer("bias", bias.contiguous())
            else:
                self.bias = None

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
        if self.wbits == 4:
            if x.dtype in (torch.float16, torch.bfloat16):
                return self._gemm(x, bias=self._bias_as(x.dtype))
            weight = self.dequantize(x.dtype)
        else:
            weight = kernels.int4_dequant(self._q8_qweight, self._q8_scales, self._q8_qzeros, self.g_idx,
                                          self.in_features, self.out_features, x.dtype, v1=self.v1,
                                          wbits=self.wbits)
        return F.linear(x, weight, self._bias_as(x.dtype))

    # 8-bit layers hold the checkpoint tensors themselves.
    def checkpoint_tensors(self):
        if self.wbits == 4:
            return super().checkpoint_tensors()
        return self._q8_qweight, self._q8_scales, self._q8_qzeros

    def load_checkpoint(self, qweight, scales, qzeros, g_idx=None) -> None:
        if self.wbits == 4:
            return super().load_checkpoint(qweight, scales, qzeros, g_idx=g_idx)
        dev = self._q8_qweight.device
        self._q8_qweight = qweight.to(dev).contiguous()
        self._q8_scales = scales.to(dev).contiguous()
        self._q8_qzeros = qzeros.to(dev).contiguous()

    def _apply(self, fn, recurse=True):
        if self.wbits == 4:
            return super()._apply(fn, recurse=recurse)
        qw, qz, gi = self._q8_qweight, self._q8_qzeros, self.g_idx
        result = torch.nn.Module._apply(self, fn, recurse=recurse)
        if self._q8_qweight.dtype != torch.int32:
            self._q8_qweight = qw.to(self._q8_qweight.device)
        if self._q8_qzeros.dtype != torch.int32:
            self._q8_qzeros = qz.to(self._q8_qzeros.device)
        if self.g_idx.dtype != torch.long:
            self.g_idx = gi.to(self.g_idx.device)
        return result

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"wbits={self.wbits}, groupsize={self.groupsize}, packed=True, backend=hip")
