"""Torch-CPU restatement of the reference's two CPU evaluation paths, for the
timed CPU baseline of bench.py: TEST INFRASTRUCTURE ONLY (only tests/ and
bench.py's cpu_baseline leg import it; the product never does).

The reference runs these paths in torch on the host; this module does the
same arithmetic in torch, so the baseline is timed on the same library
(oneDNN / MKL GEMMs, torch integer ops):

  packed  dequantize the whole weight on every call, then F.linear
          (PackedGPTQLinear.forward, layers/packed_gptq_linear.py:66-74;
          PackedRTNLinear.forward, layers/packed_linear.py:53-56)
  eager   dequantize once at load, then F.linear per call
          (backend.build_eager, backend.py:246-264)

Dequantization restates quant_utils.dequant_gptq_to_fp (quant_utils.py:50-69:
integer unpack along K, v1 zero restore, group gather, one fp32 product
rounded to the compute dtype) and dequant_extra_u8_to_weight
(quant_utils.py:72-103: nibble split, every op in the compute dtype).
Pinned by tests/test_oracle.py: the dequantized weights equal the numpy
oracle's bit for bit, the GEMMs are within the oracle's GEMM tolerance.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

_SHIFTS4 = torch.arange(0, 32, 4, dtype=torch.int32)


def unpack_codes(packed: torch.Tensor, num_rows: int, wbits: int = 4) -> torch.Tensor:
    """int32 [R, C] packed along dim 0 -> int32 codes [num_rows, C]
    (quant_utils._unpack_rows, quant_utils.py:12-28)."""
    per = 32 // wbits
    shifts = torch.arange(0, 32, wbits, dtype=torch.int32)
    mask = (1 << wbits) - 1
    R, C = packed.shape
    codes = (packed.unsqueeze(1) >> shifts.view(1, per, 1)) & mask  # [R, per, C]
    return codes.reshape(R * per, C)[:num_rows]


def dequant_gptq(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor, g_idx: torch.Tensor,
                 in_features: int, out_features: int, dtype: torch.dtype, v1: bool = True,
                 wbits: int = 4) -> torch.Tensor:
    """[N, K] weight in ``dtype``: RNE(f32(s[g(k), n]) * f32(code - zero))."""
    mask = (1 << wbits) - 1
    w = unpack_codes(qweight, in_features, wbits)  # [K, N]
    z = unpack_codes(qzeros.t().contiguous(), out_features, wbits).t()  # [G, N]
    if v1:
        z = (z + 1) & mask
    g = g_idx.long()
    prod = scales.float()[g] * (w - z[g]).float()  # [K, N], exact in fp32
    return prod.t().to(dtype)


def rtn_dequant(qweight_u8: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, in_features: int,
                dtype: torch.dtype) -> torch.Tensor:
    """[rows, K] weight, every operation in ``dtype``: RNE(RNE(w - RNE(z)) * RNE(s))."""
    q = qweight_u8.to(torch.int32)
    codes = torch.stack([q & 0xF, q >> 4], dim=-1).reshape(q.shape[0], -1)[:, :in_features]
    w = codes.to(dtype)
    G = scales.shape[1]
    gs = in_features // G
    s = scales.to(dtype).repeat_interleave(gs, dim=1)
    z = zeros.to(dtype).repeat_interleave(gs, dim=1)
    return (w - z) * s


class PackedGPTQ:
    """The packed path: the checkpoint tensors, dequantized on every call."""

    def __init__(self, qweight, scales, qzeros, g_idx, in_features, out_features, dtype, v1=True, bias=None):
        self.args = (qweight, scales, qzeros, g_idx, in_features, out_features)
        self.dtype, self.v1 = dtype, v1
        self.bias = None if bias is None else bias.to(dtype)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        w = dequant_gptq(*self.args, self.dtype, self.v1)
        return F.linear(x, w, self.bias)

    def eager(self) -> "Eager":
        return Eager(dequant_gptq(*self.args, self.dtype, self.v1), self.bias)


class PackedRTN:
    """The packed RTN path (dequant in the compute dtype on every call)."""

    def __init__(self, qweight_u8, scales, zeros, in_features, dtype, bias=None):
        self.args = (qweight_u8, scales, zeros, in_features)
        self.dtype = dtype
        self.bias = None if bias is None else bias.to(dtype)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(x, rtn_dequant(*self.args, self.dtype), self.bias)

    def eager(self) -> "Eager":
        return Eager(rtn_dequant(*self.args, self.dtype), self.bias)


class Eager:
    """The eager path: a dequantized weight kept in the compute dtype."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None):
        self.weight, self.bias = weight, bias

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(x, self.weight, self.bias)


def embedding(ids: torch.Tensor, qweight_u8, scales, zeros, embedding_dim: int) -> torch.Tensor:
    """PackedEmbedding.forward (layers/packed_linear.py:93-104): gather, then
    RTN-dequant in the scales' dtype."""
    flat = ids.reshape(-1).long()
    dtype = scales.dtype if scales.dtype.is_floating_point else torch.float16
    return rtn_dequant(qweight_u8[flat], scales[flat], zeros[flat], embedding_dim, dtype)
