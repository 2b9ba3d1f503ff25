"""RTN uint8-nibble Linear and Embedding on the HIP library.

API of the reference's ``layers/packed_linear.py`` (PackedRTNLinear :22-63,
PackedEmbedding :65-110). Weights stay packed (two 4-bit codes per byte, low
nibble first); dequant follows ``dequant_extra_u8_to_weight``
(quant_utils.py:72-103), every operation rounded to the compute dtype.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _hip, kernels


class PackedRTNLinear(nn.Module):
    """nn.Linear-compatible RTN int4 packed Linear.

    fp16/bf16 activations run the fused ``oc_rtn_linear`` kernel; fp32
    activations (and shapes the fused kernel does not take: K % 32 != 0 or
    groups of a size not divisible by 8) dequantize on the device with
    ``oc_rtn_dequant`` and call ``F.linear``, as the reference does.
    """

    def __init__(
        self,
        in_features: int,
        out_features: int,
        qweight_u8: torch.Tensor,
        scales: torch.Tensor,
        zeros: torch.Tensor,
        bias: torch.Tensor | None = None,
    ) -> None:
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.register_buffer("qweight_u8", qweight_u8.contiguous())
        self.register_buffer("scales", scales.contiguous())
        self.register_buffer("zeros", zeros.contiguous())
        if bias is not None:
            self.register_parameter("bias", nn.Parameter(bias.detach(), requires_grad=False))
        else:
            self.bias = None

    def _fused_ok(self, x: torch.Tensor) -> bool:
        K, G = self.in_features, self.scales.shape[1]
        return (x.dtype in (torch.float16, torch.bfloat16) and K % 32 == 0 and K % G == 0
                and (K // G) % 8 == 0 and self.out_features % 8 == 0
                and self.qweight_u8.shape[1] % 4 == 0)

    def _materialize(self, dtype: torch.dtype) -> torch.Tensor:
        return kernels.rtn_dequant(self.qweight_u8, self.scales, self.zeros, self.in_features,
                                   self.out_features, dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        bias = self.bias.to(x.dtype) if self.bias is not None else None
        if self._fused_ok(x):
            c = kernels.rtn_linear(x.reshape(-1, self.in_features), self.qweight_u8, self.scales,
                                   self.zeros, self.in_features, bias)
            return c.reshape(*x.shape[:-1], self.out_features)
        return F.linear(x, self._materialize(x.dtype), bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, packed=int4, backend=hip")


class PackedEmbedding(nn.Module):
    """nn.Embedding-compatible RTN int4 packed table (one gather+dequant launch).

    Output dtype is the scales' dtype, or fp16 for non-float scales
    (packed_linear.py:98). Ids outside ``[-V, V)`` produce zero rows and set
    ``self.bad_id_flag`` (a device int32, checked on demand by
    :meth:`check_ids`); the reference's torch indexing raises instead.
    """

    def __init__(
        self,
        num_embeddings: int,
        embedding_dim: int,
        qweight_u8: torch.Tensor,
        scales: torch.Tensor,
        zeros: torch.Tensor,
        padding_idx: int | None = None,
    ) -> None:
        super().__init__()
        self.num_embeddings = int(num_embeddings)
        self.embedding_dim = int(embedding_dim)
        self.padding_idx = padding_idx
        self.register_buffer("qweight_u8", qweight_u8.contiguous())
        self.register_buffer("scales", scales.contiguous())
        self.register_buffer("zeros", zeros.contiguous())
        self.register_buffer("bad_id_flag", torch.zeros(1, dtype=torch.int32,
                                                        device=qweight_u8.device), persistent=False)
        self._call = None  # the table's fixed call arguments, bound at the first device forward

    def _bind(self, q, sc, z, flag) -> tuple:
        dtype = sc.dtype if sc.dtype.is_floating_point else torch.float16
        mid = (q.data_ptr(), q.shape[0], q.shape[1], sc.data_ptr(), _hip.dtype_code(sc.dtype), z.data_ptr(),
               _hip.dtype_code(z.dtype), sc.shape[1], self.embedding_dim)
        return (q, sc, z, flag, q.get_device(), dtype, mid, _hip.dtype_code(dtype), flag.data_ptr())

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        b = self._buffers
        q, sc, z, flag = b["qweight_u8"], b["scales"], b["zeros"], b["bad_id_flag"]
        call = self._call
        if q.is_cuda and (call is None or call[0] is not q or call[1] is not sc or call[2] is not z
                          or call[3] is not flag or call[6][0] != q.data_ptr()):
            call = self._call = self._bind(q, sc, z, flag)
        ids = input_ids
        if (call is not None and q.is_cuda and ids.is_cuda and ids.dtype is torch.int64 and ids.is_contiguous()
                and ids.get_device() == call[4] and sc.is_cuda and z.is_cuda and flag.is_cuda):
            # Fast path: ids already int64 and contiguous on the table's device.
            T = ids.numel()
            rows = torch.empty((T, self.embedding_dim), dtype=call[5], device=ids.device)
            _hip.check(_hip.lib().oc_rtn_embedding(ids.data_ptr(), T, *call[6], rows.data_ptr(), call[7], call[8],
                                                   _hip._raw_stream(call[4])), "oc_rtn_embedding")
        else:
            dtype = sc.dtype if sc.dtype.is_floating_point else torch.float16
            rows = kernels.rtn_embedding(input_ids, q, sc, z, self.embedding_dim, dtype, flag)
        return rows.reshape(*input_ids.shape, self.embedding_dim)

    def check_ids(self) -> None:
        """Raise IndexError if any lookup so far used an out-of-range id."""
        if int(self.bad_id_flag.item()) != 0:
            self.bad_id_flag.zero_()
            raise IndexError(f"embedding id out of range for num_embeddings={self.num_embeddings}")

    def extra_repr(self) -> str:
        return (f"num_embeddings={self.num_embeddings}, "
                f"embedding_dim={self.embedding_dim}, packed=int4, backend=hip")
