"""Packed int4 / int2 Linear for DeepSeek-V4 QEP weights on the HIP library.

API of the reference's ``layers/dsv4_packed_linear.py`` (dequant_dsv4_packed
:22-56, Dsv4PackedLinear :59-102): ``qweight_packed`` uint8 with ``8 // wbits``
codes per byte along the in-dim, groupwise fp16 ``scales`` / ``qzeros`` in
either orientation, ``w = (q - z) * s`` in fp32 then cast to the compute type.

Where the reference dequantizes the whole weight per call and runs
``F.linear``, fp16/bf16 activations here run one fused kernel
(``oc_dsv4_gemm``, the LDS-tiled MFMA GEMM reading the packed rows directly).
Layers whose buffers stay on the host (routed experts, ``buffer_device="cpu"``)
keep them in pinned memory and stage them per call through
:mod:`onecomp_runtime.offload` (asynchronous copies on a side stream into a
slot pool, overlapping the previous expert's GEMM; ``prefetch()`` starts a
copy early). Shapes the fused kernel does not take (K % 32 != 0, groups not a
multiple of 8) and fp32 activations dequantize on the device
(``oc_dsv4_dequant``, bit-exact) and call ``F.linear``.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import kernels, offload


@torch.no_grad()
def dequant_dsv4_packed(p: dict, dtype: torch.dtype = torch.bfloat16, device=None) -> torch.Tensor:
    """Dense (out, in) weight from a DSV4 packed dict, on the HIP device
    (``device``, else the tensors' device, which must be a HIP device)."""
    qw, sc, qz = p["qweight_packed"], p["scales"], p["qzeros"]
    if device is not None:
        qw, sc, qz = qw.to(device), sc.to(device), qz.to(device)
    return kernels.dsv4_dequant(qw, sc, qz, wbits=int(p["wbits"]), groupsize=int(p["groupsize"]),
                                in_features=int(p["in_features"]), dtype=dtype)


class Dsv4PackedLinear(nn.Module):
    """nn.Linear-compatible packed int4/int2 Linear for DSV4 QEP weights.

    Buffers stay where they are registered (``buffer_device``): on the host
    (pinned) for offloaded experts, staged to the input's device per call; on
    the HIP device for the dense path.
    """

    def __init__(self, packed: dict, bias: torch.Tensor | None = None, buffer_device="cpu") -> None:
        super().__init__()
        self.in_features = int(packed["in_features"])
        self.out_features = int(packed["qweight_packed"].shape[0])
        self.wbits = int(packed["wbits"])
        self.groupsize = int(packed["groupsize"])
        dev = torch.device(buffer_device)
        for name in ("qweight_packed", "scales", "qzeros"):
            t = packed[name].contiguous()
            t = offload.pinned(t) if dev.type == "cpu" else t.to(dev)
            self.register_buffer(name, t)
        if bias is not None:
            self.register_parameter("bias", nn.Parameter(bias.detach(), requires_grad=False))
        else:
            self.bias = None
        self._bias_cache: tuple | None = None

    def _packed_dict(self, qw=None, sc=None, qz=None) -> dict:
        return {"qweight_packed": self.qweight_packed if qw is None else qw,
                "scales": self.scales if sc is None else sc, "qzeros": self.qzeros if qz is None else qz,
                "wbits": self.wbits, "groupsize": self.groupsize, "in_features": self.in_features}

    def _fused_ok(self, x: torch.Tensor) -> bool:
        per = 8 // self.wbits
        rb = self.qweight_packed.shape[1]
        return (x.dtype in (torch.float16, torch.bfloat16) and self.wbits in (2, 4)
                and self.in_features % 32 == 0 and (self.groupsize <= 0 or self.groupsize % 8 == 0)
                and rb >= self.in_features // per and rb % (4 if self.wbits == 4 else 2) == 0)

    def prefetch(self, device: torch.device | str | None = None) -> None:
        """Start copying host-resident buffers to ``device`` (default: the
        current HIP device) on the staging stream; the next forward there
        reuses the copy."""
        if self.qweight_packed.is_cuda:
            return
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        offload.stager.stage([self.qweight_packed, self.scales, self.qzeros], dev, prefetch=True)

    def _device_buffers(self, device: torch.device):
        if self.qweight_packed.device == device:
            return (self.qweight_packed, self.scales, self.qzeros), None
        views, slot = offload.stager.stage([self.qweight_packed, self.scales, self.qzeros], device)
        offload.stager.use(slot)
        return tuple(views), slot

    def _bias_as(self, dtype: torch.dtype) -> torch.Tensor | None:
        b = self.bias
        if b is None:
            return None
        c = self._bias_cache
        if c is not None and c[0] is b and c[1] == b._version and c[2] == dtype and c[3].device == b.device:
            return c[3]
        out = b.to(dtype)
        self._bias_cache = (b, b._version, dtype, out)
        return out

    @property
    def weight(self) -> torch.Tensor:
        """Dequantized dense (out, in) bf16 weight, on the HIP device (host
        buffers are staged to the current device)."""
        dev = self.qweight_packed.device if self.qweight_packed.is_cuda else torch.device(
            "cuda", torch.cuda.current_device())
        (qw, sc, qz), slot = self._device_buffers(dev)
        w = dequant_dsv4_packed(self._packed_dict(qw, sc, qz), dtype=torch.bfloat16)
        if slot is not None:
            offload.stager.release(slot)
        return w

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("Dsv4PackedLinear runs on the HIP device; there is no CPU fallback")
        (qw, sc, qz), slot = self._device_buffers(x.device)
        bias = self._bias_as(x.dtype)
        if bias is not None and bias.device != x.device:
            bias = bias.to(x.device)
        try:
            if self._fused_ok(x):
                y = kernels.dsv4_gemm(x.reshape(-1, self.in_features), qw, sc, qz, wbits=self.wbits,
                                      groupsize=self.groupsize, in_features=self.in_features, bias=bias)
                return y.reshape(*x.shape[:-1], self.out_features)
            w = dequant_dsv4_packed(self._packed_dict(qw, sc, qz), dtype=x.dtype)
            return F.linear(x, w, bias)
        finally:
            if slot is not None:
                offload.stager.release(slot)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"packed=int{self.wbits}, groupsize={self.groupsize}, backend=hip")


def run_routed_experts(experts: list[Dsv4PackedLinear], x: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
    """Y[t * topk + j] = experts[e(t, j)](x[t]) for every routed pair, experts
    taken in id order with the next used experts' weights prefetched while the
    current one computes (host-resident experts). Ids outside [0, E) give zero
    rows. Routing is a stable sort on the device (``oc_moe_route``); the used
    experts' row counts come to the host once."""
    T, topk = topk_ids.shape
    E = len(experts)
    N = experts[0].out_features
    y = torch.zeros((T * topk, N), dtype=x.dtype, device=x.device)
    off, pairs = kernels.moe_route(topk_ids.to(x.device), E)
    counts = off.cpu().tolist()
    used = [e for e in range(E) if counts[e + 1] > counts[e]]
    depth = max(1, offload.stager.num_slots - 1)
    for i in range(min(depth, len(used))):
        experts[used[i]].prefetch(x.device)
    for i, e in enumerate(used):
        if i + depth < len(used):
            experts[used[i + depth]].prefetch(x.device)
        rows = pairs[counts[e]:counts[e + 1]].long()
        y.index_copy_(0, rows, experts[e](x.index_select(0, rows // topk)))
    return y


__all__ = ["Dsv4PackedLinear", "dequant_dsv4_packed", "run_routed_experts"]
