"""Fused int4 dequant + GEMM layers on the HIP library.

API of the reference's ``layers/fused_int4_linear.py`` (FusedInt4Linear
:958-1246, fused_int4_gemm :388-537, FusedInt4LinearPaddedGroups :761-955,
FusedInt4LinearAnyGroup :639-758). Every forward is one launch of
``oc_int4_gemm`` on torch's current stream.

Layout. All classes share one load-time plan (``oc_int4_plan_groups``):
the packed rows are re-laid into uniform groups of ``group_rows`` (a
multiple of 32) physical rows -- odd group sizes get 32-row slots with zero
rows (the reference's ``_repack_groups_to_32``, :94-124), act-order ``g_idx``
sorts rows by group -- and ``oc_int4_prepare`` writes the weight once into
the tiled device layout the kernels stream: 16-column tiles whose 32-row
steps are 256 contiguous bytes, with the tile's scales and zeros (restored
to their value, so v1 and v2 checkpoints run the same kernels) beside them.
The layer keeps only the tiled tensors (``qweight_tiled``, ``scales_tiled``,
``zeros_tiled``); checkpoint-format tensors given on the CPU are held until
the first device forward prepares them.
"""
from __future__ import annotations

import torch

from .. import _hip, _profile, kernels


class _HipGPTQLinear(torch.nn.Module):
    """Shared state and forward of the packed GPTQ int4 layers."""

    def _setup(self, in_features: int, out_features: int, qweight: torch.Tensor,
               scales: torch.Tensor, qzeros: torch.Tensor, bias: torch.Tensor | None,
               groupsize: int, g_idx: torch.Tensor | None, v1: bool, kind: str) -> None:
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.groupsize = int(groupsize)
        self.v1 = bool(v1)
        self._kind = kind
        if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
            raise ValueError("qweight and qzeros must be int32")
        if self.out_features % 8 != 0:
            raise ValueError(f"out_features must be a multiple of 8, got {self.out_features}")
        if qweight.shape[1] != self.out_features:
            raise ValueError(f"qweight has {qweight.shape[1]} columns, expected {self.out_features}")
        rows_expected = (self.in_features + 7) // 8
        if qweight.shape[0] < rows_expected:
            raise ValueError(f"qweight K-dim mismatch: got {qweight.shape[0]}, expected {rows_expected}")
        plan = kernels.plan_groups(self.in_features, self.groupsize, g_idx)
        if scales.shape[0] < plan.num_groups or scales.shape[1] != self.out_features:
            raise ValueError(f"scales shape {tuple(scales.shape)} does not cover "
                             f"{plan.num_groups} groups x {self.out_features}")
        if tuple(qzeros.shape[1:]) != (self.out_features // 8,) or qzeros.shape[0] < plan.num_groups:
            raise ValueError(f"qzeros shape {tuple(qzeros.shape)} does not cover "
                             f"{plan.num_groups} groups x {self.out_features // 8}")
        self.k_phys = plan.k_phys
        self.group_rows = plan.group_rows
        self.num_phys_groups = plan.num_groups
        if scales.dtype not in (torch.float16, torch.bfloat16):
            scales = scales.to(torch.float16)
        # The kernels read activations through kmap (physical -> input row) and
        # kinv (input -> physical row) only when the rows moved.
        kmap, kinv = kernels.row_maps(plan, qweight.device)
        self.register_buffer("kmap", kmap, persistent=False)
        self.register_buffer("kinv", kinv, persistent=False)
        self.register_buffer("qweight_tiled", None)
        self.register_buffer("scales_tiled", None)
        self.register_buffer("zeros_tiled", None)
        # Checkpoint-format tensors waiting for the first device forward.
        self.register_buffer("_src_qweight", qweight, persistent=False)
        self.register_buffer("_src_scales", scales, persistent=False)
        self.register_buffer("_src_qzeros", qzeros, persistent=False)
        if bias is not None:
            self.register_buffer("bias", bias.contiguous())
        else:
            self.bias = None
        self._weights = None
        if qweight.is_cuda:
            self._prepare()

    def _prepare(self) -> kernels.TiledWeights:
        """Write the tiled layout on the layer's device and drop the sources."""
        w = kernels.prepare(self._src_qweight, self._src_scales, self._src_qzeros,
                            in_features=self.in_features, out_features=self.out_features,
                            kmap=self.kmap, k_phys=self.k_phys, group_rows=self.group_rows, v1=self.v1)
        self.qweight_tiled, self.scales_tiled, self.zeros_tiled = w.qt, w.st, w.zt
        self._src_qweight = self._src_scales = self._src_qzeros = None
        self._weights = w
        return w

    def tiled(self) -> kernels.TiledWeights:
        w = self._weights
        if w is None or w.qt is not self.qweight_tiled or w.st is not self.scales_tiled:
            if self.qweight_tiled is None:
                if not self._src_qweight.is_cuda:
                    raise RuntimeError(
                        f"{type(self).__name__} runs on the HIP device; move the layer there first "
                        f"(its weights are on {self._src_qweight.device})")
                return self._prepare()
            w = kernels.TiledWeights(self.qweight_tiled, self.scales_tiled, self.zeros_tiled,
                                     self.out_features, self.k_phys, self.group_rows)
            self._weights = w
        return w

    def _gemm(self, x: torch.Tensor) -> torch.Tensor:
        orig_dtype = x.dtype
        if orig_dtype == torch.float32:
            # fp32 input is computed in fp16 and returned as fp32
            # (fused_int4_linear.py:415-419, :535-536).
            x = x.to(torch.float16)
        a_2d = x.reshape(-1, self.in_features)
        if _profile.PROFILE_SHAPES:
            _profile.record(self._kind, a_2d.shape[0], self.in_features, self.out_features)
        c = kernels.int4_gemm(a_2d, self.tiled(), in_features=self.in_features, kmap=self.kmap,
                              kinv=self.kinv, bias=self.bias)
        out = c.reshape(*x.shape[:-1], self.out_features)
        if orig_dtype == torch.float32:
            out = out.to(torch.float32)
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._gemm(x)

    def dequantize(self, dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """Dense [out_features, in_features] weight, values as the reference's
        ``dequant_gptq_to_fp`` (exact fp32 product, one rounding to dtype)."""
        return kernels.dequant_tiled(self.tiled(), self.kmap, self.in_features, dtype)

    @torch.no_grad()
    def warmup(self, m_values=(32, 128, 256, 1024, 2250)) -> None:
        """Run one forward per M so workspaces are sized before timing.

        The kernels are compiled ahead of time; there is no JIT to trigger.
        """
        ref = self.qweight_tiled if self.qweight_tiled is not None else self._src_qweight
        device = ref.device
        if device.type != "cuda":
            return
        scales = self.scales_tiled if self.scales_tiled is not None else self._src_scales
        dtype = scales.dtype if scales.dtype in (torch.float16, torch.bfloat16) else torch.float16
        for m in m_values:
            if m <= 0:
                continue
            self.forward(torch.zeros((int(m), self.in_features), dtype=dtype, device=device))
        torch.cuda.synchronize(device)

    def _apply(self, fn, recurse=True):
        # Keep integer buffers int32 across .to(dtype=...) and scales 16-bit
        # (fused_int4_linear.py:1230-1246).
        before = {n: getattr(self, n) for n in ("qweight_tiled", "zeros_tiled", "kmap", "_src_qweight",
                                                "_src_qzeros")}
        kinv_before = self.kinv
        result = super()._apply(fn, recurse=recurse)
        for name, old in before.items():
            new = getattr(self, name)
            if new is not None and new.dtype != torch.int32:
                setattr(self, name, old.to(new.device))
        if self.kinv is not None and self.kinv.dtype != torch.int16:
            self.kinv = kinv_before.to(self.kinv.device)
        for name in ("scales_tiled", "_src_scales"):
            t = getattr(self, name)
            if t is not None and t.dtype not in (torch.float16, torch.bfloat16):
                setattr(self, name, t.to(torch.float16))
        return result

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"groupsize={self.groupsize}, v1={self.v1}, k_phys={self.k_phys}, "
                f"group_rows={self.group_rows}, backend=hip")


class FusedInt4Linear(_HipGPTQLinear):
    """Drop-in int4 GPTQ (groupsize 32) Linear on the HIP fused kernels.

    Constructor and attributes as the reference (fused_int4_linear.py:966-1014);
    ``v1`` (keyword) selects the zero convention of the checkpoint format,
    "gptq" (v1, the reference's only mode) or "gptq_v2".
    """

    def __init__(self, in_features: int, out_features: int, qweight: torch.Tensor,
                 scales: torch.Tensor, qzeros: torch.Tensor, bias: torch.Tensor | None = None,
                 groupsize: int = 32, *, v1: bool = True):
        super().__init__()
        assert groupsize == 32, "FusedInt4Linear supports groupsize=32 only"
        self._setup(in_features, out_features, qweight, scales, qzeros, bias, 32, None, v1, "fused")

    @classmethod
    def from_gptq_linear(cls, layer) -> "FusedInt4Linear":
        """Build from a GPTQ Linear (4-bit, groupsize 32), reusing its packed buffers."""
        assert layer.wbits == 4, f"FusedInt4Linear requires wbits=4, got {layer.wbits}"
        assert layer.groupsize == 32, f"FusedInt4Linear requires groupsize=32, got {layer.groupsize}"
        return cls(in_features=layer.in_features, out_features=layer.out_features,
                   qweight=layer.qweight, scales=layer.scales.to(torch.float16),
                   qzeros=layer.qzeros, bias=layer.bias if layer.bias is not None else None,
                   groupsize=32, v1=getattr(layer, "v1", True))


class FusedInt4LinearPaddedGroups(_HipGPTQLinear):
    """Odd groupsize (< 32) GPTQ int4 layer, re-laid into 32-row groups.

    Same constructor checks as the reference (fused_int4_linear.py:770-811).
    """

    def __init__(self, in_features: int, out_features: int, qweight: torch.Tensor,
                 scales: torch.Tensor, qzeros: torch.Tensor, bias: torch.Tensor | None = None,
                 groupsize: int = 32, *, v1: bool = True):
        super().__init__()
        if groupsize == 32:
            raise ValueError("FusedInt4LinearPaddedGroups is only for odd groupsizes")
        if groupsize <= 0 or groupsize > 32:
            raise ValueError(f"groupsize must be in 1..32, got {groupsize}")
        if in_features % groupsize != 0:
            raise ValueError(f"in_features={in_features} must be divisible by groupsize={groupsize}")
        self.num_groups = int(in_features) // int(groupsize)
        self._setup(in_features, out_features, qweight, scales, qzeros, bias, groupsize, None, v1,
                    "padded")
        self.padded_in_features = self.k_phys


class FusedInt4LinearAnyGroup(_HipGPTQLinear):
    """GPTQ int4 layer of any groupsize (reference: fused_int4_linear.py:639-758)."""

    def __init__(self, in_features: int, out_features: int, qweight: torch.Tensor,
                 scales: torch.Tensor, qzeros: torch.Tensor, bias: torch.Tensor | None = None,
                 groupsize: int = 32, *, v1: bool = True):
        super().__init__()
        self._setup(in_features, out_features, qweight, scales, qzeros, bias, groupsize, None, v1,
                    "any_group")


def fused_int4_gemm(a: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                    qzeros: torch.Tensor, bias: torch.Tensor | None = None,
                    groupsize: int = 32) -> torch.Tensor:
    """``c = a @ dequantize(qweight) + bias`` (reference: fused_int4_linear.py:388-537).

    Same contract: v1 zeros, groupsize 32, fp16/bf16/fp32 input (fp32 is
    computed in fp16 and returned as fp32), scales cast to the activation type.
    """
    assert groupsize == 32, "fused_int4_gemm currently supports groupsize=32 only"
    assert qweight.dtype == torch.int32
    assert qzeros.dtype == torch.int32
    assert a.dtype in (torch.float16, torch.bfloat16, torch.float32), f"unsupported a.dtype={a.dtype}"
    orig_dtype = a.dtype
    if a.dtype == torch.float32:
        a = a.to(torch.float16)
    if scales.dtype != a.dtype:
        scales = scales.to(a.dtype)
    leading_shape = a.shape[:-1]
    K = a.shape[-1]
    a_2d = a.reshape(-1, K)
    N = scales.shape[1]
    assert qweight.shape == (K // 8, N), (
        f"qweight shape mismatch: expected ({K//8}, {N}), got {tuple(qweight.shape)}")
    assert scales.shape == (K // groupsize, N), (
        f"scales shape mismatch: expected ({K//groupsize}, {N}), got {tuple(scales.shape)}")
    assert qzeros.shape == (K // groupsize, N // 8), (
        f"qzeros shape mismatch: expected ({K//groupsize}, {N//8}), got {tuple(qzeros.shape)}")
    assert N % 8 == 0, f"N must be a multiple of 8 (qzeros packing), got N={N}"
    assert K % 32 == 0, f"K must be a multiple of 32 (groupsize), got K={K}"
    if bias is not None:
        bias = bias.to(a.dtype)
    # The functional form has no load time: the tiled layout is written per
    # call (one extra pass over the packed weight).
    w = kernels.prepare(qweight.contiguous(), scales.contiguous(), qzeros.contiguous(), in_features=K,
                        out_features=N, kmap=None, k_phys=K, group_rows=32, v1=True)
    c = kernels.int4_gemm(a_2d, w, in_features=K, bias=bias)
    out = c.reshape(*leading_shape, N)
    if orig_dtype == torch.float32:
        out = out.to(torch.float32)
    return out


__all__ = [
    "FusedInt4Linear",
    "FusedInt4LinearAnyGroup",
    "FusedInt4LinearPaddedGroups",
    "fused_int4_gemm",
]
