"""Int4-packed Conv1d / ConvTranspose1d on the HIP library.

API of the reference's ``layers/packed_conv.py``: nibble pack / unpack
(:23-45), the RTN conv-weight quantizer (:63-90), the DAC-VAE style pad /
unpad (:93-120), ``PackedInt4Conv1d`` (:123-170), ``PackedInt4ConvTranspose1d``
(:173-222), ``quantize_conv_module`` and ``replace_conv_with_packed``
(:225-339). Weights keep the reference buffers (``qweight`` uint8 nibbles,
``scales`` / ``zeros`` [rows, groups], ``cols``); the dequant is the RTN one,
every op rounded in the compute dtype.

Where the reference dequantizes the whole weight per call and runs
``F.conv1d`` / ``F.conv_transpose1d``, fp16/bf16 activations with groups = 1
run as GEMMs over the packed rows (``oc_rtn_conv1d``: im2col chunks times the
RTN tiled kernel, fp32 partials, one rounding into [B, C, T];
``oc_rtn_conv_transpose1d``: the weight re-laid once with its codes transposed,
GEMM over input positions and a deterministic col2im). Other shapes dequantize
on the device (``oc_rtn_dequant``, bit-exact) and call the torch conv.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _hip, kernels
from .._hip import check, dtype_code, lib, ptr

_COUNTER = 512 * 1024  # the GEMM workspace's counter area, left untouched


def pack_int4_nibbles(w_int: torch.Tensor) -> torch.Tensor:
    """Codes [rows, cols] (0..15) -> uint8 [rows, ceil(cols / 2)]; column 2j in
    the low nibble of byte j, 2j + 1 in the high one."""
    rows, cols = w_int.shape
    c = w_int.to(torch.int32) & 0xF
    if cols % 2:
        c = torch.cat([c, torch.zeros(rows, 1, dtype=c.dtype, device=c.device)], dim=1)
    return (c[:, 0::2] | (c[:, 1::2] << 4)).to(torch.uint8).contiguous()


def unpack_int4_nibbles(packed: torch.Tensor, cols: int) -> torch.Tensor:
    """uint8 [rows, half] -> int16 codes [rows, cols]."""
    p = packed.to(torch.int16)
    return torch.stack([p & 0xF, (p >> 4) & 0xF], dim=-1).reshape(p.shape[0], -1)[:, :cols]


def quantize_conv_weight(weight: torch.Tensor, groupsize: int = -1):
    """RTN 4-bit quantization of a 2-D conv weight: per row, or per group of
    ``groupsize`` columns when it divides them; asymmetric min/max, scale =
    (max - min) / 15 (at least 1e-8), zero = round(-min / scale), codes
    clamp(round(w / scale) + zero, 0, 15); all-zero groups use [-1, 1].
    Returns (qweight uint8, scales fp16 [rows, G], zeros fp16 [rows, G], cols)."""
    if weight.dim() != 2:
        raise ValueError("flatten weight to 2-D before quantization")
    rows, cols = weight.shape
    G = cols // groupsize if groupsize > 0 and cols % groupsize == 0 else 1
    w = weight.float().reshape(rows, G, cols // G)
    hi, lo = w.amax(dim=-1, keepdim=True), w.amin(dim=-1, keepdim=True)
    flat = (hi == 0) & (lo == 0)
    hi = torch.where(flat, torch.ones_like(hi), hi)
    lo = torch.where(flat, -torch.ones_like(lo), lo)
    scale = ((hi - lo) / 15).clamp(min=1e-8)
    zero = torch.round(-lo / scale)
    q = torch.clamp(torch.round(w / scale) + zero, 0, 15).to(torch.int32).reshape(rows, cols)
    return (pack_int4_nibbles(q), scale.reshape(rows, G).to(torch.float16),
            zero.reshape(rows, G).to(torch.float16), cols)


def conv1d_pads(length: int, kernel_size: int, stride: int, dilation: int, pad_mode: str,
                causal: bool) -> tuple[int, int]:
    """(left, right) zero padding of a NormConv1d input (the reference's
    _conv1d_pad, packed_conv.py:93-108): enough for whole output frames."""
    if pad_mode == "none":
        return 0, 0
    span = (kernel_size - 1) * dilation + 1
    total = span - stride
    frames = (length - span + total) / stride + 1
    extra = (math.ceil(frames) - 1) * stride + (kernel_size - total) - length
    if causal:
        return total, extra
    right = extra // 2
    return total - right, right + extra


def _conv1d_pad(x: torch.Tensor, kernel_size: int, stride: int, dilation: int, pad_mode: str,
                causal: bool) -> torch.Tensor:
    left, right = conv1d_pads(x.shape[-1], kernel_size, stride, dilation, pad_mode, causal)
    return x if left == right == 0 else F.pad(x, (left, right))


def _convtranspose1d_unpad(x: torch.Tensor, kernel_size: int, stride: int, pad_mode: str,
                           causal: bool) -> torch.Tensor:
    """Crop of a NormConvTranspose1d output (packed_conv.py:111-120)."""
    if pad_mode == "none":
        return x
    total = kernel_size - stride
    if causal:
        return x[..., :x.shape[-1] - total]
    right = total // 2
    return x[..., total - right:x.shape[-1] - right]


class _PackedConvBase(nn.Module):
    def _init_common(self, in_channels, out_channels, kernel_size, stride, padding, dilation, groups, rows, ck,
                     qweight, scales, zeros, cols, bias, causal, pad_mode):
        self.in_channels, self.out_channels = int(in_channels), int(out_channels)
        self.kernel_size, self.stride, self.padding = int(kernel_size), int(stride), int(padding)
        self.dilation, self.groups = int(dilation), int(groups)
        self.causal, self.pad_mode = causal, pad_mode
        if qweight is None:  # an empty layer to load a state into
            qweight = torch.zeros(rows, (ck + 1) // 2, dtype=torch.uint8)
            scales = torch.zeros(rows, 1, dtype=torch.float16)
            zeros = torch.zeros(rows, 1, dtype=torch.float16)
            cols = ck
        self.register_buffer("qweight", qweight.contiguous())
        self.register_buffer("scales", scales.contiguous())
        self.register_buffer("zeros", zeros.contiguous())
        self.cols = int(cols)
        if bias is not None:
            self.register_parameter("bias", nn.Parameter(bias.detach(), requires_grad=False))
        else:
            self.bias = None

    def _dequant(self, dtype: torch.dtype) -> torch.Tensor:
        return kernels.rtn_dequant(self.qweight, self.scales, self.zeros, self.cols, self.qweight.shape[0], dtype)

    def _bias_as(self, dtype):
        return self.bias.to(dtype) if self.bias is not None else None

    @staticmethod
    def _workspace(device: torch.device, nbytes: int):
        idx = device.index if device.index is not None else torch.cuda.current_device()
        stream = _hip._raw_stream(idx)
        ws = _hip.workspace.get(idx, nbytes + _COUNTER, stream)
        return ws.data_ptr() + _COUNTER, nbytes, stream


class PackedInt4Conv1d(_PackedConvBase):
    """NormConv1d-compatible int4 packed Conv1d (pad included)."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: int, stride: int = 1, padding: int = 0,
                 dilation: int = 1, groups: int = 1, qweight: torch.Tensor | None = None,
                 scales: torch.Tensor | None = None, zeros: torch.Tensor | None = None, cols: int | None = None,
                 bias: torch.Tensor | None = None, causal: bool = False, pad_mode: str = "auto"):
        super().__init__()
        self._init_common(in_channels, out_channels, kernel_size, stride, padding, dilation, groups, out_channels,
                          (in_channels // groups) * kernel_size, qweight, scales, zeros, cols, bias, causal, pad_mode)
        self._tile_cache = None  # (key, qt, sz, fast flags): the large-M kernel's layout, built on first use

    def _materialize(self, dtype: torch.dtype) -> torch.Tensor:
        return self._dequant(dtype).reshape(self.out_channels, self.in_channels // self.groups, self.kernel_size)

    def _fused_ok(self, x: torch.Tensor) -> bool:
        K, G = self.cols, self.scales.shape[1]
        return (x.is_cuda and x.dtype in (torch.float16, torch.bfloat16) and self.groups == 1 and x.dim() == 3
                and K == self.in_channels * self.kernel_size and K % 32 == 0 and K % G == 0 and (K // G) % 8 == 0
                and self.qweight.shape[1] % 4 == 0 and self.qweight.is_cuda)

    def _tiles(self, x: torch.Tensor, rows: int):
        """(qt, sz, fast) of the large-M kernel's layout (oc_rtn_tile_prepare),
        built on the first call with enough output rows for it (1024) and
        cached until the weight tensors change; (None, None, 0) where the
        layout does not apply."""
        K, G = self.cols, self.scales.shape[1]
        gs = K // G
        if (rows < 1024 or self.scales.dtype != self.zeros.dtype
                or self.scales.dtype not in (torch.float16, torch.bfloat16) or gs % 32 != 0
                or (gs // 32) & (gs // 32 - 1) != 0 or self.out_channels % 8 != 0):
            return None, None, 0
        key = tuple((t.data_ptr(), t._version) for t in (self.qweight, self.scales, self.zeros))
        if self._tile_cache is None or self._tile_cache[0] != key:
            N, tiles, dev = self.out_channels, (self.out_channels + 15) // 16, self.qweight.device
            qt = torch.empty(tiles * (K // 32) * 64, dtype=torch.int32, device=dev)
            sz = torch.empty(tiles * G * 16, dtype=torch.int32, device=dev)
            fast = torch.empty(2, dtype=torch.int32, device=dev)
            check(lib().oc_rtn_tile_prepare(ptr(self.qweight), N, self.qweight.shape[1], K,
                                            ptr(self.scales.contiguous()), ptr(self.zeros.contiguous()),
                                            dtype_code(self.scales.dtype), G, ptr(qt), ptr(sz), ptr(fast),
                                            _hip.stream_of(dev)),
                  "oc_rtn_tile_prepare")
            self._tile_cache = (key, qt, sz, tuple(int(v) for v in fast.cpu()))
        _, qt, sz, fast = self._tile_cache
        return qt, sz, fast[0 if x.dtype == torch.bfloat16 else 1]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("PackedInt4Conv1d runs on the HIP device; there is no CPU fallback")
        bias = self._bias_as(x.dtype)
        if not self._fused_ok(x):
            x = _conv1d_pad(x, self.kernel_size, self.stride, self.dilation, self.pad_mode, self.causal)
            return F.conv1d(x, self._materialize(x.dtype), bias, self.stride, self.padding, self.dilation,
                            self.groups)
        x = x.contiguous()
        B, C, L = x.shape
        left, right = conv1d_pads(L, self.kernel_size, self.stride, self.dilation, self.pad_mode, self.causal)
        L_pad = L + left + right + 2 * self.padding
        T = (L_pad - self.dilation * (self.kernel_size - 1) - 1) // self.stride + 1
        y = torch.empty((B, self.out_channels, max(T, 0)), dtype=x.dtype, device=x.device)
        if T <= 0:
            return y
        qt, sz, fast = self._tiles(x, B * T)
        nbytes = int(lib().oc_rtn_conv1d_workspace_bytes(B, C, self.out_channels, self.kernel_size, T))
        ws, nbytes, stream = self._workspace(x.device, nbytes)
        check(lib().oc_rtn_conv1d_prepared(ptr(x), dtype_code(x.dtype), B, C, L, ptr(self.qweight),
                                           self.qweight.shape[1], ptr(self.scales), dtype_code(self.scales.dtype),
                                           ptr(self.zeros), dtype_code(self.zeros.dtype), self.scales.shape[1],
                                           ptr(qt), ptr(sz), fast, self.out_channels, self.kernel_size, self.stride,
                                           self.dilation, left + self.padding, T, ptr(bias),
                                           dtype_code(bias.dtype) if bias is not None else 0, ptr(y), ws, nbytes,
                                           stream),
              "oc_rtn_conv1d_prepared")
        return y

    def extra_repr(self) -> str:
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, stride={self.stride}, "
                f"dilation={self.dilation}, groups={self.groups}, packed=int4, backend=hip")


class PackedInt4ConvTranspose1d(_PackedConvBase):
    """NormConvTranspose1d-compatible int4 packed ConvTranspose1d (unpad included)."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: int, stride: int = 1, padding: int = 0,
                 output_padding: int = 0, dilation: int = 1, groups: int = 1, qweight: torch.Tensor | None = None,
                 scales: torch.Tensor | None = None, zeros: torch.Tensor | None = None, cols: int | None = None,
                 bias: torch.Tensor | None = None, causal: bool = False, pad_mode: str = "auto"):
        super().__init__()
        self.output_padding = int(output_padding)
        self._init_common(in_channels, out_channels, kernel_size, stride, padding, dilation, groups, in_channels,
                          (out_channels // groups) * kernel_size, qweight, scales, zeros, cols, bias, causal,
                          pad_mode)
        self._transposed = None  # (key, qweight_t, scales_t, zeros_t): the GEMM layout, built on first use
        self._tile_cache = {}  # activation dtype -> (key, qt, szt, fast): the large-M kernel's layout

    def _materialize(self, dtype: torch.dtype) -> torch.Tensor:
        return self._dequant(dtype).reshape(self.in_channels, self.out_channels // self.groups, self.kernel_size)

    def _fused_ok(self, x: torch.Tensor) -> bool:
        N, G = self.cols, self.scales.shape[1]
        return (x.is_cuda and x.dtype in (torch.float16, torch.bfloat16) and self.groups == 1 and x.dim() == 3
                and N == self.out_channels * self.kernel_size and self.in_channels % 32 == 0 and N % G == 0
                and self.scales.dtype == self.zeros.dtype and self.scales.dtype in (torch.float16, torch.bfloat16)
                and self.qweight.is_cuda)

    def _gemm_layout(self):
        key = tuple((t.data_ptr(), t._version) for t in (self.qweight, self.scales, self.zeros))
        if self._transposed is None or self._transposed[0] != key:
            rows, G = self.in_channels, self.scales.shape[1]
            dev = self.qweight.device
            qt = torch.empty((self.cols, rows // 2), dtype=torch.uint8, device=dev)
            st = torch.empty((G, rows), dtype=self.scales.dtype, device=dev)
            zt = torch.empty((G, rows), dtype=self.zeros.dtype, device=dev)
            check(lib().oc_rtn_transpose_prepare(ptr(self.qweight), rows, self.qweight.shape[1], self.cols,
                                                 ptr(self.scales.contiguous()), ptr(self.zeros.contiguous()), G,
                                                 ptr(qt), ptr(st), ptr(zt), _hip.stream_of(dev)),
                  "oc_rtn_transpose_prepare")
            self._transposed = (key, qt, st, zt)
        return self._transposed[1:]

    def _tiles(self, x: torch.Tensor, positions: int):
        """(qt, szt, fast) of the large-M kernel's layout for x's dtype
        (oc_rtn_tile_prepare_t), built on the first call with 1024 or more
        input positions and cached until the weight tensors change; (None,
        None, 0) where the layout does not apply."""
        N, G = self.cols, self.scales.shape[1]
        if positions < 1024 or (N // G) % 16 != 0 or N % 8 != 0:
            return None, None, 0
        key = tuple((t.data_ptr(), t._version) for t in (self.qweight, self.scales, self.zeros))
        hit = self._tile_cache.get(x.dtype)
        if hit is None or hit[0] != key:
            K, tiles, dev = self.in_channels, (N + 15) // 16, self.qweight.device
            qt = torch.empty(tiles * (K // 32) * 64, dtype=torch.int32, device=dev)
            szt = torch.empty(tiles * K, dtype=torch.int32, device=dev)
            fast = torch.empty(1, dtype=torch.int32, device=dev)
            check(lib().oc_rtn_tile_prepare_t(ptr(self.qweight), K, self.qweight.shape[1], N,
                                              ptr(self.scales.contiguous()), ptr(self.zeros.contiguous()),
                                              dtype_code(self.scales.dtype), G, dtype_code(x.dtype), ptr(qt),
                                              ptr(szt), ptr(fast), _hip.stream_of(dev)),
                  "oc_rtn_tile_prepare_t")
            hit = (key, qt, szt, int(fast.cpu()[0]))
            self._tile_cache[x.dtype] = hit
        return hit[1], hit[2], hit[3]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("PackedInt4ConvTranspose1d runs on the HIP device; there is no CPU fallback")
        bias = self._bias_as(x.dtype)
        if not self._fused_ok(x):
            y = F.conv_transpose1d(x, self._materialize(x.dtype), bias, self.stride, self.padding,
                                   self.output_padding, self.groups, self.dilation)
            return _convtranspose1d_unpad(y, self.kernel_size, self.stride, self.pad_mode, self.causal)
        x = x.contiguous()
        B, C, L = x.shape
        L_out = ((L - 1) * self.stride - 2 * self.padding + self.dilation * (self.kernel_size - 1)
                 + self.output_padding + 1)
        y = torch.empty((B, self.out_channels, max(L_out, 0)), dtype=x.dtype, device=x.device)
        if L_out > 0 and L > 0:
            qt, st, zt = self._gemm_layout()
            wt, szt, fast = self._tiles(x, L)
            nbytes = int(lib().oc_rtn_conv_transpose1d_workspace_bytes(B, C, L, self.out_channels,
                                                                       self.kernel_size, L_out))
            ws, nbytes, stream = self._workspace(x.device, nbytes)
            check(lib().oc_rtn_conv_transpose1d_prepared(ptr(x), dtype_code(x.dtype), B, C, L, ptr(qt), ptr(st),
                                                         ptr(zt), dtype_code(st.dtype), st.shape[0], ptr(wt),
                                                         ptr(szt), fast, self.out_channels, self.kernel_size,
                                                         self.stride, self.dilation, self.padding, L_out, ptr(bias),
                                                         dtype_code(bias.dtype) if bias is not None else 0, ptr(y),
                                                         ws, nbytes, stream),
                  "oc_rtn_conv_transpose1d_prepared")
        return _convtranspose1d_unpad(y, self.kernel_size, self.stride, self.pad_mode, self.causal)

    def extra_repr(self) -> str:
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, stride={self.stride}, "
                f"dilation={self.dilation}, groups={self.groups}, packed=int4, backend=hip")


def _first(v):
    return v[0] if isinstance(v, tuple) else v


def quantize_conv_module(mod: nn.Module, groupsize: int = 32):
    """A Conv1d / ConvTranspose1d (weight norm removed) -> its packed layer."""
    weight = mod.weight.detach()
    bias = mod.bias.detach() if mod.bias is not None else None
    qweight, scales, zeros, cols = quantize_conv_weight(weight.reshape(weight.shape[0], -1), groupsize=groupsize)
    common = dict(kernel_size=_first(mod.kernel_size), stride=_first(mod.stride), padding=_first(mod.padding),
                  dilation=_first(mod.dilation), groups=mod.groups, qweight=qweight, scales=scales, zeros=zeros,
                  cols=cols, bias=bias, causal=getattr(mod, "causal", False),
                  pad_mode=getattr(mod, "pad_mode", "none"))
    if isinstance(mod, nn.ConvTranspose1d):
        return PackedInt4ConvTranspose1d(mod.in_channels, mod.out_channels,
                                         output_padding=_first(mod.output_padding), **common)
    return PackedInt4Conv1d(mod.in_channels, mod.out_channels, **common)


def replace_conv_with_packed(model: nn.Module, *, groupsize: int = 32,
                             cast_remaining_to: torch.dtype | None = torch.float16) -> dict:
    """Swap every (Norm)Conv1d / (Norm)ConvTranspose1d for its packed layer;
    cast the remaining floating tensors to ``cast_remaining_to``. Returns
    {"replaced", "bytes_before", "bytes_after", "ratio"}."""
    kinds = ("NormConv1d", "NormConvTranspose1d", "Conv1d", "ConvTranspose1d")
    targets = [(n, m) for n, m in model.named_modules() if type(m).__name__ in kinds and hasattr(m, "kernel_size")]
    before = after = 0
    for name, mod in targets:
        try:
            nn.utils.remove_weight_norm(mod)
        except (ValueError, AttributeError):
            pass
        before += sum(p.numel() * p.element_size() for p in mod.parameters(recurse=False))
        packed = quantize_conv_module(mod, groupsize=groupsize)
        after += sum(t.numel() * t.element_size() for t in list(packed.buffers(recurse=False))
                     + list(packed.parameters(recurse=False)))
        parent_name, _, child = name.rpartition(".")
        setattr(model.get_submodule(parent_name) if parent_name else model, child, packed)
    if cast_remaining_to is not None:
        for mod in model.modules():
            if isinstance(mod, _PackedConvBase):
                continue
            for key, p in list(mod._parameters.items()):
                if p is not None and p.dtype.is_floating_point and p.dtype != cast_remaining_to:
                    mod._parameters[key] = nn.Parameter(p.data.to(cast_remaining_to), requires_grad=p.requires_grad)
            for key, b in list(mod._buffers.items()):
                if b is not None and b.dtype.is_floating_point and b.dtype != cast_remaining_to:
                    mod._buffers[key] = b.to(cast_remaining_to)
        for mod in model.modules():
            if isinstance(mod, nn.LSTM):
                mod.flatten_parameters()
    return {"replaced": len(targets), "bytes_before": before, "bytes_after": after,
            "ratio": after / before if before else 0.0}


__all__ = ["PackedInt4Conv1d", "PackedInt4ConvTranspose1d", "pack_int4_nibbles", "unpack_int4_nibbles",
           "quantize_conv_weight", "quantize_conv_module", "replace_conv_with_packed"]
