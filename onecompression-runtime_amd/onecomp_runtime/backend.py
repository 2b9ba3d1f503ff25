"""Backend selection and per-layer int4 module construction.

API of the reference's ``backend.py`` (:51-321). The MI355X build adds the
``hip`` backend, which is what ``auto`` resolves to: every quantized layer is
served by the HIP library, whatever its groupsize, act-order or zero format:

    - groupsize 32, no act-order          -> FusedInt4Linear
    - odd groupsize < 32, no act-order    -> FusedInt4LinearPaddedGroups
    - anything else (act-order, gs 64/128, 8-bit) -> PackedGPTQLinear
      (act-order rows sorted at load time, fused GEMM per call)

``fused`` and ``packed`` keep their reference meaning (same layer classes,
HIP kernels underneath); ``eager`` dequantizes once, on the device, into a
plain ``nn.Linear``. The GemLite family is never available here and raises
exactly as the reference does without GemLite. Unlike the reference's
``build_fused`` (:206-215), every builder honours ``checkpoint_format``
("gptq" = v1 zeros, "gptq_v2" = stored zeros).
"""
from __future__ import annotations

from typing import Any

import torch

from .layers.fused_int4_linear import (
    FusedInt4Linear,
    FusedInt4LinearAnyGroup,
    FusedInt4LinearPaddedGroups,
)
from .layers.gemlite_int4_linear import gemlite_available
from .layers.packed_gptq_linear import PackedGPTQLinear
from .quant_utils import dequant_gptq_to_fp

_DTYPES = {
    "float16": torch.float16,
    "fp16": torch.float16,
    "bfloat16": torch.bfloat16,
    "bf16": torch.bfloat16,
    "float32": torch.float32,
    "fp32": torch.float32,
}

_GEMLITE_BACKENDS = ("gemlite", "a8w4", "a8w4_ffn_up", "mxfp4_ffn", "mxfp4_ffn_up", "nvfp4_ffn")
KNOWN_BACKENDS = _GEMLITE_BACKENDS + ("hip", "fused", "packed", "eager")


def resolve_dtype(dtype: str | torch.dtype) -> torch.dtype:
    if isinstance(dtype, torch.dtype):
        return dtype
    try:
        return _DTYPES[str(dtype).lower()]
    except KeyError:
        raise ValueError(f"unsupported dtype: {dtype!r}")


def is_v1(entry: dict[str, Any]) -> bool:
    """Zero-point convention of the checkpoint ("gptq_v2" stores zeros as is)."""
    return entry.get("checkpoint_format", "gptq") != "gptq_v2"


def can_use_fused(entry: dict[str, Any]) -> bool:
    """True if a layer meets the groupsize-32 fused kernel constraints (backend.py:60-68)."""
    return (
        not bool(entry.get("actorder", False))
        and int(entry["wbits"]) == 4
        and int(entry["groupsize"]) == 32
        and int(entry["in_features"]) % 32 == 0
        and int(entry["out_features"]) % 8 == 0
    )


def can_use_fused_any_group(entry: dict[str, Any]) -> bool:
    """True if the generic fused path can run this GPTQ int4 layer (backend.py:71-78)."""
    return (
        not bool(entry.get("actorder", False))
        and int(entry["wbits"]) == 4
        and int(entry["in_features"]) % 8 == 0
        and int(entry["out_features"]) % 8 == 0
    )


def can_use_fused_padded_groups(entry: dict[str, Any]) -> bool:
    """True if odd groups can be re-laid out into 32-row groups (backend.py:81-92)."""
    gs = int(entry["groupsize"])
    in_features = int(entry["in_features"])
    return (
        not bool(entry.get("actorder", False))
        and int(entry["wbits"]) == 4
        and gs != 32
        and 0 < gs < 32
        and in_features % gs == 0
        and int(entry["out_features"]) % 8 == 0
    )


def resolve_backend(backend: str | None, use_fused: bool = True) -> str:
    """Pick the int4 GEMM backend (reference: backend.py:103-144).

    ``use_fused=False`` forces eager. ``"auto"`` resolves to ``"hip"``.
    """
    if not use_fused:
        return "eager"
    b = (backend or "auto").lower()
    if b == "auto":
        return "hip"
    if b in _GEMLITE_BACKENDS and not gemlite_available():
        raise RuntimeError(
            f"backend={b!r} requested but the 'gemlite' package is not "
            "importable; use backend='hip' (or 'fused')"
        )
    if b not in KNOWN_BACKENDS:
        raise ValueError(f"unknown backend: {backend!r}")
    return b


def _bias(st: dict, device: torch.device):
    return st["bias"].to(device) if "bias" in st else None


def build_fused(entry: dict, st: dict, device: torch.device) -> FusedInt4Linear:
    return FusedInt4Linear(
        in_features=int(entry["in_features"]),
        out_features=int(entry["out_features"]),
        qweight=st["qweight"].to(device),
        scales=st["scales"].to(device=device, dtype=torch.float16),
        qzeros=st["qzeros"].to(device),
        bias=_bias(st, device),
        groupsize=32,
        v1=is_v1(entry),
    )


def build_fused_any_group(entry: dict, st: dict, device: torch.device) -> FusedInt4LinearAnyGroup:
    return FusedInt4LinearAnyGroup(
        in_features=int(entry["in_features"]),
        out_features=int(entry["out_features"]),
        qweight=st["qweight"].to(device),
        scales=st["scales"].to(device=device, dtype=torch.float16),
        qzeros=st["qzeros"].to(device),
        bias=_bias(st, device),
        groupsize=int(entry["groupsize"]),
        v1=is_v1(entry),
    )


def build_fused_padded_groups(entry: dict, st: dict, device: torch.device) -> FusedInt4LinearPaddedGroups:
    return FusedInt4LinearPaddedGroups(
        in_features=int(entry["in_features"]),
        out_features=int(entry["out_features"]),
        qweight=st["qweight"].to(device),
        scales=st["scales"].to(device=device, dtype=torch.float16),
        qzeros=st["qzeros"].to(device),
        bias=_bias(st, device),
        groupsize=int(entry["groupsize"]),
        v1=is_v1(entry),
    )


def build_eager(entry: dict, st: dict, dtype: torch.dtype, device: torch.device) -> torch.nn.Linear:
    """Dequantize once (on the device) into a plain nn.Linear (backend.py:246-264)."""
    in_f, out_f = int(entry["in_features"]), int(entry["out_features"])
    g_idx = st.get("g_idx")
    if g_idx is None:
        gs = int(entry["groupsize"])
        g_idx = (torch.arange(in_f) // gs).to(torch.long)
    weight = dequant_gptq_to_fp(
        qweight=st["qweight"].to(device), scales=st["scales"].to(device),
        qzeros=st["qzeros"].to(device), g_idx=g_idx.to(device), in_features=in_f,
        out_features=out_f, dtype=dtype, v1=is_v1(entry), wbits=int(entry.get("wbits", 4)),
    )
    has_bias = "bias" in st
    lin = torch.nn.Linear(in_f, out_f, bias=has_bias, device=device, dtype=dtype)
    with torch.no_grad():
        lin.weight.copy_(weight)
        if has_bias:
            lin.bias.copy_(st["bias"].to(dtype=dtype, device=device))
    return lin


def build_packed(entry: dict, st: dict, dtype: torch.dtype, device: torch.device) -> PackedGPTQLinear:
    in_f, out_f = int(entry["in_features"]), int(entry["out_features"])
    g_idx = st.get("g_idx")
    return PackedGPTQLinear(
        in_features=in_f,
        out_features=out_f,
        qweight=st["qweight"].to(device),
        scales=st["scales"].to(device=device, dtype=dtype),
        qzeros=st["qzeros"].to(device),
        g_idx=g_idx.to(device) if g_idx is not None else None,
        bias=_bias(st, device),
        groupsize=int(entry["groupsize"]),
        wbits=int(entry["wbits"]),
        v1=is_v1(entry),
    )


def build_hip(entry: dict, st: dict, dtype: torch.dtype, device: torch.device) -> torch.nn.Module:
    """The ``hip`` backend: every layout on the HIP kernels (see module docstring).

    Scales keep their checkpoint precision (fp16; fp32 is narrowed to fp16),
    so every layer dequantizes exactly like the eager path.
    """
    if can_use_fused(entry):
        return build_fused(entry, st, device)
    if can_use_fused_padded_groups(entry):
        return build_fused_padded_groups(entry, st, device)
    scales = st["scales"]
    if scales.dtype not in (torch.float16, torch.bfloat16):
        scales = scales.to(torch.float16)
    return build_packed(entry, st, scales.dtype, device)


def build_quant_layer(entry: dict, st: dict, backend: str, dtype: torch.dtype, device: torch.device):
    """Dispatch a single quant-layer build, returning ``(module, kind)``
    (reference: backend.py:285-321). ``kind`` is ``"hip"``, ``"fused"``,
    ``"packed"`` or ``"eager"``.
    """
    if backend in _GEMLITE_BACKENDS:
        resolve_backend(backend)  # raises: GemLite is never importable here
    if backend == "hip":
        return build_hip(entry, st, dtype, device), "hip"
    if backend == "fused" and can_use_fused(entry):
        return build_fused(entry, st, device), "fused"
    if backend == "fused" and can_use_fused_padded_groups(entry):
        return build_fused_padded_groups(entry, st, device), "fused"
    if backend == "fused" and can_use_fused_any_group(entry):
        return build_fused_any_group(entry, st, device), "fused"
    if backend in ("fused", "packed"):
        return build_packed(entry, st, dtype, device), "packed"
    return build_eager(entry, st, dtype, device), "eager"
