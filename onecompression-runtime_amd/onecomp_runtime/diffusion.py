"""Packed-checkpoint loader: ``load_int4_model``.

Contract of the reference's ``load_int4_model`` (diffusion.py:57-239, on-disk
format README.md:106-113): one ``safetensors`` file whose metadata holds
``config_json`` (the model config; keys starting with ``_`` are dropped),
``quant_layers_json`` (one entry per quantized Linear: ``name``, ``wbits``,
``groupsize``, ``actorder``, ``in_features``, ``out_features``) and
``checkpoint_format`` ("gptq" = v1 zeros, the default; "gptq_v2"); tensors
``{name}.qweight/.scales/.qzeros[.g_idx][.bias]`` per quantized layer plus the
model's other parameters and buffers under their state-dict names.

How this loader works:
  1. The manifest is read and checked (``ValueError`` without it).
  2. The model is built on the meta device and ``prepare_meta_model`` runs.
  3. Each selected quantized layer is built by ``backend.build_quant_layer``
     from its tensors, read one layer at a time straight onto the target
     device; the HIP layers write their tiled layout there at once, so the
     checkpoint tensors of one layer at most are alive beside the model.
     ``KeyError`` if a layer's parent module does not exist.
  4. The remaining parameters and persistent buffers are pulled by name:
     every meta tensor of the model that the file holds is read and assigned
     on the device (floating point ones cast to ``dtype``). Names the model
     needs but the file lacks, and file tensors the model does not have,
     raise ``RuntimeError``; tensors of quantized layers (including the
     ``.weight`` a swapped Linear had) are not counted as either.
  5. ``post_load`` runs; any parameter still on the meta device is a
     ``RuntimeError``.
  6. Warmup runs one forward per M in ``warmup_m_values`` for each distinct
     GEMM signature (output features, physical K, group rows, row map), which
     sizes the per-stream GEMM workspaces before timed or captured work.

A summary line (layer kinds, tensor count, seconds) is printed with ``label``,
and the counts are kept on the model as ``onecomp_load_report``.
"""
from __future__ import annotations

import json
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Callable, Iterable

import torch
from safetensors import safe_open

from .backend import KNOWN_BACKENDS, build_quant_layer, resolve_backend, resolve_dtype
from .layers.fused_int4_linear import _HipGPTQLinear

QUANT_SUFFIXES = ("qweight", "scales", "qzeros", "g_idx", "bias")


@dataclass
class LoadReport:
    """What a load did: layers per kind, tensors materialised, timings."""

    kinds: dict[str, int] = field(default_factory=lambda: {k: 0 for k in KNOWN_BACKENDS})
    quant_layers: list[str] = field(default_factory=list)
    tensors: int = 0
    load_s: float = 0.0
    warmup_s: float = 0.0
    warmup_signatures: int = 0

    def summary(self, device: torch.device) -> str:
        used = ", ".join(f"{k}={v}" for k, v in self.kinds.items() if v)
        return (f"{len(self.quant_layers)} quantized layers ({used or 'none'}), "
                f"{self.tensors} other tensors on {device}, {self.load_s:.2f} s")


@dataclass
class _Manifest:
    config: dict[str, Any]
    layers: list[dict[str, Any]]
    checkpoint_format: str
    keys: frozenset[str]

    @classmethod
    def read(cls, reader, path: Path) -> "_Manifest":
        md = reader.metadata() or {}
        if "config_json" not in md or "quant_layers_json" not in md:
            raise ValueError(
                f"{path} is missing 'config_json' / 'quant_layers_json' metadata; "
                "not a packed OneCompression checkpoint")
        config = {k: v for k, v in json.loads(md["config_json"]).items() if not k.startswith("_")}
        fmt = md.get("checkpoint_format", "gptq")
        layers = []
        for entry in json.loads(md["quant_layers_json"]):
            entry = dict(entry)
            entry["checkpoint_format"] = fmt  # per-layer builders read the zero convention here
            layers.append(entry)
        return cls(config, layers, fmt, frozenset(reader.keys()))

    def owned_names(self) -> set[str]:
        """State-dict names belonging to quantized layers: their packed
        tensors and the dense ``.weight`` the meta Linear declared."""
        owned = set()
        for entry in self.layers:
            name = entry["name"]
            owned.add(f"{name}.weight")
            owned.update(f"{name}.{s}" for s in QUANT_SUFFIXES)
        return owned


def _swap_quant_layers(model: torch.nn.Module, manifest: _Manifest, reader, backend: str,
                       dtype: torch.dtype, device: torch.device,
                       layer_filter: Callable[[str], bool] | None, report: LoadReport) -> None:
    for entry in manifest.layers:
        name = entry["name"]
        if layer_filter is not None and not layer_filter(name):
            continue
        parent_name, _, child = name.rpartition(".")
        try:
            parent = model.get_submodule(parent_name) if parent_name else model
        except AttributeError:
            raise KeyError(f"quant layer parent not found: {parent_name!r}") from None
        tensors = {s: reader.get_tensor(f"{name}.{s}") for s in QUANT_SUFFIXES
                   if f"{name}.{s}" in manifest.keys}
        layer, kind = build_quant_layer(entry, tensors, backend, dtype, device)
        setattr(parent, child, layer)
        report.kinds[kind] = report.kinds.get(kind, 0) + 1
        report.quant_layers.append(name)


def _meta_slots(model: torch.nn.Module, skip: set[str]) -> Iterable[tuple[str, Any, str, bool]]:
    """(state-dict name, owning module, attribute, is_parameter) of every
    parameter and persistent buffer outside the modules named in ``skip``
    (the swapped quantized layers) and their children."""
    below = tuple(f"{n}." for n in skip)
    for mod_name, mod in model.named_modules(remove_duplicate=False):
        if mod_name in skip or (below and mod_name.startswith(below)):
            continue
        prefix = f"{mod_name}." if mod_name else ""
        for attr, p in mod._parameters.items():
            if p is not None:
                yield prefix + attr, mod, attr, True
        for attr, b in mod._buffers.items():
            if b is not None and attr not in mod._non_persistent_buffers_set:
                yield prefix + attr, mod, attr, False


def _materialise(model: torch.nn.Module, manifest: _Manifest, reader, dtype: torch.dtype,
                 device: torch.device, tensor_filter: Callable[[str], bool] | None,
                 report: LoadReport) -> None:
    owned = manifest.owned_names()
    available = {k for k in manifest.keys
                 if k not in owned and (tensor_filter is None or tensor_filter(k))}
    missing, seen = [], set()
    for key, mod, attr, is_param in _meta_slots(model, set(report.quant_layers)):
        seen.add(key)
        if key not in available:
            if key not in owned:
                missing.append(key)
            continue
        t = reader.get_tensor(key)
        t = t.to(device=device, dtype=dtype if t.is_floating_point() else t.dtype)
        if is_param:
            old = mod._parameters[attr]
            mod._parameters[attr] = torch.nn.Parameter(t, requires_grad=old.requires_grad)
        else:
            mod._buffers[attr] = t
        report.tensors += 1
    if missing:
        raise RuntimeError(f"missing keys: {missing[:8]} ...")
    unexpected = sorted(available - seen)
    if unexpected:
        raise RuntimeError(f"unexpected keys: {unexpected[:8]} ...")


def _warm(model: torch.nn.Module, m_values: tuple[int, ...], device: torch.device, report: LoadReport) -> None:
    t0 = time.perf_counter()
    reps: dict[tuple, _HipGPTQLinear] = {}
    for m in model.modules():
        if isinstance(m, _HipGPTQLinear):
            sig = (m.out_features, m.in_features, m.k_phys, m.group_rows, m.kmap is not None)
            reps.setdefault(sig, m)
    for layer in reps.values():
        layer.warmup(m_values=m_values)
    if reps:
        torch.cuda.synchronize(device)
    report.warmup_s = time.perf_counter() - t0
    report.warmup_signatures = len(reps)


def load_int4_model(
    checkpoint_path: str,
    build_meta_model: Callable[[dict], torch.nn.Module],
    *,
    device: str = "cuda:0",
    dtype: str | torch.dtype = "bfloat16",
    backend: str | None = "auto",
    use_fused: bool = True,
    post_load: Callable[[torch.nn.Module], None] | None = None,
    prepare_meta_model: Callable[[torch.nn.Module], None] | None = None,
    quant_layer_filter: Callable[[str], bool] | None = None,
    tensor_filter: Callable[[str], bool] | None = None,
    warmup: bool = True,
    warmup_m_values: tuple[int, ...] = (64, 128, 256, 1024, 4096),
    label: str = "onecomp_runtime",
) -> torch.nn.Module:
    """Build ``build_meta_model(config)`` from a packed int4 checkpoint on
    ``device`` (arguments as the reference's, diffusion.py:57-72; ``backend``
    "auto" resolves to "hip")."""
    t0 = time.perf_counter()
    backend = resolve_backend(backend, use_fused)
    compute_dtype = resolve_dtype(dtype)
    dev = torch.device(device)
    path = Path(checkpoint_path)
    report = LoadReport()
    with safe_open(str(path), framework="pt", device="cpu") as reader:
        manifest = _Manifest.read(reader, path)
        with torch.device("meta"):
            model = build_meta_model(manifest.config)
        if prepare_meta_model is not None:
            prepare_meta_model(model)
        _swap_quant_layers(model, manifest, reader, backend, compute_dtype, dev, quant_layer_filter, report)
        _materialise(model, manifest, reader, compute_dtype, dev, tensor_filter, report)
    if post_load is not None:
        post_load(model)
    on_meta = [n for n, p in model.named_parameters() if p.is_meta]
    if on_meta:
        raise RuntimeError(f"parameter left on meta device: {on_meta[:8]} ...")
    model.eval()
    report.load_s = time.perf_counter() - t0
    print(f"[{label}] {report.summary(dev)}")
    if warmup and dev.type == "cuda":
        _warm(model, tuple(warmup_m_values), dev, report)
        if report.warmup_signatures:
            print(f"[{label}] warmup {1000 * report.warmup_s:.0f} ms over "
                  f"{report.warmup_signatures} GEMM signatures")
    model.onecomp_load_report = report
    return model
