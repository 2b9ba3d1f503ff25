"""Shared helpers of the GPU parity tests (no GPU work at import)."""
from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import onecomp_oracle as O

DTYPE_NAME = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def say(msg: str) -> None:
    """Name the case before a GPU step (flushed, so a crash still shows it)."""
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float32).numpy()


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def oracle_bits(vals: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    if dtype == torch.bfloat16:
        return O.f32_to_bf16_bits(vals)
    return np.asarray(vals, np.float32).astype(np.float16).view(np.uint16)


def assert_gemm_close(out: torch.Tensor, ref: np.ndarray, what: str = "") -> None:
    ok, rel, cos = O.gemm_close(np32(out), ref)
    assert ok, f"{what}: max|err|/max|ref| = {rel:.3e}, cosine = {cos:.6f}"


def layer_oracle_inputs(layer):
    """numpy views of a synthetic GPTQLayer for the oracle."""
    g_idx = layer.g_idx.numpy() if layer.g_idx is not None else O.default_g_idx(layer.K, layer.groupsize)
    return layer.qweight.numpy(), layer.scales.float().numpy(), layer.qzeros.numpy(), g_idx
