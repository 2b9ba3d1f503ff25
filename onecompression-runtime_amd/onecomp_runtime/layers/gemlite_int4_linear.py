"""GemLite names kept for import compatibility.

GemLite is a Triton library tuned for NVIDIA GPUs (reference:
layers/gemlite_int4_linear.py:20-98); this package dispatches no Triton code,
so it is never available and the GemLite backends raise as the reference does
when the package is missing (backend.py:116-131).
"""
from __future__ import annotations

import torch


def gemlite_available() -> bool:
    return False


class GemLiteInt4Linear(torch.nn.Module):
    def __init__(self, *args, **kwargs):
        raise ImportError("GemLite is not available in the MI355X build; use backend='hip'")
