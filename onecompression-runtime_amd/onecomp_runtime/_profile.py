"""Opt-in call-shape histogram (``ONECOMP_PROFILE_SHAPES=1``), printed at exit.

Same switch and output format as the reference's shape profiler
(layers/fused_int4_linear.py:37, :58-73).
"""
from __future__ import annotations

import atexit
import os

PROFILE_SHAPES = os.environ.get("ONECOMP_PROFILE_SHAPES") == "1"
SHAPE_STATS: dict[tuple[str, int, int, int], int] = {}


def record(kind: str, m: int, k: int, n: int) -> None:
    key = (kind, int(m), int(k), int(n))
    SHAPE_STATS[key] = SHAPE_STATS.get(key, 0) + 1


def _print_shape_stats() -> None:
    if not PROFILE_SHAPES or not SHAPE_STATS:
        return
    print("[onecomp-profile] fused shape calls:", flush=True)
    for (kind, m, k, n), count in sorted(SHAPE_STATS.items(), key=lambda kv: kv[1], reverse=True)[:40]:
        print(f"[onecomp-profile] {kind:14s} M={m:<5d} K={k:<5d} N={n:<5d} calls={count}", flush=True)


atexit.register(_print_shape_stats)
