"""Seeded synthetic GPTQ / RTN layers and activations for the benchmark
workloads (host-side data generation, not a compute path).

Draw order per GPTQ layer, from one ``torch.Generator`` seeded per case:
codes ``W[K, N]`` uniform 0..15, zeros ``Z[G, N]`` uniform 0..15, scales
``|N(0,1)| * 0.01 + 1e-3`` rounded to fp16, then (act-order only) ``g_idx =
randperm(K) // groupsize``. qweight packs W along K (8 codes per int32, code
i of a word at bits 4i); qzeros packs ``(Z - 1) & 0xF`` for v1 ("gptq") and
``Z`` for v2 ("gptq_v2") along N.

Workloads (K, N, M) follow the benchmark configurations:
    gptq_gs32_m16   M=16,   K=N=4096, groupsize 32, v1
    decode_actorder M=1/8,  (K,N) in (5120,5120) (5120,17408) (17408,5120) (5120,1024), act-order, v1
    dit_large_m     M=4096, (K,N) in (3072,3072) (3072,12288) (12288,3072), v2, activation outliers
    padded_gs26     M=256,  K=1040, N=3072, groupsize 26, v1
    rtn_moe         RTN linear M=512 K=1024 N=2048; RTN embedding 32768x1024, 4096 ids;
                    64-expert int4 gs32 K=4096 N=2048, 512 tokens top-8
    next rows       GPTQ gs128 4-bit and 8-bit K=N=5120 at M=1/16; DSV4 int4/int2 gs128
                    K=7168 N=2048 (device-resident at M=1; host-resident routed experts);
                    packed Conv1d 512->512 k=7 and ConvTranspose1d 1024->512 k=16 stride 8

8-bit GPTQ layers (``gptq8_layer``) draw codes 0..255, zeros 0..255 and scales
``|N(0,1)| * 0.001 + 1e-4``; qweight packs 4 codes per int32 along K (code i at
bits 8i), qzeros ``(Z - 1) & 0xFF`` (v1) 4 per int32 along N. DSV4 layers
(``dsv4_layer``) draw codes ``[N, K]`` in 0..2^wbits-1 packed along K into
uint8 (``8 // wbits`` per byte, code i at bits ``wbits * i``), integer zeros
and scales ``[G, N]`` in fp16.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

SEED_BASE = 20260


def pack_rows(codes_kn: torch.Tensor, rows_to: int | None = None) -> torch.Tensor:
    """int codes [K, N] (0..15) -> int32 [ceil(K/8) (or rows_to/8), N], packed along K."""
    K, N = codes_kn.shape
    Kp = rows_to if rows_to is not None else (K + 7) // 8 * 8
    full = torch.zeros((Kp, N), dtype=torch.int64)
    full[:K] = codes_kn.to(torch.int64) & 0xF
    full = full.reshape(Kp // 8, 8, N)
    word = torch.zeros((Kp // 8, N), dtype=torch.int64)
    for i in range(8):
        word |= full[:, i, :] << (4 * i)
    word = torch.where(word >= 2**31, word - 2**32, word)
    return word.to(torch.int32)


def pack_cols(codes_gn: torch.Tensor) -> torch.Tensor:
    """int codes [G, N] (0..15) -> int32 [G, N/8], packed along N."""
    G, N = codes_gn.shape
    c = (codes_gn.to(torch.int64) & 0xF).reshape(G, N // 8, 8)
    word = torch.zeros((G, N // 8), dtype=torch.int64)
    for i in range(8):
        word |= c[:, :, i] << (4 * i)
    word = torch.where(word >= 2**31, word - 2**32, word)
    return word.to(torch.int32)


@dataclass
class GPTQLayer:
    K: int
    N: int
    groupsize: int
    v1: bool
    qweight: torch.Tensor  # int32 [ceil(K/8) or padded, N]
    scales: torch.Tensor  # fp16 [G, N]
    qzeros: torch.Tensor  # int32 [G, N/8]
    g_idx: torch.Tensor | None  # int64 [K] (act-order) or None
    codes: torch.Tensor  # int32 [K, N] (for the oracle)
    zeros: torch.Tensor  # int32 [G, N] actual zero points


def gptq_layer(K: int, N: int, *, seed: int, groupsize: int = 32, v1: bool = True,
               act_order: bool = False, pad_rows_to: int | None = None,
               scale_dtype: torch.dtype = torch.float16) -> GPTQLayer:
    g = torch.Generator().manual_seed(seed)
    G = (K + groupsize - 1) // groupsize
    codes = torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32)
    zeros = torch.randint(0, 16, (G, N), generator=g, dtype=torch.int32)
    scales = (torch.randn(G, N, generator=g).abs() * 0.01 + 1e-3).to(scale_dtype)
    g_idx = None
    if act_order:
        g_idx = (torch.randperm(K, generator=g) // groupsize).to(torch.int64)
    stored = ((zeros - 1) & 0xF) if v1 else zeros
    return GPTQLayer(K, N, groupsize, v1, pack_rows(codes, pad_rows_to), scales, pack_cols(stored),
                     g_idx, codes, zeros)


def activations(M: int, K: int, *, seed: int, dtype: torch.dtype = torch.bfloat16,
                outliers: bool = False) -> torch.Tensor:
    """X ~ N(0,1); with ``outliers``: X * 0.5 and 1% of the channels x20."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if outliers:
        x = x * 0.5
        cols = torch.randperm(K, generator=g)[: max(1, K // 100)]
        x[:, cols] *= 20.0
    return x.to(dtype)


@dataclass
class RTNLayer:
    rows: int
    K: int
    qweight_u8: torch.Tensor  # uint8 [rows, ceil(K/2)]
    scales: torch.Tensor  # fp16 [rows, G]
    zeros: torch.Tensor  # fp16 [rows, G] (integer valued)
    codes: torch.Tensor  # int32 [rows, K]


def pack_nibbles(codes_rk: torch.Tensor) -> torch.Tensor:
    """int codes [rows, K] -> uint8 [rows, ceil(K/2)]; col 2j low nibble, 2j+1 high."""
    rows, K = codes_rk.shape
    if K % 2:
        codes_rk = torch.cat([codes_rk, torch.zeros(rows, 1, dtype=codes_rk.dtype)], dim=1)
    c = codes_rk.to(torch.int32) & 0xF
    return (c[:, 0::2] | (c[:, 1::2] << 4)).to(torch.uint8).contiguous()


def rtn_layer(rows: int, K: int, *, seed: int, groups: int = 1) -> RTNLayer:
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 16, (rows, K), generator=g, dtype=torch.int32)
    zeros = torch.randint(0, 16, (rows, groups), generator=g).to(torch.float16)
    scales = (torch.randn(rows, groups, generator=g).abs() * 0.01 + 1e-3).to(torch.float16)
    return RTNLayer(rows, K, pack_nibbles(codes), scales, zeros, codes)


def _pack_words(codes: torch.Tensor, bits: int, dim: int) -> torch.Tensor:
    """int codes -> int32 words of 32 // bits codes along ``dim`` (code i at bits ``bits * i``)."""
    per = 32 // bits
    c = (codes.to(torch.int64) & ((1 << bits) - 1)).movedim(dim, 0)
    n = c.shape[0]
    c = c.reshape(n // per, per, *c.shape[1:])
    word = torch.zeros((n // per, *c.shape[2:]), dtype=torch.int64)
    for i in range(per):
        word |= c[:, i] << (bits * i)
    word = torch.where(word >= 2**31, word - 2**32, word)
    return word.to(torch.int32).movedim(0, dim).contiguous()


@dataclass
class GPTQ8Layer:
    K: int
    N: int
    groupsize: int
    qweight: torch.Tensor  # int32 [K/4, N]
    scales: torch.Tensor  # fp16 [G, N]
    qzeros: torch.Tensor  # int32 [G, N/4] (v1: zero - 1)


def gptq8_layer(K: int, N: int, *, seed: int, groupsize: int = 128) -> GPTQ8Layer:
    g = torch.Generator().manual_seed(seed)
    G = (K + groupsize - 1) // groupsize
    codes = torch.randint(0, 256, (K, N), generator=g, dtype=torch.int32)
    zeros = torch.randint(0, 256, (G, N), generator=g, dtype=torch.int32)
    scales = (torch.randn(G, N, generator=g).abs() * 0.001 + 1e-4).to(torch.float16)
    return GPTQ8Layer(K, N, groupsize, _pack_words(codes, 8, 0), scales, _pack_words((zeros - 1) & 0xFF, 8, 1))


def dsv4_layer(N: int, K: int, *, wbits: int, seed: int, groupsize: int = 128) -> dict:
    """A ``Dsv4PackedLinear`` pack: uint8 codes [N, K / (8 // wbits)], scales / zeros fp16 [G, N]."""
    g = torch.Generator().manual_seed(seed)
    per = 8 // wbits
    G = (K + groupsize - 1) // groupsize
    codes = torch.randint(0, 1 << wbits, (N, K), generator=g, dtype=torch.int32).reshape(N, K // per, per)
    packed = torch.zeros((N, K // per), dtype=torch.int32)
    for i in range(per):
        packed |= codes[:, :, i] << (wbits * i)
    scales = (torch.randn(G, N, generator=g).abs() * 0.02 + 1e-4).to(torch.float16)
    zeros = torch.randint(0, 1 << wbits, (G, N), generator=g).to(torch.float16)
    return {"qweight_packed": packed.to(torch.uint8), "scales": scales, "qzeros": zeros, "wbits": wbits,
            "groupsize": groupsize, "in_features": K}


@dataclass
class MoEExperts:
    E: int
    K: int
    N: int
    qweight: torch.Tensor  # int32 [E, K/8, N]
    scales: torch.Tensor  # fp16 [E, K/32, N]
    qzeros: torch.Tensor  # int32 [E, K/32, N/8]
    layers: list  # per-expert GPTQLayer (codes kept only when keep_codes)


def moe_experts(E: int, K: int, N: int, *, seed: int, keep_codes: bool = True) -> MoEExperts:
    layers = [gptq_layer(K, N, seed=seed + 1000 * e) for e in range(E)]
    qw = torch.stack([l.qweight for l in layers])
    sc = torch.stack([l.scales for l in layers])
    qz = torch.stack([l.qzeros for l in layers])
    if not keep_codes:
        for l in layers:
            l.codes = None
    return MoEExperts(E, K, N, qw, sc, qz, layers)


def router_topk(T: int, E: int, topk: int, *, seed: int) -> torch.Tensor:
    """Top-k expert ids (int64 [T, topk]) of seeded N(0,1) router logits."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g)
    return torch.topk(logits, topk, dim=-1).indices


WORKLOADS = {
    "gptq_gs32_m16": dict(M=16, shapes=[(4096, 4096)], groupsize=32, v1=True, act_order=False),
    "decode_actorder": dict(M=(1, 8), shapes=[(5120, 5120), (5120, 17408), (17408, 5120), (5120, 1024)],
                            groupsize=32, v1=True, act_order=True),
    "dit_large_m": dict(M=4096, shapes=[(3072, 3072), (3072, 12288), (12288, 3072)], groupsize=32,
                        v1=False, act_order=False, outliers=True),
    "padded_gs26": dict(M=256, shapes=[(1040, 3072)], groupsize=26, v1=True, act_order=False),
    "rtn_moe": dict(rtn_linear=dict(M=512, K=1024, N=2048),
                    rtn_embedding=dict(V=32768, D=1024, T=4096),
                    moe=dict(E=64, K=4096, N=2048, T=512, topk=8)),
}
