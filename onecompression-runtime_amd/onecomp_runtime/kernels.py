"""Functional wrappers over the HIP C ABI (one function per entry point).

Each wrapper validates what the ABI cannot see (dtypes, devices, contiguity),
allocates outputs with ``torch.empty`` on the inputs' device, and launches on
torch's current stream. Nothing here computes on the host except
:func:`plan_groups`, the load-time row-layout planner.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _hip
from ._hip import check, dtype_code, lib, ptr, require_device, stream_of

try:  # CPython binding of the per-layer GEMM call (built beside the library)
    from . import _occall
except ImportError:
    _occall = None


@dataclass(frozen=True)
class GroupPlan:
    """Physical row layout of a GPTQ layer (see ``oc_int4_plan_groups``)."""

    k_phys: int
    group_rows: int
    num_groups: int
    identity: bool
    kmap: np.ndarray  # int32 [k_phys]; -1 marks a zero row
    kinv: np.ndarray | None  # uint16 [K]: physical row of each input row (k_phys <= 65536)


def plan_groups(in_features: int, groupsize: int, g_idx: torch.Tensor | None = None) -> GroupPlan:
    """Host-side planner: uniform physical groups of a multiple of 32 rows.

    Handles act-order ``g_idx`` (rows sorted by group), odd group sizes (each
    group padded to 32 rows, like the reference's ``_repack_groups_to_32``,
    layers/fused_int4_linear.py:94-124) and K padding.
    """
    K = int(in_features)
    gi = None
    if g_idx is not None:
        gi = np.ascontiguousarray(g_idx.detach().to("cpu", torch.int64).numpy())
        if gi.shape != (K,):
            raise ValueError(f"g_idx must have shape ({K},), got {tuple(gi.shape)}")
    k_phys, rows, ngroups, ident = (ctypes.c_int32() for _ in range(4))
    gptr = gi.ctypes.data if gi is not None else None
    check(
        lib().oc_int4_plan_groups(gptr, K, int(groupsize), None, 0, ctypes.byref(k_phys),
                                  ctypes.byref(rows), ctypes.byref(ngroups), ctypes.byref(ident)),
        "oc_int4_plan_groups",
    )
    kmap = np.empty(k_phys.value, dtype=np.int32)
    check(
        lib().oc_int4_plan_groups(gptr, K, int(groupsize), kmap.ctypes.data, kmap.size,
                                  ctypes.byref(k_phys), ctypes.byref(rows), ctypes.byref(ngroups),
                                  ctypes.byref(ident)),
        "oc_int4_plan_groups",
    )
    kinv = None
    if k_phys.value <= 65536:
        live = np.nonzero(kmap >= 0)[0]
        kinv = np.zeros(K, dtype=np.uint16)
        kinv[kmap[live]] = live.astype(np.uint16)
    return GroupPlan(k_phys.value, rows.value, ngroups.value, bool(ident.value), kmap, kinv)


def row_maps(plan: GroupPlan, device) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """Device copies of a plan's kmap (int32) and kinv (uint16 bits in an
    int16 tensor); both None for the identity layout."""
    if plan.identity:
        return None, None
    kmap = torch.from_numpy(plan.kmap).to(device)
    kinv = None if plan.kinv is None else torch.from_numpy(plan.kinv.view(np.int16)).to(device)
    return kmap, kinv


@dataclass
class TiledWeights:
    """A GPTQ layer in the tiled device layout of ``oc_int4_prepare``."""

    qt: torch.Tensor  # int32 [tiles, K_phys/32, 16, 4] (8-bit: [..., 8])
    st: torch.Tensor  # fp16/bf16 [tiles, G, 16]
    zt: torch.Tensor  # int32 [tiles, G, 2] (8-bit: [tiles, G, 4])
    N: int
    k_phys: int
    group_rows: int
    wbits: int = 4


def prepare(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor, *, in_features: int,
            out_features: int, kmap: torch.Tensor | None, k_phys: int, group_rows: int,
            v1: bool, wbits: int = 4) -> TiledWeights:
    """Build the tiled layout on the device (load time): rows permuted by
    ``kmap`` into uniform groups, zeros restored to their value. ``wbits``
    4 (``oc_int4_prepare``) or 8 (``oc_int8_prepare``)."""
    if wbits not in (4, 8):
        raise ValueError(f"wbits must be 4 or 8, got {wbits}")
    per = 32 // wbits
    dev = require_device(qweight, scales, qzeros, kmap)
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise ValueError("qweight and qzeros must be int32")
    if scales.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"scales must be fp16 or bf16, got {scales.dtype}")
    qweight, scales, qzeros = qweight.contiguous(), scales.contiguous(), qzeros.contiguous()
    N = int(out_features)
    tiles = (N + 15) // 16
    G = k_phys // group_rows
    if qweight.dim() != 2 or qweight.shape[1] != N or qweight.shape[0] < (int(in_features) + per - 1) // per:
        raise ValueError(f"qweight shape {tuple(qweight.shape)} does not hold {in_features} x {N} codes")
    if scales.dim() != 2 or scales.shape[1] != N or scales.shape[0] < G:
        raise ValueError(f"scales shape {tuple(scales.shape)} does not cover {G} groups x {N}")
    if qzeros.dim() != 2 or qzeros.shape[1] != N // per or qzeros.shape[0] < G:
        raise ValueError(f"qzeros shape {tuple(qzeros.shape)} does not cover {G} groups x {N // per}")
    if kmap is not None and (kmap.dtype != torch.int32 or kmap.numel() != k_phys):
        raise ValueError(f"kmap must be int32 with {k_phys} entries")
    qt = torch.empty((tiles, k_phys // 32, 16, 4 if wbits == 4 else 8), dtype=torch.int32, device=dev)
    st = torch.empty((tiles, G, 16), dtype=scales.dtype, device=dev)
    zt = torch.empty((tiles, G, 2 if wbits == 4 else 4), dtype=torch.int32, device=dev)
    fn = lib().oc_int4_prepare if wbits == 4 else lib().oc_int8_prepare
    check(
        fn(ptr(qweight), int(in_features), N, ptr(kmap), int(k_phys), int(group_rows),
           ptr(scales), dtype_code(scales.dtype), ptr(qzeros),
           _hip.OC_ZERO_V1 if v1 else _hip.OC_ZERO_V2, ptr(qt), ptr(st), ptr(zt), stream_of(dev)),
        f"oc_int{wbits}_prepare",
    )
    return TiledWeights(qt, st, zt, N, int(k_phys), int(group_rows), int(wbits))


def export_checkpoint(w: TiledWeights, *, row_src: torch.Tensor | None, out_rows: int, out_groups: int,
                      v1: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Checkpoint-format ``(qweight, scales, qzeros)`` from the tiled layout
    (``oc_int4_export``): qweight int32 [ceil(out_rows/8), N], code row k taken
    from physical row ``row_src[k]`` (identity when None); scales [out_groups, N]
    in the tiled scales' dtype; qzeros int32 [out_groups, N/8], v1 storing
    zero - 1. Rows and groups past the layer are zero."""
    dev = require_device(w.qt, row_src)
    if row_src is not None and (row_src.dtype != torch.int32 or row_src.numel() < out_rows):
        raise ValueError(f"row_src must be int32 with {out_rows} entries")
    N = w.N
    per = 32 // w.wbits
    qweight = torch.empty(((out_rows + per - 1) // per, N), dtype=torch.int32, device=dev)
    scales = torch.empty((out_groups, N), dtype=w.st.dtype, device=dev)
    qzeros = torch.empty((out_groups, N // per), dtype=torch.int32, device=dev)
    fn = lib().oc_int4_export if w.wbits == 4 else lib().oc_int8_export
    check(
        fn(ptr(w.qt), ptr(w.st), ptr(w.zt), N, w.k_phys, w.group_rows, ptr(row_src),
           int(out_rows), int(out_groups), _hip.OC_ZERO_V1 if v1 else _hip.OC_ZERO_V2,
           ptr(qweight), ptr(scales), ptr(qzeros), stream_of(dev)),
        f"oc_int{w.wbits}_export",
    )
    return qweight, scales, qzeros


def dequant_tiled(w: TiledWeights, kmap: torch.Tensor | None, in_features: int,
                  dtype: torch.dtype) -> torch.Tensor:
    """Dense [N, in_features] weight (original K order) from the tiled layout."""
    dev = require_device(w.qt, kmap)
    out = torch.empty((w.N, int(in_features)), dtype=dtype, device=dev)
    fn = lib().oc_int4_dequant_tiled if w.wbits == 4 else lib().oc_int8_dequant_tiled
    check(
        fn(ptr(w.qt), ptr(w.st), dtype_code(w.st.dtype), ptr(w.zt), ptr(kmap), w.N,
           w.k_phys, w.group_rows, int(in_features), ptr(out), dtype_code(dtype), stream_of(dev)),
        f"oc_int{w.wbits}_dequant_tiled",
    )
    return out


def unpack_rows(packed: torch.Tensor, num_rows: int, wbits: int) -> torch.Tensor:
    """int32 [R, C] of packed codes -> int32 [num_rows, C] (quant_utils.py:12-28)."""
    if 32 % wbits != 0:
        raise ValueError(f"wbits must divide 32, got {wbits}")
    dev = require_device(packed)
    packed = packed.contiguous()
    if packed.dtype != torch.int32:
        raise ValueError("packed must be int32")
    R, C = packed.shape
    out = torch.empty((num_rows, C), dtype=torch.int32, device=dev)
    check(lib().oc_unpack_rows(ptr(packed), R, C, int(wbits), int(num_rows), ptr(out), stream_of(dev)),
          "oc_unpack_rows")
    return out


def int4_dequant(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
                 g_idx: torch.Tensor | None, in_features: int, out_features: int,
                 dtype: torch.dtype, v1: bool = True, wbits: int = 4,
                 groupsize: int | None = None) -> torch.Tensor:
    """Dense [out, in] weight, bit-exact with quant_utils.dequant_gptq_to_fp."""
    dev = require_device(qweight, scales, qzeros, g_idx)
    K, N = int(in_features), int(out_features)
    gi32 = None
    if g_idx is not None:
        gi32 = g_idx.to(device=dev, dtype=torch.int32).contiguous()
    elif groupsize is None:
        raise ValueError("either g_idx or groupsize is required")
    qweight, scales, qzeros = qweight.contiguous(), scales.contiguous(), qzeros.contiguous()
    out = torch.empty((N, K), dtype=dtype, device=dev)
    check(
        lib().oc_int4_dequant(ptr(qweight), ptr(scales), dtype_code(scales.dtype), ptr(qzeros),
                              _hip.OC_ZERO_V1 if v1 else _hip.OC_ZERO_V2, ptr(gi32),
                              int(groupsize or 0), int(wbits), K, N, ptr(out), dtype_code(dtype),
                              stream_of(dev)),
        "oc_int4_dequant",
    )
    return out


def int4_gemm(a_2d: torch.Tensor, w: TiledWeights, *, in_features: int,
              kmap: torch.Tensor | None = None, kinv: torch.Tensor | None = None,
              bias: torch.Tensor | None = None,
              out: torch.Tensor | None = None, regime: int = _hip.OC_REGIME_AUTO) -> torch.Tensor:
    """C[M, N] = A @ dequant(W) + bias on the HIP device (fp32 accumulation).

    This is the per-call hot path of every GPTQ layer, kept lean: one
    device check, one output allocation, one ABI call.
    """
    qt = w.qt
    if not (a_2d.is_cuda and qt.is_cuda):
        require_device(a_2d, qt)  # raises with the reason
    idx = a_2d.get_device()
    if qt.get_device() != idx:
        raise ValueError(f"activations on cuda:{idx}, weights on cuda:{qt.get_device()}")
    adt = a_2d.dtype
    if adt is not torch.bfloat16 and adt is not torch.float16:
        raise ValueError(f"activations must be fp16 or bf16, got {adt}")
    if (a_2d.stride(-1) != 1 or a_2d.stride(0) % 8 or a_2d.data_ptr() % 16
            or (a_2d.shape[0] - 1) * a_2d.stride(0) + a_2d.shape[1] >= 1 << 30):
        # The kernels read 16-byte row segments (and address a block of rows
        # below 2 GiB with 32-bit offsets): copy into compact rows padded to 8.
        K = a_2d.shape[1]
        buf = torch.empty((a_2d.shape[0], (K + 7) // 8 * 8), dtype=adt, device=a_2d.device)
        a_2d = buf[:, :K].copy_(a_2d)
    M = a_2d.shape[0]
    N = w.N
    if out is None:
        out = torch.empty((M, N), dtype=adt, device=a_2d.device)
    stream = _hip._raw_stream(idx)
    ws, nbytes = _hip.gemm_workspace(idx, M, N, w.k_phys, w.group_rows, kmap is not None, regime, stream,
                                     w.wbits)
    args = (
        a_2d.data_ptr(), a_2d.stride(0), _DT[adt], M, in_features, qt.data_ptr(), w.st.data_ptr(),
        _DT[w.st.dtype], w.zt.data_ptr(), N, w.k_phys, w.group_rows,
        None if kmap is None else kmap.data_ptr(), None if kinv is None else kinv.data_ptr(),
        None if bias is None else bias.data_ptr(), 0 if bias is None else _DT[bias.dtype],
        out.data_ptr(), out.stride(0), None if ws is None else ws.data_ptr(), nbytes,
    )
    if w.wbits == 4:
        status = _gemm_fn()(*args, regime, stream)
    else:
        status = lib().oc_int8_gemm(*args, stream)
    if status:
        check(status, f"oc_int{w.wbits}_gemm")
    return out


_DT = {torch.float16: _hip.OC_DTYPE_F16, torch.bfloat16: _hip.OC_DTYPE_BF16,
       torch.float32: _hip.OC_DTYPE_F32}


class LayerCall:
    """One layer's GEMM call with its constant arguments bound once (weights,
    shape, row maps): the per-call work is the activation and output
    pointers, the stream and the workspace of this batch size. The call goes
    through the CPython binding ``_occall.Layer`` when it is built (else
    through ctypes, the same entry point). Activations that are not compact
    16-bit rows on the layer's device take ``int4_gemm`` (which validates,
    copies or raises)."""

    __slots__ = ("w", "qt", "in_features", "kmap", "kinv", "idx", "N", "fn", "mid", "ws", "has_kmap", "h")

    def __init__(self, w: TiledWeights, in_features: int, kmap: torch.Tensor | None,
                 kinv: torch.Tensor | None) -> None:
        self.w, self.qt, self.in_features, self.kmap, self.kinv = w, w.qt, int(in_features), kmap, kinv
        self.idx = w.qt.get_device()
        self.N = w.N
        self.has_kmap = kmap is not None
        self.fn = _gemm_fn() if w.wbits == 4 else lib().oc_int8_gemm
        self.mid = (self.in_features, w.qt.data_ptr(), w.st.data_ptr(), _DT[w.st.dtype], w.zt.data_ptr(), w.N,
                    w.k_phys, w.group_rows, None if kmap is None else kmap.data_ptr(),
                    None if kinv is None else kinv.data_ptr())
        self.ws: dict = {}  # (M, stream) -> (workspace pointer, bytes)
        self.h = None
        if _occall is not None:
            self.h = _occall.Layer(ctypes.cast(self.fn, ctypes.c_void_p).value, w.wbits, *self.mid)

    def __call__(self, a_2d: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        adt = a_2d.dtype
        M = a_2d.shape[0]
        if ((adt is not torch.bfloat16 and adt is not torch.float16) or not a_2d.is_cuda
                or a_2d.get_device() != self.idx or a_2d.stride(-1) != 1 or a_2d.stride(0) % 8
                or a_2d.data_ptr() % 16 or M * a_2d.stride(0) >= 1 << 30):
            return int4_gemm(a_2d, self.w, in_features=self.in_features, kmap=self.kmap, kinv=self.kinv,
                             bias=bias)
        out = torch.empty((M, self.N), dtype=adt, device=a_2d.device)
        stream = _hip._raw_stream(self.idx)
        key = (M, stream)
        wsp = self.ws.get(key)
        if wsp is None:
            w = self.w
            ws, nbytes = _hip.gemm_workspace(self.idx, M, self.N, w.k_phys, w.group_rows, self.has_kmap,
                                             _hip.OC_REGIME_AUTO, stream, w.wbits)
            wsp = (None if ws is None else ws.data_ptr(), nbytes, ws)
            if len(self.ws) > 64:
                self.ws.clear()
            self.ws[key] = wsp  # (a buffer the stream outgrows later stays allocated and valid)
        h = self.h
        if h is not None:
            status = h(a_2d.data_ptr(), a_2d.stride(0), _DT[adt], M, None if bias is None else bias.data_ptr(),
                       0 if bias is None else _DT[bias.dtype], out.data_ptr(), out.stride(0), wsp[0], wsp[1], stream)
        elif self.w.wbits == 4:
            status = self.fn(a_2d.data_ptr(), a_2d.stride(0), _DT[adt], M, *self.mid,
                             None if bias is None else bias.data_ptr(), 0 if bias is None else _DT[bias.dtype],
                             out.data_ptr(), out.stride(0), wsp[0], wsp[1], _hip.OC_REGIME_AUTO, stream)
        else:
            status = self.fn(a_2d.data_ptr(), a_2d.stride(0), _DT[adt], M, *self.mid,
                             None if bias is None else bias.data_ptr(), 0 if bias is None else _DT[bias.dtype],
                             out.data_ptr(), out.stride(0), wsp[0], wsp[1], stream)
        if status:
            check(status, f"oc_int{self.w.wbits}_gemm")
        return out


_GEMM_FN = None


def _gemm_fn():
    global _GEMM_FN
    if _GEMM_FN is None:
        _GEMM_FN = lib().oc_int4_gemm
    return _GEMM_FN


def rtn_dequant(qweight_u8: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
                in_features: int, out_features: int, dtype: torch.dtype) -> torch.Tensor:
    """Dense [rows, in] weight, bit-exact with quant_utils.dequant_extra_u8_to_weight."""
    dev = require_device(qweight_u8, scales, zeros)
    qweight_u8, scales, zeros = qweight_u8.contiguous(), scales.contiguous(), zeros.contiguous()
    rows = int(out_features)
    K = int(in_features)
    G = scales.shape[1]
    out = torch.empty((rows, K), dtype=dtype, device=dev)
    check(
        lib().oc_rtn_dequant(ptr(qweight_u8), rows, qweight_u8.shape[1], ptr(scales),
                             dtype_code(scales.dtype), ptr(zeros), dtype_code(zeros.dtype), G, K,
                             ptr(out), dtype_code(dtype), stream_of(dev)),
        "oc_rtn_dequant",
    )
    return out


def rtn_linear(x_2d: torch.Tensor, qweight_u8: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
               in_features: int, bias: torch.Tensor | None = None) -> torch.Tensor:
    """Fused PackedRTNLinear forward for fp16/bf16 activations."""
    dev = require_device(x_2d, qweight_u8, scales, zeros, bias)
    if x_2d.stride(-1) != 1:
        x_2d = x_2d.contiguous()
    M = x_2d.shape[0]
    N = qweight_u8.shape[0]
    G = scales.shape[1]
    c = torch.empty((M, N), dtype=x_2d.dtype, device=dev)
    check(
        lib().oc_rtn_linear(ptr(x_2d), x_2d.stride(0), dtype_code(x_2d.dtype), M, int(in_features),
                            ptr(qweight_u8), qweight_u8.shape[1], ptr(scales), dtype_code(scales.dtype),
                            ptr(zeros), dtype_code(zeros.dtype), G, N, ptr(bias),
                            dtype_code(bias.dtype) if bias is not None else 0, ptr(c), c.stride(0),
                            stream_of(dev)),
        "oc_rtn_linear",
    )
    return c


def rtn_embedding(ids: torch.Tensor, qweight_u8: torch.Tensor, scales: torch.Tensor,
                  zeros: torch.Tensor, embedding_dim: int, dtype: torch.dtype,
                  bad_id_flag: torch.Tensor | None = None) -> torch.Tensor:
    """out[t, :] = RTN dequant of table row ids[t], shape [T, D]."""
    dev = require_device(ids, qweight_u8, scales, zeros, bad_id_flag)
    flat = ids.reshape(-1)
    if flat.dtype != torch.int64:
        flat = flat.long()
    flat = flat.contiguous()
    D = int(embedding_dim)
    out = torch.empty((flat.shape[0], D), dtype=dtype, device=dev)
    check(
        lib().oc_rtn_embedding(ptr(flat), flat.shape[0], ptr(qweight_u8), qweight_u8.shape[0],
                               qweight_u8.shape[1], ptr(scales), dtype_code(scales.dtype), ptr(zeros),
                               dtype_code(zeros.dtype), scales.shape[1], D, ptr(out), dtype_code(dtype),
                               ptr(bad_id_flag), stream_of(dev)),
        "oc_rtn_embedding",
    )
    return out


def moe_route(topk_ids: torch.Tensor, num_experts: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Stable counting sort of routed (token, slot) pairs by expert."""
    dev = require_device(topk_ids)
    ids = topk_ids.to(torch.int64).contiguous()
    T, topk = ids.shape
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    sorted_pairs = torch.empty(T * topk, dtype=torch.int32, device=dev)
    check(lib().oc_moe_route(ptr(ids), T, topk, int(num_experts), ptr(offsets), ptr(sorted_pairs),
                             stream_of(dev)), "oc_moe_route")
    return offsets, sorted_pairs


def prepare_experts(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor, *,
                    group_rows: int = 32, v1: bool = True) -> TiledWeights:
    """Stacked per-expert GPTQ tensors [E, K/8, N] / [E, G, N] / [E, G, N/8]
    -> tiled layout with a leading expert axis."""
    E, K8, N = qweight.shape
    K = 8 * K8
    parts = [prepare(qweight[e], scales[e], qzeros[e], in_features=K, out_features=N, kmap=None,
                     k_phys=K, group_rows=group_rows, v1=v1) for e in range(E)]
    return TiledWeights(torch.stack([p.qt for p in parts]), torch.stack([p.st for p in parts]),
                        torch.stack([p.zt for p in parts]), N, K, group_rows)


def int4_moe_gemm(x: torch.Tensor, topk: int, w: TiledWeights, expert_offsets: torch.Tensor,
                  sorted_pairs: torch.Tensor) -> torch.Tensor:
    """Y[t*topk + j, :] = x[t] @ dequant(W_{e(t,j)}) for every routed pair."""
    dev = require_device(x, w.qt, expert_offsets, sorted_pairs)
    x = x.contiguous()
    T, K = x.shape
    E = w.qt.shape[0]
    if expert_offsets.dtype != torch.int32 or expert_offsets.numel() != E + 1:
        raise ValueError(f"expert_offsets must be int32 with {E + 1} entries (one expert per weight)")
    if sorted_pairs.dtype != torch.int32 or sorted_pairs.numel() < T * topk:
        raise ValueError(f"sorted_pairs must be int32 with {T * topk} entries")
    if K != w.k_phys:
        raise ValueError(f"x has {K} features, the experts {w.k_phys}")
    y = torch.empty((T * topk, w.N), dtype=x.dtype, device=dev)
    check(
        lib().oc_int4_moe_gemm(ptr(x), x.stride(0), dtype_code(x.dtype), T, int(topk), K, ptr(w.qt), ptr(w.st),
                               dtype_code(w.st.dtype), ptr(w.zt), int(w.group_rows), E, w.N,
                               ptr(expert_offsets), ptr(sorted_pairs), ptr(y), y.stride(0), stream_of(dev)),
        "oc_int4_moe_gemm",
    )
    return y


def _dsv4_strides(scales: torch.Tensor, out_features: int, in_features: int, groupsize: int):
    """Element strides (per output row, per group) of a DSV4 scale/zero tensor,
    whichever of the reference's orientations it has (dsv4_packed_linear.py:40-51)."""
    if groupsize <= 0:
        return 1, 0
    G = (in_features + groupsize - 1) // groupsize
    if tuple(scales.shape) == (out_features, G):
        return G, 1
    if tuple(scales.shape) == (G, out_features):
        return 1, out_features
    raise ValueError(f"scales shape {tuple(scales.shape)} is neither ({out_features}, {G}) nor ({G}, {out_features})")


def dsv4_dequant(qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, *, wbits: int,
                 groupsize: int, in_features: int, dtype: torch.dtype) -> torch.Tensor:
    """Dense [out, in] weight, bit-exact with dequant_dsv4_packed (oc_dsv4_dequant)."""
    dev = require_device(qweight, scales, zeros)
    qweight, scales, zeros = qweight.contiguous(), scales.contiguous(), zeros.contiguous()
    N = qweight.shape[0]
    sn, sg = _dsv4_strides(scales, N, in_features, groupsize)
    out = torch.empty((N, int(in_features)), dtype=dtype, device=dev)
    check(lib().oc_dsv4_dequant(ptr(qweight), N, qweight.shape[1], int(wbits), int(in_features), ptr(scales),
                                dtype_code(scales.dtype), ptr(zeros), dtype_code(zeros.dtype), int(groupsize), sn,
                                sg, ptr(out), dtype_code(dtype), stream_of(dev)), "oc_dsv4_dequant")
    return out


def dsv4_gemm(x_2d: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, *,
              wbits: int, groupsize: int, in_features: int, bias: torch.Tensor | None = None) -> torch.Tensor:
    """C[M, N] = x @ dequant_dsv4(W)^T + bias (oc_dsv4_gemm), fp16/bf16 x."""
    dev = require_device(x_2d, qweight, scales, zeros, bias)
    if x_2d.stride(-1) != 1 or x_2d.stride(0) % 8 or x_2d.data_ptr() % 16:
        x_2d = x_2d.contiguous()
    M, K = x_2d.shape
    N = qweight.shape[0]
    sn, sg = _dsv4_strides(scales, N, in_features, groupsize)
    out = torch.empty((M, N), dtype=x_2d.dtype, device=dev)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    stream = _hip._raw_stream(idx)
    nbytes = int(lib().oc_dsv4_gemm_workspace_bytes(M, N, K))
    ws = _hip.workspace.get(idx, nbytes, stream)
    check(lib().oc_dsv4_gemm(ptr(x_2d), x_2d.stride(0), dtype_code(x_2d.dtype), M, int(in_features), ptr(qweight),
                             qweight.shape[1], int(wbits), ptr(scales), dtype_code(scales.dtype), ptr(zeros),
                             dtype_code(zeros.dtype), int(groupsize), sn, sg, N, ptr(bias),
                             dtype_code(bias.dtype) if bias is not None else 0, ptr(out), out.stride(0), ptr(ws),
                             nbytes, stream), "oc_dsv4_gemm")
    return out
