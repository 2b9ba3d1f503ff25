"""CPU oracle of the int4 dequant + GEMM path: TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's CPU ("eager"/"packed") path. Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
it, and only to check results against (or as the timed CPU baseline); the
product never calls it.

Values of 16-bit floats are carried as float32 arrays holding exactly
representable values; rounding to a 16-bit type is explicit (``round_to``).
Each function cites the reference function it restates (paths relative to
the onecompression-runtime tree).

How each function is pinned (tests/test_oracle.py):
    round_to                -> torch's own fp32->bf16/fp16 conversions (the
                               reference's arithmetic), incl. ties, NaN, inf,
                               overflow and subnormals
    unpack_rows / zeros     -> hand-derived known answers (tests/golden/kats.json),
                               sign-bit words, pack/unpack round trips
    dequant_gptq            -> exact rational brute force (kats.json), closed
                               special cases (s=1, z=8), v1/v2 and g_idx identities
    rtn_dequant             -> torch's 16-bit elementwise ops applied in the
                               reference's order on adversarial inputs; nibble KATs
    dsv4_unpack / dequant   -> exact-rational known answers (kats.json: byte
                               order, fp32 sub and mul rounding, output rounding),
                               pack/unpack round trip, orientation identity
    embedding               -> row gather identity + output-dtype rule
    conv1d / conv_transpose -> torch's float64 F.conv1d / F.conv_transpose1d
    linear / gptq_linear    -> float64 brute force on tiny shapes; act-order and
                               padded-groups invariances
    moe                     -> per-pair brute force
"""
from __future__ import annotations

import numpy as np

_F32 = np.float32


# ---------------------------------------------------------------------------
# Rounding
def f32_to_bf16_bits(x) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit pattern (NaN stays a quiet NaN)."""
    x = np.ascontiguousarray(x, dtype=_F32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    out = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(_F32)


def round_to(x, dtype: str) -> np.ndarray:
    """Round float32 values to ``dtype`` ('bf16', 'f16', 'f32'); returns float32."""
    x = np.asarray(x, dtype=_F32)
    if dtype == "f32":
        return x.copy()
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    if dtype == "f16":
        with np.errstate(over="ignore"):
            return x.astype(np.float16).astype(_F32)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# GPTQ formats
def unpack_rows(packed, num_rows: int, wbits: int) -> np.ndarray:
    """quant_utils._unpack_rows (quant_utils.py:12-28): value i of word r is
    row r*(32/wbits)+i, at bits wbits*i; rows past num_rows are dropped."""
    if 32 % wbits:
        raise ValueError(f"wbits must divide 32, got {wbits}")
    p = np.asarray(packed, dtype=np.int32).view(np.uint32)
    per = 32 // wbits
    mask = np.uint32((1 << wbits) - 1)
    R, C = p.shape
    out = np.empty((R, per, C), dtype=np.int32)
    for i in range(per):
        out[:, i, :] = (p >> np.uint32(wbits * i)) & mask
    return out.reshape(R * per, C)[:num_rows]


def unpack_int_weights(packed, wbits: int, original_shape) -> np.ndarray:
    """quant_utils.unpack_int_weights (quant_utils.py:36-42): -> [out, in]."""
    return np.ascontiguousarray(unpack_rows(packed, original_shape[1], wbits).T)


def unpack_zeros(qzeros, wbits: int, out_features: int) -> np.ndarray:
    """quant_utils.unpack_zeros (quant_utils.py:45-47): [G, N/per] -> [G, N]."""
    qz = np.ascontiguousarray(np.asarray(qzeros, dtype=np.int32).T)
    return np.ascontiguousarray(unpack_rows(qz, out_features, wbits).T)


def pack_rows(codes_kn, wbits: int = 4) -> np.ndarray:
    """Inverse of unpack_rows (layers/fused_int4_linear.py:76-91 on [K, N])."""
    c = np.asarray(codes_kn, dtype=np.uint32)
    per = 32 // wbits
    K, N = c.shape
    Kp = -(-K // per) * per
    full = np.zeros((Kp, N), dtype=np.uint32)
    full[:K] = c & np.uint32((1 << wbits) - 1)
    full = full.reshape(Kp // per, per, N)
    word = np.zeros((Kp // per, N), dtype=np.uint32)
    for i in range(per):
        word |= full[:, i, :] << np.uint32(wbits * i)
    return word.view(np.int32)


def pack_zeros(zeros_gn, v1: bool, wbits: int = 4) -> np.ndarray:
    """Zeros [G, N] -> qzeros [G, N/per]; v1 stores (z - 1) & mask."""
    z = np.asarray(zeros_gn, dtype=np.int64)
    mask = (1 << wbits) - 1
    stored = ((z - 1) & mask) if v1 else (z & mask)
    return np.ascontiguousarray(pack_rows(np.ascontiguousarray(stored.T), wbits).T)


def dequant_gptq(qweight, scales, qzeros, g_idx, in_features: int, out_features: int,
                 dtype: str, v1: bool = True, wbits: int = 4) -> np.ndarray:
    """quant_utils.dequant_gptq_to_fp (quant_utils.py:50-69) -> [N, K] float32
    holding values of ``dtype``: RNE_dtype(f32(s) * f32(w - z)), with
    v1 zeros restored as (z + 1) & mask and groups gathered by g_idx."""
    w = unpack_int_weights(qweight, wbits, (out_features, in_features))  # [N, K]
    z = unpack_zeros(qzeros, wbits, out_features)  # [G, N]
    if v1:
        z = (z + 1) & ((1 << wbits) - 1)
    g = np.asarray(g_idx, dtype=np.int64)
    s = np.asarray(scales, dtype=_F32)[g, :].T  # [N, K]
    ze = z[g, :].T
    prod = s * (w.astype(_F32) - ze.astype(_F32))
    return round_to(prod, dtype)


def default_g_idx(in_features: int, groupsize: int) -> np.ndarray:
    """g(k) = k // groupsize (layers/packed_gptq_linear.py:53-56)."""
    return np.arange(in_features, dtype=np.int64) // groupsize


def repack_groups_to_32(qweight, in_features: int, out_features: int, groupsize: int):
    """layers/fused_int4_linear.py:94-124: each group of `groupsize` rows moved
    into a 32-row slot (rest zero codes); returns (qweight_padded, 32*G)."""
    if groupsize <= 0 or groupsize > 32:
        raise ValueError(f"groupsize must be in 1..32, got {groupsize}")
    if in_features % groupsize:
        raise ValueError("in_features must be divisible by groupsize")
    G = in_features // groupsize
    w = unpack_rows(qweight, in_features, 4)  # [K, N]
    padded = np.zeros((G * 32, out_features), dtype=np.int32)
    for g in range(G):
        padded[32 * g: 32 * g + groupsize] = w[groupsize * g: groupsize * (g + 1)]
    return pack_rows(padded, 4), G * 32


# ---------------------------------------------------------------------------
# RTN formats
def rtn_unpack(qweight_u8, in_features: int) -> np.ndarray:
    """Byte j -> cols 2j (low nibble), 2j+1 (high) (quant_utils.py:85-90,
    layers/packed_conv.py:36-45); cropped to in_features."""
    q = np.asarray(qweight_u8, dtype=np.uint8)
    rows, half = q.shape
    out = np.empty((rows, half, 2), dtype=np.int32)
    out[:, :, 0] = q & 0x0F
    out[:, :, 1] = (q >> 4) & 0x0F
    return out.reshape(rows, 2 * half)[:, :in_features]


def rtn_pack(codes) -> np.ndarray:
    """layers/packed_conv.py:23-33."""
    c = np.asarray(codes, dtype=np.int64)
    rows, cols = c.shape
    if cols % 2:
        c = np.concatenate([c, np.zeros((rows, 1), dtype=np.int64)], axis=1)
    return ((c[:, 0::2] & 0xF) | ((c[:, 1::2] & 0xF) << 4)).astype(np.uint8)


def rtn_dequant(qweight_u8, scales, zeros, in_features: int, out_features: int,
                dtype: str) -> np.ndarray:
    """quant_utils.dequant_extra_u8_to_weight (quant_utils.py:72-103): every
    op in ``dtype`` with its own rounding: RNE(RNE(w - RNE(z)) * RNE(s))."""
    w = rtn_unpack(qweight_u8, in_features).astype(_F32)  # exact in every dtype
    s = round_to(np.asarray(scales, dtype=_F32), dtype)
    z = round_to(np.asarray(zeros, dtype=_F32), dtype)
    G = s.shape[1]
    if G != 1 and in_features % G:
        raise RuntimeError(f"in_features={in_features} not divisible by num_groups={G}")
    gs = in_features // G
    se = np.repeat(s, gs, axis=1)
    ze = np.repeat(z, gs, axis=1)
    d = round_to(w - ze, dtype)
    return round_to(d * se, dtype)


def embedding_dtype(scales_dtype: str) -> str:
    """Output dtype rule of PackedEmbedding (layers/packed_linear.py:98)."""
    return scales_dtype if scales_dtype in ("bf16", "f16", "f32") else "f16"


def embedding(ids, qweight_u8, scales, zeros, embedding_dim: int, dtype: str) -> np.ndarray:
    """PackedEmbedding.forward (layers/packed_linear.py:93-104): gather rows
    (negative ids wrap as in torch indexing) then RTN-dequant them."""
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    V = np.asarray(qweight_u8).shape[0]
    if ((flat < -V) | (flat >= V)).any():
        raise IndexError("embedding id out of range")
    flat = np.where(flat < 0, flat + V, flat)
    q = np.asarray(qweight_u8)[flat]
    return rtn_dequant(q, np.asarray(scales)[flat], np.asarray(zeros)[flat], embedding_dim,
                       flat.shape[0], dtype)


# ---------------------------------------------------------------------------
# DSV4 (DeepSeek-V4 QEP) uint8 packing along the in-dim
def dsv4_unpack(qweight_packed, wbits: int, in_features: int) -> np.ndarray:
    """dequant_dsv4_packed's unpack (layers/dsv4_packed_linear.py:28-35): byte
    j of row n holds columns per*j + i at bits wbits*i, per = 8 // wbits;
    cropped to in_features. -> int32 [out, in]."""
    per = 8 // wbits
    q = np.asarray(qweight_packed, dtype=np.uint8).astype(np.int32)
    out_f, ncol = q.shape
    codes = np.empty((out_f, ncol, per), dtype=np.int32)
    for i in range(per):
        codes[:, :, i] = (q >> (wbits * i)) & ((1 << wbits) - 1)
    return codes.reshape(out_f, ncol * per)[:, :in_features]


def dsv4_pack(codes, wbits: int) -> np.ndarray:
    """Inverse of dsv4_unpack: int codes [out, in] -> uint8 [out, ceil(in / per)]."""
    per = 8 // wbits
    c = np.asarray(codes, dtype=np.int64)
    out_f, k = c.shape
    kp = (k + per - 1) // per * per
    full = np.zeros((out_f, kp), dtype=np.int64)
    full[:, :k] = c & ((1 << wbits) - 1)
    full = full.reshape(out_f, kp // per, per)
    b = np.zeros((out_f, kp // per), dtype=np.int64)
    for i in range(per):
        b |= full[:, :, i] << (wbits * i)
    return b.astype(np.uint8)


def dequant_dsv4(qweight_packed, scales, qzeros, wbits: int, groupsize: int, in_features: int,
                 dtype: str) -> np.ndarray:
    """dequant_dsv4_packed (layers/dsv4_packed_linear.py:22-56) -> [out, in]
    float32 holding values of ``dtype``: in fp32, (q - z) then * s (each op
    rounded), one rounding to ``dtype``. Scales / zeros [G, out] or [out, G]
    (transposed when shaped (out, G), :49-50); groupsize <= 0: one per row."""
    q = dsv4_unpack(qweight_packed, wbits, in_features)
    out_f = q.shape[0]
    s = np.asarray(scales, dtype=_F32)
    z = np.asarray(qzeros, dtype=_F32)
    if groupsize <= 0:
        se, ze = s.reshape(out_f, 1), z.reshape(out_f, 1)
    else:
        G = (in_features + groupsize - 1) // groupsize
        if s.shape == (out_f, G):
            s, z = s.T, z.T
        g = np.arange(in_features) // groupsize
        se, ze = s[g, :].T, z[g, :].T
    d = q.astype(_F32) - ze
    return round_to((d * se).astype(_F32), dtype)


# ---------------------------------------------------------------------------
# Convolutions (F.conv1d / F.conv_transpose1d with groups = 1, as the packed
# conv layers call them after dequant, layers/packed_conv.py:162-170, :211-222)
def conv1d(x, weight, bias, stride: int, dilation: int, pad_left: int, T: int, out_dtype: str) -> np.ndarray:
    """y[b, o, t] = bias[o] + sum_{ci, kk} w[o, ci, kk] x[b, ci, t s + kk d - pad_left]
    (zeros outside the input), fp32 accumulation, one rounding."""
    x = np.asarray(x, dtype=_F32)
    w = np.asarray(weight, dtype=_F32)
    B, C, L = x.shape
    O, _, k = w.shape
    y = np.zeros((B, O, T), dtype=_F32)
    t = np.arange(T)
    for kk in range(k):
        pos = t * stride + kk * dilation - pad_left
        ok = (pos >= 0) & (pos < L)
        xs = np.zeros((B, C, T), dtype=_F32)
        xs[:, :, ok] = x[:, :, pos[ok]]
        y += np.matmul(w[:, :, kk], xs)  # [O, C] @ [B, C, T]
    if bias is not None:
        y += np.asarray(bias, dtype=_F32)[None, :, None]
    return round_to(y, out_dtype)


def conv_transpose1d(x, weight, bias, stride: int, dilation: int, padding: int, L_out: int,
                     out_dtype: str) -> np.ndarray:
    """y[b, o, t] = bias[o] + sum_{ci, kk, j : j s + kk d - padding = t} w[ci, o, kk] x[b, ci, j],
    fp32 accumulation, one rounding. weight [C_in, C_out, k]."""
    x = np.asarray(x, dtype=_F32)
    w = np.asarray(weight, dtype=_F32)
    B, C, L = x.shape
    _, O, k = w.shape
    y = np.zeros((B, O, L_out), dtype=_F32)
    j = np.arange(L)
    for kk in range(k):
        t = j * stride + kk * dilation - padding
        ok = (t >= 0) & (t < L_out)
        contrib = np.matmul(np.ascontiguousarray(w[:, :, kk].T), x)  # [O, C] @ [B, C, L]
        np.add.at(y, (slice(None), slice(None), t[ok]), contrib[:, :, ok])
    if bias is not None:
        y += np.asarray(bias, dtype=_F32)[None, :, None]
    return round_to(y, out_dtype)


# ---------------------------------------------------------------------------
# GEMM
def linear(x, weight, bias=None, out_dtype: str = "bf16", accumulate=np.float32) -> np.ndarray:
    """F.linear on the CPU: fp32 accumulation of 16-bit inputs, bias added in
    fp32, one rounding to the output dtype (layers/packed_gptq_linear.py:74)."""
    xa = np.asarray(x, dtype=accumulate)
    wa = np.asarray(weight, dtype=accumulate)
    acc = xa @ wa.T
    if bias is not None:
        acc = acc + np.asarray(bias, dtype=accumulate)
    return round_to(acc.astype(_F32), out_dtype)


def gptq_linear(x, qweight, scales, qzeros, g_idx, in_features: int, out_features: int,
                dtype: str, v1: bool = True, bias=None, wbits: int = 4,
                accumulate=np.float32) -> np.ndarray:
    """PackedGPTQLinear.forward (layers/packed_gptq_linear.py:66-74) and the
    eager path (backend.py:246-264): dequant to ``dtype``, then F.linear."""
    w = dequant_gptq(qweight, scales, qzeros, g_idx, in_features, out_features, dtype, v1, wbits)
    b = round_to(bias, dtype) if bias is not None else None
    return linear(x, w, b, dtype, accumulate)


def rtn_linear(x, qweight_u8, scales, zeros, in_features: int, out_features: int, dtype: str,
               bias=None, accumulate=np.float32) -> np.ndarray:
    """PackedRTNLinear.forward (layers/packed_linear.py:53-56)."""
    w = rtn_dequant(qweight_u8, scales, zeros, in_features, out_features, dtype)
    b = round_to(bias, dtype) if bias is not None else None
    return linear(x, w, b, dtype, accumulate)


def moe(x, topk_ids, expert_weights, dtype: str, accumulate=np.float32) -> np.ndarray:
    """Per-expert loop (no reference grouped GEMM; its MoE path runs one
    F.linear per expert, layers/dsv4_packed_linear.py:95-98):
    Y[t*topk + j] = x[t] @ Wd_{e(t,j)}^T. ``expert_weights[e]`` is the
    dequantized [N, K] weight of expert e."""
    ids = np.asarray(topk_ids, dtype=np.int64)
    T, topk = ids.shape
    N = expert_weights[0].shape[0]
    y = np.zeros((T * topk, N), dtype=_F32)
    flat = ids.reshape(-1)
    xa = np.asarray(x, dtype=_F32)
    for e in np.unique(flat):
        pairs = np.nonzero(flat == e)[0]
        y[pairs] = linear(xa[pairs // topk], expert_weights[e], None, dtype, accumulate)
    return y


def gemm_close(out, ref, rel: float = 2e-2, min_cos: float = 0.9999) -> tuple[bool, float, float]:
    """The GEMM tolerance: max|out - ref| <= rel * max|ref| and cosine >= min_cos."""
    o = np.asarray(out, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    err = float(np.max(np.abs(o - r))) if o.size else 0.0
    scale = float(np.max(np.abs(r))) if r.size else 0.0
    denom = float(np.linalg.norm(o) * np.linalg.norm(r))
    cos = float(o @ r / denom) if denom > 0 else 1.0
    return (err <= rel * scale and cos >= min_cos), err / scale if scale else err, cos
