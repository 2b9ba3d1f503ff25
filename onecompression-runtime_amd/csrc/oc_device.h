// Device-side building blocks shared by every kernel of libonecomp_hip.so:
// element-type helpers, the exact GPTQ dequant, the RTN per-op-rounded dequant
// and the gfx950 MFMA wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oc_internal.h"

namespace oc {

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short v8i16;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 v8f16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float v4f32;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float v2f32;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 v2f16;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 v2bf16;

template <typename To, typename From>
__device__ __forceinline__ To bitcast(const From &v) {
  return __builtin_bit_cast(To, v);
}

// ---- scalar conversions (all round-to-nearest-even) ------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return bitcast<float>(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(bitcast<_Float16>(h));
}
// Two floats -> packed pair (lo = a, hi = b), RNE (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  v2f32 v = {a, b};
  return bitcast<uint32_t>(__builtin_convertvector(v, v2bf16));
}
__device__ __forceinline__ uint32_t pack2_f16(float a, float b) {
  v2f32 v = {a, b};
  return bitcast<uint32_t>(__builtin_convertvector(v, v2f16));
}
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (DT == OC_DTYPE_BF16) return pack2_bf16(a, b);
  else return pack2_f16(a, b);
}
// Round a float to the 16-bit type DT and return it widened back to float.
template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == OC_DTYPE_F32) {
    return x;
  } else if constexpr (DT == OC_DTYPE_BF16) {
    return bf16_to_f32(static_cast<uint16_t>(pack2_bf16(x, 0.f)));
  } else {
    return static_cast<float>(static_cast<_Float16>(x));
  }
}
template <int DT>
__device__ __forceinline__ float load_as_f32(const void *p, int64_t i) {
  if constexpr (DT == OC_DTYPE_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
  else if constexpr (DT == OC_DTYPE_F16) return f16_to_f32(static_cast<const uint16_t *>(p)[i]);
  else return static_cast<const float *>(p)[i];
}
// Runtime-typed scalar load (load-time / epilogue paths only).
__device__ __forceinline__ float load_any_f32(const void *p, int64_t i, int dt) {
  switch (dt) {
    case OC_DTYPE_BF16: return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    case OC_DTYPE_F16: return f16_to_f32(static_cast<const uint16_t *>(p)[i]);
    case OC_DTYPE_F32: return static_cast<const float *>(p)[i];
    case OC_DTYPE_U8: return static_cast<float>(static_cast<const uint8_t *>(p)[i]);
    case OC_DTYPE_I32: return static_cast<float>(static_cast<const int32_t *>(p)[i]);
    default: return 0.f;
  }
}

// ---- GPTQ dequant ------------------------------------------------------------
//
// The reference dequant (quant_utils.py:68-69) is one exact fp32 product
// s * (w - z) followed by a single rounding to the output type: with s a
// 16-bit float (<= 11 significant bits) and |w - z| <= 15 the product has at
// most 15 significant bits, so fp32 holds it exactly.
//
// Each 4-bit code w is placed in the mantissa of the fp16 number 1024.0
// (bits 0x6400): at bits 0-3 it reads as 1024 + w, at bits 4-7 as 1024 + 16w.
// With c = -s * (1024 + z) and, for the second form, s16 = s / 16 and
// c16 = -s * (64 + z), every product s * (1024 + w), s16 * (1024 + 16w) and
// both constants need at most 22 significant bits, so fma(h, s, c) yields the
// exact s * (w - z) (v_fma_mix_f32 reads the fp16 operand directly). One
// shift, four and-or, eight fma and four pack ops dequantize one 8-code word.

// (x & mask) | magic in one VALU op (mask from an SGPR, magic from a VGPR).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(magic));
  return r;
}

struct GroupParam {
  float s;    // scale (exact fp32)
  float c;    // -s * (1024 + zero)
  float s16;  // s / 16
  float c16;  // -s * (64 + zero)
};

__device__ __forceinline__ GroupParam make_group_param(float s, int zero) {
  const float zf = static_cast<float>(zero);
  GroupParam p;
  p.s = s;
  p.c = -s * (zf + 1024.f);
  p.s16 = s * 0.0625f;
  p.c16 = -s * (zf + 64.f);
  return p;
}

// Codes 0, 1, 4, 5 of a packed word (code i at bits 4i) with one group
// parameter: returns {codes 0|1, codes 4|5} as packed pairs, each value
// rounded once (RNE) to DT. Applied to q >> 8 it yields codes 2, 3, 6, 7.
template <int DT>
__device__ __forceinline__ uint2 dequant8_half(uint32_t q, GroupParam gp) {
  const uint32_t magic = 0x64006400u;
  const v2f16 h0 = bitcast<v2f16>(and_or(q, 0x000F000Fu, magic));  // 1024 + codes 0, 4
  const v2f16 h1 = bitcast<v2f16>(and_or(q, 0x00F000F0u, magic));  // 1024 + 16 * codes 1, 5
  const float f0 = __builtin_fmaf(static_cast<float>(h0[0]), gp.s, gp.c);
  const float f4 = __builtin_fmaf(static_cast<float>(h0[1]), gp.s, gp.c);
  const float f1 = __builtin_fmaf(static_cast<float>(h1[0]), gp.s16, gp.c16);
  const float f5 = __builtin_fmaf(static_cast<float>(h1[1]), gp.s16, gp.c16);
  return uint2{pack2<DT>(f0, f1), pack2<DT>(f4, f5)};
}

// Dequantize the 8 codes of one packed word (code i at bits 4i) with one
// group parameter; returns 4 dwords holding the 8 results in natural order
// (dword d = codes 2d, 2d+1), each rounded once (RNE) to DT.
template <int DT>
__device__ __forceinline__ uint4 dequant8(uint32_t q, GroupParam gp) {
  const uint2 lo = dequant8_half<DT>(q, gp);       // codes 0|1, 4|5
  const uint2 hi = dequant8_half<DT>(q >> 8, gp);  // codes 2|3, 6|7
  return uint4{lo.x, hi.x, lo.y, hi.y};
}

// 8-bit GPTQ codes: the 8 codes of two words (code i = byte i % 4 of word
// i / 4), each RNE_DT(s * (code - zero)). With c = -s * zero exact, fma(code,
// s, c) is the exact product s * (code - zero) (a 16-bit scale times an
// integer of at most 9 bits fits fp32), rounded once on packing.
template <int DT>
__device__ __forceinline__ uint4 dequant8_u8(uint32_t q0, uint32_t q1, float s, float c) {
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = __builtin_fmaf(static_cast<float>((q0 >> (8 * i)) & 0xFFu), s, c);
    f[4 + i] = __builtin_fmaf(static_cast<float>((q1 >> (8 * i)) & 0xFFu), s, c);
  }
  return uint4{pack2<DT>(f[0], f[1]), pack2<DT>(f[2], f[3]), pack2<DT>(f[4], f[5]), pack2<DT>(f[6], f[7])};
}

// DSV4 codes (layers/dsv4_packed_linear.py:47-56): the 8 codes of q (code i
// at bits BITS * i), each RNE_DT((f32(code) - z) * s) with the subtraction and
// the product rounded in fp32 as the reference's torch ops do (two separate
// fp32 operations, not a fused multiply-add).
// The fp32 product passes through an empty asm (no instruction): folded into
// the fp16 packing conversion (v_fma_mixlo_f16), it would be rounded once
// instead of to fp32 first, and differ from the reference on fp16 ties.
__device__ __forceinline__ float opaque(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

template <int DT, int BITS>
__device__ __forceinline__ uint4 dsv4_dequant8(uint32_t q, float s, float z) {
  float f[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float d = __fsub_rn(static_cast<float>((q >> (BITS * i)) & ((1u << BITS) - 1)), z);
    f[i] = opaque(__fmul_rn(d, s));
  }
  return uint4{pack2<DT>(f[0], f[1]), pack2<DT>(f[2], f[3]), pack2<DT>(f[4], f[5]), pack2<DT>(f[6], f[7])};
}

// ---- tiled GPTQ layout ("tile16") ---------------------------------------------
//
// Built once per layer by oc_int4_prepare. Output features are cut into tiles
// of 16; within a tile the 32-row K steps follow each other, and within a K
// step the 16 columns' 4 packed words (rows 8w..8w+7 of the step, w = 0..3)
// are adjacent, so one 16-byte load gives a lane a whole 32-row group of one
// column and a wave reads 1 KB of consecutive bytes per instruction:
//   word(t, ks, c, w)   qt[((t * KS + ks) * 16 + c) * 4 + w]
//   scale(t, g, c)      st[(t * G + g) * 16 + c]
//   zero word(t, g, h)  zt[(t * G + g) * 2 + h]   (columns 8h..8h+7, stored
//                                                   as the zero itself)
// KS = K_phys / 32 and G = K_phys / group_rows; columns past N are zero.
// 8-bit layers use the same tiles with 8 words per column and K step (rows
// 4w..4w+3 of the step in word w, one byte each) and 4 zero bytes per word:
//   word8(t, ks, c, w)  qt[((t * KS + ks) * 16 + c) * 8 + w]
//   zero word8(t, g, h) zt[(t * G + g) * 4 + h]   (columns 4h..4h+3)
constexpr int TILE_N = 16;

__device__ __forceinline__ int tile_zero(uint32_t zword, int c) {
  return static_cast<int>((zword >> (4 * (c & 7))) & 0xFu);
}

// Zero point of column n from a packed qzeros row, with the v1/v2 convention.
__device__ __forceinline__ int unpack_zero(uint32_t zword, int n, int zero_mode) {
  const int zst = static_cast<int>((zword >> (4 * (n & 7))) & 0xFu);
  return zero_mode == OC_ZERO_V1 ? ((zst + 1) & 0xF) : zst;
}

// ---- RTN dequant (per-op rounding) --------------------------------------------
//
// quant_utils.py:91-103 evaluates (w - z) * s in the compute dtype, each torch
// op rounding its result. Each op is emulated as an fp32 op followed by one
// RNE to DT; for + - * on p-bit operands an intermediate of >= 2p+2 bits makes
// this double rounding harmless (fp32: 24 >= 18 for bf16, 24 >= 24 for fp16).
struct RtnParam {
  float zq;  // RNE_DT(zero)
  float sq;  // RNE_DT(scale)
};

template <int DT>
__device__ __forceinline__ float rtn_value(int code, RtnParam p) {
  const float d = round_to<DT>(static_cast<float>(code) - p.zq);
  return round_to<DT>(d * p.sq);
}

template <int DT>
__device__ __forceinline__ uint4 rtn_dequant8(uint32_t q, RtnParam p) {
  float f[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = rtn_value<DT>(static_cast<int>((q >> (4 * i)) & 0xFu), p);
  uint4 r;
  r.x = pack2<DT>(f[0], f[1]);
  r.y = pack2<DT>(f[2], f[3]);
  r.z = pack2<DT>(f[4], f[5]);
  r.w = pack2<DT>(f[6], f[7]);
  return r;
}

// Exact shortcut of rtn_dequant8 for 16-bit DT. With an integral zero
// |zq| <= 240 and a scale 2^-100 < sq < 2^100: c - zq is an integer of at
// most 8 bits (exact in bf16 and fp16, so the first rounding is the
// identity), (c - zq) sq and zq sq have at most 19 significant bits (exact in
// fp32), so fma(c, sq, -zq sq) is the exact product and the pack rounds it
// once, as the reference's second rounding does. A positive scale also gives
// the same signed zeros (c = zq: +0 either way).
template <int DT>
__device__ __forceinline__ bool rtn_fast_ok(RtnParam p) {
  return p.zq == __builtin_rintf(p.zq) && __builtin_fabsf(p.zq) <= 240.f && p.sq > 0x1p-100f && p.sq < 0x1p100f;
}
template <int DT>
__device__ __forceinline__ uint4 rtn_dequant8_fast(uint32_t q, RtnParam p) {
  const float nzs = -p.zq * p.sq;
  const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;  // codes 0 2 4 6 | 1 3 5 7
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __builtin_fmaf(static_cast<float>((lo >> (8 * i)) & 0xFFu), p.sq, nzs);
    f[2 * i + 1] = __builtin_fmaf(static_cast<float>((hi >> (8 * i)) & 0xFFu), p.sq, nzs);
  }
  return uint4{pack2<DT>(f[0], f[1]), pack2<DT>(f[2], f[3]), pack2<DT>(f[4], f[5]), pack2<DT>(f[6], f[7])};
}

// Codes 0-3 of q (bits 0-15) as rtn_dequant8_fast computes them, with
// nzs = -zq * sq: returns {codes 0|1, codes 2|3}. Applied to q >> 16 it
// yields codes 4-7.
template <int DT>
__device__ __forceinline__ uint2 rtn_fast_half(uint32_t q, float sq, float nzs) {
  const uint32_t lo = q & 0x0F0Fu, hi = (q >> 4) & 0x0F0Fu;  // codes 0 2 | 1 3
  const float f0 = __builtin_fmaf(static_cast<float>(lo & 0xFFu), sq, nzs);
  const float f1 = __builtin_fmaf(static_cast<float>(hi & 0xFFu), sq, nzs);
  const float f2 = __builtin_fmaf(static_cast<float>(lo >> 8), sq, nzs);
  const float f3 = __builtin_fmaf(static_cast<float>(hi >> 8), sq, nzs);
  return uint2{pack2<DT>(f0, f1), pack2<DT>(f2, f3)};
}

// ---- MFMA -----------------------------------------------------------------------
//
// v_mfma_f32_16x16x32_{bf16,f16} operand layout (one wave, lane l):
//   A[16 x 32]: lane l holds row (l % 16), k = 8*(l / 16) + 0..7
//   B[32 x 16]: lane l holds col (l % 16), k = 8*(l / 16) + 0..7
//   D[16 x 16]: lane l holds col (l % 16), rows 4*(l / 16) + 0..3
template <int DT>
__device__ __forceinline__ v4f32 mfma16x16x32(uint4 a, uint4 b, v4f32 acc) {
  if constexpr (DT == OC_DTYPE_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<v8i16>(a), bitcast<v8i16>(b), acc, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<v8f16>(a), bitcast<v8f16>(b), acc, 0, 0, 0);
  }
}

}  // namespace oc
