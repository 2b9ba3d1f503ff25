// Large-M fused int4 GEMM with 256-row wave tiles for gfx950.
//
// Workgroup tile: 256 rows x 64*WN columns, 4 waves (one per SIMD). Each wave
// owns WN 16-column tiles and all 256 rows, so every weight is dequantized
// once per workgroup and feeds 256 rows of MFMA work: per 32-row K step a wave
// issues 16 x WN v_mfma_f32_16x16x32 against WN dequantized B operands and
// holds 64*WN fp32 accumulators per lane. Dequantization (dequant8: exact fp32
// product, one RNE) costs ~20 VALU per weight word against 16 MFMAs per word,
// about a third of the MFMA time, and overlaps it.
//
// Operand flow, one 32-row K step per stage:
//   global -> LDS   buffer DMA (buffer_load ... lds, no registers) into a ring
//                   of NS slots, NS-1 stages ahead: the 256 x 32 activation
//                   block (16 KB, 16-byte chunks swizzled per row), the
//                   workgroup's weight words, scales and zero words;
//   LDS -> VGPRs    one stage ahead of the MFMAs: while the MFMAs of stage s
//                   run from one register set, the wave reads stage s+1's A
//                   fragments and weight words into the other and dequantizes
//                   them.
// One barrier per stage. Every wave issues the same number of DMA instructions
// per stage (lanes and waves without a job read out of the buffer range, which
// returns zero, into a pad), and no other vector memory instruction runs in the
// loop, so "this wave's copies of stage s+1 landed" is a fixed vmcnt.
//
// FMT_RTN (WN = 3): RTN codes re-laid into the same tiles (oc_rtn_tile_prepare)
// with one word per (tile, group, column) holding the 16-bit scale and zero;
// each code is the exact single-rounding value fma(code, sq, -zq sq) (the
// host routes only layers whose every group allows it). FMT_RTN_T (WN = 3):
// the same tiles of a weight whose quant groups run along the output columns
// (ConvTranspose1d, oc_rtn_tile_prepare_t): one word per (tile, K row) holding
// sq | zq << 16, already rounded to DT, so every code of a word has its own
// row's parameters. A K split over grid slices writes fp32 partials
// [split][M][N] for the caller's epilogue.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "oc_gemm_common.h"

namespace oc {

constexpr int WIDE_NS = 4;  // LDS ring depth (stages), default

// One weight/metadata ring slot, in dwords.
//   W: 4*WN tiles x 64 words (tile-major, as in global memory)
//   S: 16-bit scales [tile][16 columns]
//   Z: zero words [tile][2]
//   P: pad destination of jobless DMAs
// DMA jobs per wave and stage (besides the 4 activation DMAs):
//   WN = 4: 16-byte DMA: wave w copies tiles 4w..4w+3 to W + 256w;
//           4-byte DMA: waves 0-1 copy the scales of tiles 8w..8w+7 to S + 64w,
//           wave 2 the zero words to Z (lanes 0-31), wave 3 a pad.
//   WN = 3: 16-byte DMA: waves 0-2 copy tiles 4w..4w+3, wave 3 the scales
//           (lanes 0-23) to S; 4-byte DMA: wave 0 the zero words (lanes 0-23),
//           waves 1-3 a pad.
//   RTN (WN = 3 or 2): 16-byte DMA: waves w < WN copy tiles 4w..4w+3, the
//           others a pad (Z, 1 KB); 4-byte DMA: waves w < WN copy the
//           scale|zero words of tiles 4w..4w+3 to S + 64w (16 words per
//           tile), the others a pad.
//   RTN_T (WN = 3 or 2): the 32 row words of each tile and K step at
//           S + 32 tile: 16-byte DMA: waves w < WN copy tiles 4w..4w+3,
//           wave WN the row words of tiles 0-7, a wave past it a pad (Z,
//           1 KB); 4-byte DMA (WN = 3): waves 0-1 the row words of tiles
//           8+2w, 9+2w, the others (and every wave at WN = 2) a pad.
template <int WN, int FMT = FMT_GPTQ>
struct WideLayout {
  static constexpr int TILES = 4 * WN;
  static constexpr int W = 0;
  static constexpr int S = 256 * WN;
  static constexpr int Z = S + (FMT == FMT_RTN ? 16 * TILES : FMT == FMT_RTN_T ? 32 * TILES : WN == 4 ? 128 : 256);
  static constexpr int P = Z + (FMT == FMT_RTN || FMT == FMT_RTN_T ? 256 : 64);
  static constexpr int DW = P + 64;
};

// Codes 0-3 of q (bits 0-15), code i with its K row's parameter word
// pw[i] = sq | zq << 16 (DT bits): {codes 0|1, codes 2|3}, each
// fma(code, sq, -zq sq) rounded once. Applied to q >> 16 with the next four
// rows' words it yields codes 4-7.
template <int DT>
__device__ __forceinline__ uint2 rtnt_half(uint32_t q, uint4 pw) {
  const uint32_t lo = q & 0x0F0Fu, hi = (q >> 4) & 0x0F0Fu;  // codes 0 2 | 1 3
  const uint32_t w[4] = {pw.x, pw.y, pw.z, pw.w};
  const uint32_t c[4] = {lo & 0xFFu, hi & 0xFFu, lo >> 8, hi >> 8};
  float f[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float sq = half_to_f32<DT>(w[i] & 0xFFFFu);
    f[i] = __builtin_fmaf(static_cast<float>(c[i]), sq, -half_to_f32<DT>(w[i] >> 16) * sq);
  }
  return uint2{pack2<DT>(f[0], f[1]), pack2<DT>(f[2], f[3])};
}

// A buffer offset no resource reaches (reads return zero, no memory access);
// voffset + OOB_OFFSET stays below 2^32 because every voffset is below 2^31.
constexpr uint32_t OOB_OFFSET = 0x80000000u;

template <int DT, int SDT, int WN, int NS, int FMT>
__global__ __launch_bounds__(256, 1) void gemm_wide_kernel(GemmParams p) {
  using L = WideLayout<WN, FMT>;
  constexpr bool RTNT = FMT == FMT_RTN_T;
  constexpr bool RTN = FMT == FMT_RTN || RTNT;  // K slices, fp32 partials, wave 3's 16-byte job
  static_assert(NS == 4 || NS == 6, "ring depth");
  static_assert(FMT == FMT_GPTQ || (RTN && (WN == 3 || WN == 2)), "formats");
  constexpr int BM = 256;
  constexpr int AST = BM * 4;  // uint4 per activation slot
  constexpr int DMA = 6;       // DMA instructions per wave and stage
  static_assert(NS % 2 == 0, "register sets alternate with the ring slots");
  // One distinct LDS array per ring slot (the compiler's wait insertion tells
  // DMA targets apart by array); slots past NS are one element.
  __shared__ __attribute__((aligned(1024))) uint4 A0[AST], A1[AST], A2[AST], A3[AST], A4[NS > 4 ? AST : 1],
      A5[NS > 5 ? AST : 1];
  __shared__ __attribute__((aligned(1024))) uint32_t W0[L::DW], W1[L::DW], W2[L::DW], W3[L::DW],
      W4[NS > 4 ? L::DW : 1], W5[NS > 5 ? L::DW : 1];
  auto slot_a = [&](auto U) -> uint4 * {
    constexpr int u = decltype(U)::value;
    if constexpr (u == 0) return A0;
    else if constexpr (u == 1) return A1;
    else if constexpr (u == 2) return A2;
    else if constexpr (u == 3) return A3;
    else if constexpr (u == 4) return A4;
    else return A5;
  };
  auto slot_w = [&](auto U) -> uint32_t * {
    constexpr int u = decltype(U)::value;
    if constexpr (u == 0) return W0;
    else if constexpr (u == 1) return W1;
    else if constexpr (u == 2) return W2;
    else if constexpr (u == 3) return W3;
    else if constexpr (u == 4) return W4;
    else return W5;
  };

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int quad = lane >> 4, c16 = lane & 15;
  const int nbn = (p.N + 16 * L::TILES - 1) / (16 * L::TILES);
  const int nbm = (p.M + BM - 1) / BM;
  // Workgroups of one K slice (RTN) and row block (they share activation
  // rows) on one XCD.
  const int flat = xcd_block(blockIdx.x, gridDim.x);
  const int zs = RTN ? flat / (nbn * nbm) : 0, fl = flat - zs * (nbn * nbm);
  const int bx = fl % nbn, by = fl / nbn;
  const int t0 = bx * L::TILES;
  const int m0 = by * BM;
  const int tiles = (p.N + TILE_N - 1) / TILE_N;
  const int KS = p.KS;
  const int kb = RTN ? zs * p.ksteps_per_split : 0;              // this slice's first K step
  const int nsteps = RTN ? min(KS - kb, p.ksteps_per_split) : KS;  // and its count (>= 1)

  const __amdgpu_buffer_rsrc_t rs_a = buffer_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rs_q = buffer_rsrc(p.qw, static_cast<int64_t>(tiles) * KS * 256);
  const __amdgpu_buffer_rsrc_t rs_s =
      buffer_rsrc(p.scales, RTNT ? static_cast<int64_t>(tiles) * p.K_phys * 4
                                 : static_cast<int64_t>(tiles) * p.G * (RTN ? 64 : 32));
  const __amdgpu_buffer_rsrc_t rs_z = buffer_rsrc(p.zeros, static_cast<int64_t>(tiles) * p.G * 8);

  // Activation DMA i of wave w fills rows 16 (4w + i) + lane / 4 of the slot,
  // 16-byte position lane % 4, with chunk (position ^ big_swz(row)) of the row.
  // Rows past M re-read row M - 1 (never stored).
  uint32_t avo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int l = 16 * (4 * wave + i) + (lane >> 2);
    const int r = min(m0 + l, p.M - 1);
    avo[i] = static_cast<uint32_t>(static_cast<int64_t>(r) * p.lda * 2 + 16 * ((lane & 3) ^ big_swz(l)));
  }
  // Weight jobs (tiles past N re-read the last tile; never stored).
  auto tile_at = [&](int t) { return min(t0 + t, tiles - 1); };
  __amdgpu_buffer_rsrc_t rs_x, rs_y;
  uint32_t vo_x, vo_y;
  int x_kind, y_kind;  // 0: words, 1: scales, 2: zeros, 3: pad (soffset selector)
  int x_dst, y_dst;    // dword offsets in the slot
  if (RTNT && wave == WN) {
    rs_x = rs_s;
    vo_x = static_cast<uint32_t>(tile_at(lane >> 3)) * p.K_phys * 4 + 16 * (lane & 7);
    x_kind = 5;
    x_dst = L::S;
  } else if (RTN && wave >= WN) {
    rs_x = rs_q;
    vo_x = OOB_OFFSET;
    x_kind = 3;
    x_dst = L::Z;
  } else if (WN == 3 && wave == 3) {
    rs_x = rs_s;
    vo_x = lane < 24 ? static_cast<uint32_t>(tile_at(lane >> 1)) * p.G * 32 + 16 * (lane & 1) : OOB_OFFSET;
    x_kind = 1;
    x_dst = L::S;
  } else {
    rs_x = rs_q;
    vo_x = static_cast<uint32_t>(tile_at(4 * wave + (lane >> 4))) * KS * 256 + 16 * (lane & 15);
    x_kind = 0;
    x_dst = L::W + 256 * wave;
  }
  if (RTNT) {
    const bool job = WN == 3 && wave < 2;
    rs_y = rs_s;
    vo_y = job ? static_cast<uint32_t>(tile_at(8 + 2 * wave + (lane >> 5))) * p.K_phys * 4 + 4 * (lane & 31)
               : OOB_OFFSET;
    y_kind = job ? 5 : 3;
    y_dst = job ? L::S + 256 + 64 * wave : L::P;
  } else if (RTN) {
    rs_y = rs_s;
    vo_y = wave < WN ? static_cast<uint32_t>(tile_at(4 * wave + (lane >> 4))) * p.G * 64 + 4 * (lane & 15)
                     : OOB_OFFSET;
    y_kind = wave < WN ? 4 : 3;
    y_dst = wave < WN ? L::S + 64 * wave : L::P;
  } else if (WN == 4 && wave < 2) {
    rs_y = rs_s;
    vo_y = static_cast<uint32_t>(tile_at(8 * wave + (lane >> 3))) * p.G * 32 + 4 * (lane & 7);
    y_kind = 1;
    y_dst = L::S + 64 * wave;
  } else if ((WN == 4 && wave == 2) || (WN == 3 && wave == 0)) {
    rs_y = rs_z;
    vo_y = lane < 2 * L::TILES ? static_cast<uint32_t>(tile_at(lane >> 1)) * p.G * 8 + 4 * (lane & 1) : OOB_OFFSET;
    y_kind = 2;
    y_dst = L::Z;
  } else {
    rs_y = rs_z;
    vo_y = OOB_OFFSET;
    y_kind = 3;
    y_dst = L::P;
  }
  auto soff = [&](int kind, int ks, int g) -> uint32_t {
    return kind == 0   ? 256u * ks
           : kind == 1 ? 32u * g
           : kind == 2 ? 8u * g
           : kind == 4 ? 64u * g
           : kind == 5 ? 128u * ks
                       : 0u;
  };

  // The copies of K step ks into one slot, one DMA instruction at a time
  // (d = 0-3: activation rows, 4: 16-byte weight job, 5: 4-byte job), so a
  // stage can spread them out. Past the end the activations read as zero
  // (out-of-range offset) and the weights repeat the last step, so the
  // padding steps of the last ring cycle add nothing.
  // ks counts this slice's steps (K step kb + ks).
  auto issue_one = [&](uint4 *as, uint32_t *ws, int ks, int d) {
    const int kk = kb + min(ks, nsteps - 1);
    const int g = kk >> p.gshift;  // the host routes only power-of-two group steps here
    if (d < 4) dma16(rs_a, avo[d], ks < nsteps ? 64u * (kb + ks) : OOB_OFFSET, as + 64 * (4 * wave + d));
    else if (d == 4) dma16(rs_x, vo_x, soff(x_kind, kk, g), ws + x_dst);
    else dma4(rs_y, vo_y, soff(y_kind, kk, g), ws + y_dst);
  };
  auto issue = [&](uint4 *as, uint32_t *ws, int ks) {
#pragma unroll
    for (int d = 0; d < DMA; ++d) issue_one(as, ws, ks, d);
  };

  // Register state: the A fragments of the 16 row tiles (refilled from the
  // next stage right after their MFMAs issue, so each read has a whole stage
  // to land) and two sets of dequantized B operands.
  uint4 a[16], b0[WN], b1[WN];

  // Weight words, scales and zero words of this wave's tiles for one stage
  // (RTN: zw holds the column's scale | zero << 16).
  struct Meta {
    uint32_t q[WN], zw[WN];
    uint16_t sv[WN];
    uint4 pw[RTNT ? WN : 1][2];  // RTN_T: the row words of the lane's 8 K rows per tile
  };
  auto read_meta = [&](const uint32_t *ws) {
    const uint16_t *sb = reinterpret_cast<const uint16_t *>(ws + L::S);
    Meta m;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int tj = WN * wave + j;
      m.q[j] = ws[L::W + tj * 64 + c16 * 4 + quad];
      if constexpr (RTNT) {
        m.zw[j] = 0;
        m.sv[j] = 0;
        m.pw[j][0] = reinterpret_cast<const uint4 *>(ws + L::S + tj * 32 + 8 * quad)[0];
        m.pw[j][1] = reinterpret_cast<const uint4 *>(ws + L::S + tj * 32 + 8 * quad)[1];
      } else if constexpr (RTN) {
        m.zw[j] = ws[L::S + tj * 16 + c16];
        m.sv[j] = 0;
      } else {
        m.sv[j] = sb[tj * 16 + c16];
        m.zw[j] = ws[L::Z + tj * 2 + (c16 >> 3)];
      }
    }
    return m;
  };
  // RTN group parameter: s = RNE_DT(scale), c = -RNE_DT(zero) * s.
  auto rtn_gp = [&](uint32_t w) {
    GroupParam g{};
    g.s = round_to<DT>(scale_f32<SDT>(w & 0xFFFFu));
    g.c = -round_to<DT>(scale_f32<SDT>(w >> 16)) * g.s;
    return g;
  };
  auto dequant1 = [&](const Meta &m, int j) {
    if constexpr (RTNT) {
      const uint2 lo = rtnt_half<DT>(m.q[j], m.pw[j][0]);
      const uint2 hi = rtnt_half<DT>(m.q[j] >> 16, m.pw[j][1]);
      return uint4{lo.x, lo.y, hi.x, hi.y};
    } else if constexpr (RTN) {
      const GroupParam g = rtn_gp(m.zw[j]);
      const uint2 lo = rtn_fast_half<DT>(m.q[j], g.s, g.c), hi = rtn_fast_half<DT>(m.q[j] >> 16, g.s, g.c);
      return uint4{lo.x, lo.y, hi.x, hi.y};
    } else {
      return dequant8<DT>(m.q[j], make_group_param(scale_f32<SDT>(m.sv[j]), tile_zero(m.zw[j], c16)));
    }
  };  // (prologue)
  auto read_a = [&](const uint4 *as, int t) {
    const int row = 16 * t + c16;
    return as[row * 4 + (quad ^ big_swz(row))];
  };

  v4f32 acc[16][WN];
#pragma unroll
  for (int t = 0; t < 16; ++t)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[t][j] = v4f32{0.f, 0.f, 0.f, 0.f};

  // Stage s computes with the A fragments and B set s % 2 read in the
  // previous stage, reads stage s + 1 (slot u + 1) behind its MFMAs and
  // refills slot u (read by every wave before the barrier) with stage s + NS.
  auto step = [&](auto U, int s) {
    constexpr int u = decltype(U)::value;
    constexpr int un = (u + 1) % NS;
    uint4 *as = slot_a(U);
    uint32_t *ws = slot_w(U);
    const uint4 *asn = slot_a(ic<un>{});
    const uint32_t *wsn = slot_w(ic<un>{});
    uint4 *bc = u % 2 == 0 ? b0 : b1;
    uint4 *bn = u % 2 == 0 ? b1 : b0;
    wait_vmcnt<DMA * (NS - 2)>();  // this wave's copies of stage s + 1 landed ...
    barrier_no_fence();            // ... and everyone's; slot u is free
    const Meta m = read_meta(wsn);
    // Row tile t: its WN MFMAs, each followed by a share of the next stage's
    // dequantization, then the refill of a[t]; DMA d of stage s + NS issues in
    // row tile 2d (issued together they queue up behind each other and stall
    // the wave at the top of the stage). The dequantization of tile j
    // runs in three parts (group parameter; codes 0, 1, 4, 5; codes 2, 3, 6,
    // 7) in row tiles 2 + 3j .. 4 + 3j, so VALU work issues while the matrix
    // pipe is busy. Scheduling barriers keep this order (otherwise the reads
    // are hoisted, both stages' fragments are live at once, and the VALU work
    // bunches up between MFMAs).
    GroupParam gp[WN];
    uint2 lo[WN];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
#pragma unroll
      // Weights as the A operand and activations as B: the result tile is
      // C^T, so a lane holds 4 consecutive output columns of one row.
      for (int j = 0; j < WN; ++j) acc[t][j] = mfma16x16x32<DT>(bc[j], a[t], acc[t][j]);
      a[t] = read_a(asn, t);
      if (t % 2 == 0 && t / 2 < DMA) issue_one(as, ws, s + NS, t / 2);
      constexpr int PARTS = 3 * WN;
      const int part = t - 2;
      if (part >= 0 && part < PARTS) {
        const int j = part / 3;
        if constexpr (RTNT) {
          // (the row words arrive with the stage's metadata; part 0 idles)
          if (part % 3 == 1) {
            lo[j] = rtnt_half<DT>(m.q[j], m.pw[j][0]);  // codes 0-3
          } else if (part % 3 == 2) {
            const uint2 hi = rtnt_half<DT>(m.q[j] >> 16, m.pw[j][1]);  // codes 4-7
            bn[j] = uint4{lo[j].x, lo[j].y, hi.x, hi.y};
          }
        } else if constexpr (RTN) {
          if (part % 3 == 0) {
            gp[j] = rtn_gp(m.zw[j]);
          } else if (part % 3 == 1) {
            lo[j] = rtn_fast_half<DT>(m.q[j], gp[j].s, gp[j].c);  // codes 0-3
          } else {
            const uint2 hi = rtn_fast_half<DT>(m.q[j] >> 16, gp[j].s, gp[j].c);  // codes 4-7
            bn[j] = uint4{lo[j].x, lo[j].y, hi.x, hi.y};
          }
        } else if (part % 3 == 0) {
          gp[j] = make_group_param(scale_f32<SDT>(m.sv[j]), tile_zero(m.zw[j], c16));
        } else if (part % 3 == 1) {
          lo[j] = dequant8_half<DT>(m.q[j], gp[j]);
        } else {
          const uint2 hi = dequant8_half<DT>(m.q[j] >> 8, gp[j]);
          bn[j] = uint4{lo[j].x, hi.x, lo[j].y, hi.y};
        }
      }
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // up to three VALU
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // the A refill
      if (t % 2 == 0 && t / 2 < DMA) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // the DMA
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  issue(A0, W0, 0);
  issue(A1, W1, 1);
  issue(A2, W2, 2);
  issue(A3, W3, 3);
  if constexpr (NS > 4) issue(A4, W4, 4);
  if constexpr (NS > 5) issue(A5, W5, 5);
  wait_vmcnt<DMA * (NS - 1)>();
  barrier_no_fence();
  {
    const Meta m = read_meta(W0);
#pragma unroll
    for (int t = 0; t < 16; ++t) a[t] = read_a(A0, t);
#pragma unroll
    for (int j = 0; j < WN; ++j) b0[j] = dequant1(m, j);
  }
  // Whole ring cycles only (no remainder code: it would give the loop's
  // accumulators other registers and cost copies every iteration).
  for (int s0 = 0; s0 < nsteps; s0 += NS) {
    step(ic<0>{}, s0);
    step(ic<1>{}, s0 + 1);
    step(ic<2>{}, s0 + 2);
    step(ic<3>{}, s0 + 3);
    if constexpr (NS > 4) step(ic<4>{}, s0 + 4);
    if constexpr (NS > 5) step(ic<5>{}, s0 + 5);
  }
  wait_vmcnt<0>();  // no DMA outlives the workgroup's LDS

  // Epilogue: acc[t][j][i] = C[m0 + 16t + c16][16 (t0 + WN wave + j) + 4 quad + i]:
  // four consecutive columns per lane, stored as one 8-byte write when the
  // output rows allow it (N is a multiple of 8, so a group of four is either
  // wholly inside N or wholly outside).
  if constexpr (RTN) {
    // fp32 partials of this K slice (N % 4 == 0: 16-byte stores), no bias.
    float *part = p.partials + static_cast<int64_t>(zs) * p.M * p.N;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n0 = TILE_N * (t0 + WN * wave + j) + 4 * quad;
      if (n0 >= p.N) continue;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int r = m0 + 16 * t + c16;
        if (r >= p.M) continue;
        const v4f32 v = acc[t][j];
        *reinterpret_cast<float4 *>(part + static_cast<int64_t>(r) * p.N + n0) = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  } else {
  const bool vec8 = ((reinterpret_cast<uintptr_t>(p.c) | static_cast<uintptr_t>(p.ldc * 2)) & 7) == 0;
  // Every bias value first: loads (behind dtype branches) mixed with the
  // stores made the compiler wait for all memory operations, the previous
  // stores included, before each store (48 serialized stores per wave,
  // ~8 us of an 80 us DiT GEMM).
  float bvs[WN][4];
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int n0 = TILE_N * (t0 + WN * wave + j) + 4 * quad;
#pragma unroll
    for (int i = 0; i < 4; ++i) bvs[j][i] = n0 < p.N ? bias_at(p, n0 + i) : 0.f;
  }
  wait_vmcnt<0>();  // on every path, so no store below waits for memory
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int n0 = TILE_N * (t0 + WN * wave + j) + 4 * quad;
    if (n0 >= p.N) continue;
    const float *bv = bvs[j];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int r = m0 + 16 * t + c16;
      if (r >= p.M) continue;
      const int64_t off = static_cast<int64_t>(r) * p.ldc + n0;
      const v4f32 v = acc[t][j];
      if (vec8) {
        const uint2 pk{pack2<DT>(v[0] + bv[0], v[1] + bv[1]), pack2<DT>(v[2] + bv[2], v[3] + bv[3])};
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p.c) + off) = pk;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) store_c<DT>(p.c, off + i, v[i] + bv[i]);
      }
    }
  }
  }
}

template <int DT, int SDT, int WN>
static void launch_wide_t(const GemmParams &p_in, hipStream_t s) {  // GPTQ: bf16/fp16 output with bias
  // ONECOMP_HIP_WIDE_NS = 6 selects the 6-slot ring (tuning only).
  static const int ns = env_int("ONECOMP_HIP_WIDE_NS", WIDE_NS);
  const GemmParams &p = p_in;
  const int nbn = (p.N + 64 * WN - 1) / (64 * WN), nbm = (p.M + 255) / 256;
  if (ns == 6) hipLaunchKernelGGL((gemm_wide_kernel<DT, SDT, WN, 6, FMT_GPTQ>), dim3(nbn * nbm), dim3(256), 0, s, p);
  else hipLaunchKernelGGL((gemm_wide_kernel<DT, SDT, WN, 4, FMT_GPTQ>), dim3(nbn * nbm), dim3(256), 0, s, p);
}

template <int DT, int SDT>
static void launch_wide_d(const GemmParams &p, int wn, hipStream_t s) {
  if (wn == 3) launch_wide_t<DT, SDT, 3>(p, s);
  else launch_wide_t<DT, SDT, 4>(p, s);
}

// RTN tiles (WN = 3, 4-slot ring) into fp32 partials: p.ksplit slices of
// p.ksteps_per_split K steps each.
template <int DT, int SDT>
static void launch_rtn_wide_t(const GemmParams &p, int wn, hipStream_t s) {
  static const int ns = env_int("ONECOMP_HIP_RTN_WIDE_NS", WIDE_NS);
  const int nbn = (p.N + 64 * wn - 1) / (64 * wn), nbm = (p.M + 255) / 256;
  const dim3 g(nbn * nbm * p.ksplit);
  if (wn == 2) hipLaunchKernelGGL((gemm_wide_kernel<DT, SDT, 2, 4, FMT_RTN>), g, dim3(256), 0, s, p);
  else if (ns == 6) hipLaunchKernelGGL((gemm_wide_kernel<DT, SDT, 3, 6, FMT_RTN>), g, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((gemm_wide_kernel<DT, SDT, 3, 4, FMT_RTN>), g, dim3(256), 0, s, p);
}

template <int DT>
static void launch_rtnt_wide_t(const GemmParams &p, int wn, hipStream_t s) {
  static const int ns = env_int("ONECOMP_HIP_RTN_WIDE_NS", WIDE_NS);
  const int nbn = (p.N + 64 * wn - 1) / (64 * wn), nbm = (p.M + 255) / 256;
  const dim3 g(nbn * nbm * p.ksplit);
  if (wn == 2) hipLaunchKernelGGL((gemm_wide_kernel<DT, DT, 2, 4, FMT_RTN_T>), g, dim3(256), 0, s, p);
  else if (ns == 6) hipLaunchKernelGGL((gemm_wide_kernel<DT, DT, 3, 6, FMT_RTN_T>), g, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((gemm_wide_kernel<DT, DT, 3, 4, FMT_RTN_T>), g, dim3(256), 0, s, p);
}

void launch_rtnt_wide(const GemmParams &p, int a_dtype, int wn, hipStream_t s) {
  if (a_dtype == OC_DTYPE_BF16) launch_rtnt_wide_t<OC_DTYPE_BF16>(p, wn, s);
  else launch_rtnt_wide_t<OC_DTYPE_F16>(p, wn, s);
}

void launch_rtn_wide(const GemmParams &p, int a_dtype, int scale_dtype, int wn, hipStream_t s) {
  const bool bf = a_dtype == OC_DTYPE_BF16, sbf = scale_dtype == OC_DTYPE_BF16;
  if (bf && sbf) launch_rtn_wide_t<OC_DTYPE_BF16, OC_DTYPE_BF16>(p, wn, s);
  else if (bf) launch_rtn_wide_t<OC_DTYPE_BF16, OC_DTYPE_F16>(p, wn, s);
  else if (sbf) launch_rtn_wide_t<OC_DTYPE_F16, OC_DTYPE_BF16>(p, wn, s);
  else launch_rtn_wide_t<OC_DTYPE_F16, OC_DTYPE_F16>(p, wn, s);
}

void launch_gptq_wide(const GemmParams &p, int a_dtype, int scale_dtype, int wn, hipStream_t s) {
  const bool bf = a_dtype == OC_DTYPE_BF16, sbf = scale_dtype == OC_DTYPE_BF16;
  if (bf && sbf) launch_wide_d<OC_DTYPE_BF16, OC_DTYPE_BF16>(p, wn, s);
  else if (bf) launch_wide_d<OC_DTYPE_BF16, OC_DTYPE_F16>(p, wn, s);
  else if (sbf) launch_wide_d<OC_DTYPE_F16, OC_DTYPE_BF16>(p, wn, s);
  else launch_wide_d<OC_DTYPE_F16, OC_DTYPE_F16>(p, wn, s);
}

}  // namespace oc
