// Fused int4 dequant + GEMM kernels for gfx950 and their host dispatch.
//
// GPTQ weights are read in the tiled layout built by oc_int4_prepare (tile16,
// oc_device.h): every wave instruction streams 1 KB of consecutive bytes and
// a lane receives whole 32-row groups of a column. Three regimes:
//  * decode (M <= 2): VALU dot products with the scale/zero factored out of
//    each 32-row group (v_dot2_f32_{bf16,f16}); HBM-bound by construction.
//  * small M (M <= 64): v_mfma_f32_16x16x32 with one lane load feeding four
//    MFMAs (the four 8-row octets of a group); K is split over the waves of a
//    workgroup, which owns one 16-column tile (no cross-workgroup results).
//  * large M: LDS-tiled MFMA GEMM; the activation tile of each 32-row step is
//    shared through LDS by 4 waves that split the columns, and each wave
//    dequantizes only its own columns once per step.
// The MFMA regimes dequantize with dequant8() (exact fp32 product, one RNE to
// the activation type). Act-order / padded-group layers gather activations
// into physical row order first (decode does it while staging into LDS).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <type_traits>
#include <cstdlib>

#include "oc_gemm_common.h"

namespace oc {


// ---------------------------------------------------------------------------
// Decode kernel (M <= 2). grid = tiles, 64*WAVES threads. Lane (c = l%16,
// h = l/16) of wave w owns column 16t + c and the K steps lp, lp + NPH, ...
// (lp = 4w + h, NPH = 4*WAVES phases), so each wave instruction reads four
// consecutive K steps of the tile (1 KB).
//
// The scale and zero are factored out of each 32-row group:
//   sum_k x_k * s * (w_k - z) = s * (sum_k x_k * (B + w_k) - (B + z) * sum_k x_k)
// where B + w_k is the exact 16-bit number made by OR-ing the 4-bit code into
// the mantissa of B (bf16 128.0 / fp16 1024.0). The first sum runs on
// v_dot2_f32_{bf16,f16} (fp32 accumulation) against activation pairs held in
// LDS, interleaved to match the code pairs (i, i+4) of a packed word; the
// second uses per-step activation sums staged beside them.
//
// Activation staging ("x-pairs", in LDS): for row m and K step ks, 4 uint4
// of pairs (one per 8-row octet w: {x0|x4<<16, x1|x5<<16, x2|x6<<16,
// x3|x7<<16}) and a float2 (sum, B * sum): pairs [MR][KS][4] uint4, then sums
// [MR][KSP] float2 (KSP = KS rounded up to even).
//
// Act-order / padded layers read their activation rows contiguously and
// scatter each value to its physical row through kinv (logical -> physical),
// so every global access of the staging stays coalesced; a per-workgroup
// gather through kmap would touch one cache line per lane.
constexpr int DOT_PF = 2;  // K steps in flight per lane (measured: 2 beats 3-5; fewer registers, more waves)

// How the decode kernel stages its activations: contiguous rows, or rows
// scattered to their physical positions through kinv (act-order / padded).
enum { XS_CONTIG = 0, XS_SCATTER = 1 };

__host__ __device__ inline int dot_ksp(int KS) { return (KS + 1) & ~1; }
size_t dot_lds_bytes(int MR, int KS) {
  return static_cast<size_t>(MR) * (KS * 4 * sizeof(uint4) + dot_ksp(KS) * sizeof(float2));
}

template <int DT, int SDT, int MR, int XS, int WAVES, int CPW>
__global__ __launch_bounds__(64 * WAVES) void gemv_dot_kernel(GemmParams p) {
  // CPW columns per workgroup: a whole tile (16) or half of one (8; each K
  // step's half is one 128-byte line), which doubles the workgroups of
  // narrow layers. 16-byte activation words are staged SB per thread per
  // round trip (registers beyond the main loop's would cost occupancy).
  constexpr int SB = XS == XS_CONTIG ? 4 : 2;
  constexpr int NT = 64 * WAVES;
  constexpr int PPW = 64 / CPW;     // K-step phases per wave
  constexpr int NPH = PPW * WAVES;  // K-step phases per workgroup
  constexpr int SPLIT = TILE_N / CPW;
  constexpr uint32_t MAGIC = DT == OC_DTYPE_BF16 ? 0x43004300u : 0x64006400u;
  extern __shared__ __attribute__((aligned(16))) uint4 dot_lds[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int cl = lane % CPW, h = lane / CPW;
  const int lp = PPW * wave + h;
  const int blk = xcd_block(blockIdx.x, gridDim.x);
  const int t = blk / SPLIT;
  const int c = CPW * (blk % SPLIT) + cl;  // column within the tile
  const int n = TILE_N * t + c;
  const int KS = p.KS, M = p.M;
  const int ks_end = KS;
  const int KSP = (KS + 1) & ~1;
  uint4 *xpairs = dot_lds;                                          // [MR][KS * 4]
  float2 *xsum = reinterpret_cast<float2 *>(dot_lds + MR * KS * 4);  // [MR][KSP]: (sum, B * sum)
  const uint4 *qt4 = static_cast<const uint4 *>(p.qw) + static_cast<int64_t>(t) * KS * TILE_N + c;
  const uint16_t *stp = static_cast<const uint16_t *>(p.scales) + static_cast<int64_t>(t) * p.G * TILE_N + c;
  const uint32_t *ztp = static_cast<const uint32_t *>(p.zeros) + static_cast<int64_t>(t) * p.G * 2 + (c >> 3);

  struct Stage {
    uint4 q;
    uint32_t s;
    uint32_t z;
  };
  Stage st[DOT_PF];
  auto load = [&](Stage &S, int ks) {
    // Default cache policy: non-temporal loads (CPOL_WEIGHT_STREAM) made
    // this kernel slower (K=5120 N=1024 M=1: 4.3 -> 5.1 us).
    S.q = qt4[ks * TILE_N];
    const int g = ks >> p.gshift;
    S.s = stp[g * TILE_N];
    S.z = ztp[g * 2];
  };
  // Prefetches past the end re-read the last step (no branch around loads).
  const int ks_last = max(ks_end - 1, 0);
  // The head of the weight stream is in flight while activations stage.
#pragma unroll
  for (int f = 0; f < DOT_PF; ++f) load(st[f], min(lp + NPH * f, ks_last));

  const uint16_t *a = static_cast<const uint16_t *>(p.a);
  if constexpr (XS == XS_CONTIG) {
    // One thread per octet (8 physical rows = 8 logical rows); the 4 octets
    // of a K step sit in 4 consecutive lanes, which add up the step's sum.
    const int per_row = KS * 4;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const uint4 *arow = reinterpret_cast<const uint4 *>(a + static_cast<int64_t>(m) * p.lda);
      for (int base = 0; base < per_row; base += NT * SB) {
        uint4 raw[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u)  // clamped, not guarded: a branch around a load waits for it
          raw[u] = arow[min(base + NT * u + tid, per_row - 1)];
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const int i = base + NT * u + tid;
          float sum;
          const uint4 pr = octet_pairs<DT>(raw[u], sum);
          sum += __shfl_xor(sum, 1);
          sum += __shfl_xor(sum, 2);
          if (i < per_row) {
            xpairs[m * per_row + i] = pr;
            if ((i & 3) == 0) xsum[m * KSP + (i >> 2)] = make_float2(sum, dot_base<DT>() * sum);
          }
        }
      }
    }
  } else {
    uint16_t *x16 = reinterpret_cast<uint16_t *>(xpairs);
    const int K = p.K_logical, K_phys = p.K_phys;
    if (K != K_phys) {  // physical rows without a source stay zero
      for (int i = tid; i < MR * KS * 4; i += NT) xpairs[i] = make_uint4(0, 0, 0, 0);
      __syncthreads();
    }
    // Logical octets: 8 activations and their 8 physical rows (one 16-byte
    // load each); the K % 8 tail rows one by one.
    const int octets = K >> 3;
    const uint4 *kinv4 = reinterpret_cast<const uint4 *>(p.kinv);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const uint16_t *arow = a + static_cast<int64_t>(m) * p.lda;
      for (int base = 0; base < octets; base += NT * SB) {
        uint4 xv[SB], rv[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u) {  // clamped loads (the stores below are guarded)
          const int i = min(base + NT * u + tid, octets - 1);
          xv[u] = reinterpret_cast<const uint4 *>(arow)[i];
          rv[u] = kinv4[i];
        }
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const int i = base + NT * u + tid;
          if (i < octets) {
            const uint32_t xw[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
            const uint32_t rw[4] = {rv[u].x, rv[u].y, rv[u].z, rv[u].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int r0 = static_cast<int>(rw[j] & 0xFFFFu), r1 = static_cast<int>(rw[j] >> 16);
              if (r0 < K_phys) x16[xpair_slot(m, K_phys, r0)] = static_cast<uint16_t>(xw[j]);
              if (r1 < K_phys) x16[xpair_slot(m, K_phys, r1)] = static_cast<uint16_t>(xw[j] >> 16);
            }
          }
        }
      }
      for (int k = 8 * octets + tid; k < K; k += NT) {
        const int r = p.kinv[k];
        if (r < K_phys) x16[xpair_slot(m, K_phys, r)] = arow[k];
      }
    }
    __syncthreads();
    // Step sums from the staged pairs (dot2 against 1.0 pairs).
    const uint32_t ones = DT == OC_DTYPE_BF16 ? 0x3F803F80u : 0x3C003C00u;
    for (int i = tid; i < MR * KS; i += NT) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint4 pr = xpairs[4 * i + w];
        sum = dot2acc<DT>(pr.x, ones, sum);
        sum = dot2acc<DT>(pr.y, ones, sum);
        sum = dot2acc<DT>(pr.z, ones, sum);
        sum = dot2acc<DT>(pr.w, ones, sum);
      }
      const int m = i / KS, ks = i - m * KS;
      xsum[m * KSP + ks] = make_float2(sum, dot_base<DT>() * sum);
    }
  }
  __syncthreads();

  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.f;
  const uint32_t magic = MAGIC;
  // This lane's K steps lp, lp + NPH, ..., padded to whole rounds of DOT_PF
  // (the padding re-reads the last step and adds nothing); each stage is
  // consumed and then refilled in place.
  const int nks = lp < ks_end ? (ks_end - lp + NPH - 1) / NPH : 0;
  const int nks_pad = (nks + DOT_PF - 1) / DOT_PF * DOT_PF;
  for (int i0 = 0; i0 < nks_pad; i0 += DOT_PF) {
#pragma unroll
    for (int f = 0; f < DOT_PF; ++f) {
      const bool valid = i0 + f < nks;
      const int ks = min(lp + NPH * (i0 + f), ks_last);
      Stage &cur = st[f];
      // Two partial sums per row (words 0-1 and 2-3) shorten the dot2 chain.
      float d[MR][2];
#pragma unroll
      for (int m = 0; m < MR; ++m) d[m][0] = d[m][1] = 0.f;
      const uint32_t qs[4] = {cur.q.x, cur.q.y, cur.q.z, cur.q.w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t q = qs[w];
        const uint32_t b0 = and_or(q, 0x000F000Fu, magic);
        const uint32_t b1 = and_or(q >> 4, 0x000F000Fu, magic);
        const uint32_t b2 = and_or(q >> 8, 0x000F000Fu, magic);
        const uint32_t b3 = and_or(q >> 12, 0x000F000Fu, magic);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const uint4 xp = xpairs[(m * KS + ks) * 4 + w];
          float &dd = d[m][w >> 1];
          dd = dot2acc<DT>(b0, xp.x, dd);
          dd = dot2acc<DT>(b1, xp.y, dd);
          dd = dot2acc<DT>(b2, xp.z, dd);
          dd = dot2acc<DT>(b3, xp.w, dd);
        }
      }
      const float zf = static_cast<float>(tile_zero(cur.z, c));
      const float s = scale_f32<SDT>(cur.s);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float2 xs = xsum[m * KSP + ks];
        const float v = __builtin_fmaf(s, __builtin_fmaf(-zf, xs.x, (d[m][0] + d[m][1]) - xs.y), acc[m]);
        acc[m] = valid ? v : acc[m];
      }
      load(cur, min(lp + NPH * (i0 + f + DOT_PF), ks_last));
    }
  }

  // Phases h of one wave (xor CPW .. 32), then the waves through LDS in order.
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int off = CPW; off < 64; off <<= 1) acc[m] += __shfl_xor(acc[m], off);
  __syncthreads();
  float(*red)[MR][CPW] = reinterpret_cast<float(*)[MR][CPW]>(dot_lds);
  if (h == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) red[wave][m][cl] = acc[m];
  }
  __syncthreads();
  if (wave != 0 || h != 0 || n >= p.N) return;
  const float bv = bias_at(p, n);
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m >= M) break;
    float v = red[0][m][cl];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) v += red[w][m][cl];
    store_c<DT>(p.c, static_cast<int64_t>(m) * p.ldc + n, v + bv);
  }
}

// ---------------------------------------------------------------------------
// Small-M MFMA kernel (M <= 64). grid = tiles, 256 threads; wave w takes the
// quad-steps (4 K steps) w, w+4, ... of the tile. Lane (quad = l/16, c16 =
// l%16) loads the 4 words of column c16 for K step 4*qs + quad (one 16-byte
// load; the wave reads 1 KB of consecutive bytes) and feeds MFMA j with word
// j: MFMA j's K dimension runs over octet j of the 4 K steps, and the A
// operand of lane (quad, r) is x[r, 32*(4qs + quad) + 8j .. +7] to match. One
// group parameter per lane covers 32 weights.
template <int DT, int SDT, int MT, int NW, int PF>
__global__ __launch_bounds__(64 * NW) void gemv_mfma_kernel(GemmParams p) {
  // NW waves split the tile's K; PF quad-steps in flight per wave (weights
  // and the matching activations travel together: the activations are L2
  // hits, but only as early as the weights can they hide their latency).
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int quad = lane >> 4, c16 = lane & 15;
  const int t = xcd_block(blockIdx.x, gridDim.x);
  const int n = TILE_N * t + c16;
  const int KS = p.KS, M = p.M;
  const int QS = (KS + 3) / 4;
  // Branch-free buffer loads (a branch around a load made the compiler wait
  // for it before issuing the next): steps past KS and rows past M read an
  // offset beyond every buffer, which returns zeros without a memory access;
  // zero codes, scales and activations then add exactly zero.
  const int tiles = (p.N + TILE_N - 1) / TILE_N;
  const __amdgpu_buffer_rsrc_t q_rs = buffer_rsrc(p.qw, static_cast<int64_t>(tiles) * KS * 256);
  const __amdgpu_buffer_rsrc_t s_rs = buffer_rsrc(p.scales, static_cast<int64_t>(tiles) * p.G * 32);
  const __amdgpu_buffer_rsrc_t z_rs = buffer_rsrc(p.zeros, static_cast<int64_t>(tiles) * p.G * 8);
  const __amdgpu_buffer_rsrc_t a_rs = buffer_rsrc(p.a, p.a_bytes);  // host: a_bytes < 2^31
  constexpr uint32_t NOWHERE = 0xFFFFF000u;
  const uint32_t q_base = (static_cast<uint32_t>(t) * KS * TILE_N + c16) * 16u;  // + 256 ks
  const uint32_t s_base = (static_cast<uint32_t>(t) * p.G * TILE_N + c16) * 2u;  // + 32 g
  const uint32_t z_base = (static_cast<uint32_t>(t) * p.G * 2 + (c16 >> 3)) * 4u;  // + 8 g
  uint32_t a_row[MT];  // byte offset of activation row 16 tt + c16, NOWHERE past M
#pragma unroll
  for (int tt = 0; tt < MT; ++tt) {
    const int row = 16 * tt + c16;
    a_row[tt] = row < M ? static_cast<uint32_t>(row * p.lda * 2) : NOWHERE;
  }

  struct Stage {
    uint4 q;
    uint32_t s;
    uint32_t z;
    uint32_t x[MT][16];  // 4 chunks of 16 bytes per row tile (flat: stays in registers)
  };
  Stage st[PF];
  auto load = [&](Stage &S, int qs) __attribute__((always_inline)) {
    const int ks = 4 * qs + quad;
    const bool kin = ks < KS;
    const uint32_t g = static_cast<uint32_t>(group_of(p, kin ? ks : 0));
    const auto q = __builtin_amdgcn_raw_buffer_load_b128(q_rs, kin ? q_base + 256u * ks : NOWHERE, 0,CPOL_WEIGHT_STREAM);
    S.q = make_uint4(q[0], q[1], q[2], q[3]);
    S.s = __builtin_amdgcn_raw_buffer_load_b16(s_rs, kin ? s_base + 32u * g : NOWHERE, 0,CPOL_WEIGHT_STREAM);
    S.z = __builtin_amdgcn_raw_buffer_load_b32(z_rs, kin ? z_base + 8u * g : NOWHERE, 0,CPOL_WEIGHT_STREAM);
#pragma unroll
    for (int tt = 0; tt < MT; ++tt) {
      const uint32_t off = kin && a_row[tt] != NOWHERE ? a_row[tt] + 64u * ks : NOWHERE;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(a_rs, off == NOWHERE ? NOWHERE : off + 16u * j, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) S.x[tt][4 * j + e] = v[e];
      }
    }
  };
  // Quad-steps of this wave: wave, wave + NW, ...; the count is padded to
  // whole rounds of PF (the padding reads zeros).
  const int nq = wave < QS ? (QS - wave + NW - 1) / NW : 0;
  const int nq_pad = (nq + PF - 1) / PF * PF;
  static_for<0, PF>([&](auto F) __attribute__((always_inline)) {
    load(st[F], wave + NW * F);
    __builtin_amdgcn_sched_barrier(0);
  });
  v4f32 acc[MT];
#pragma unroll
  for (int tt = 0; tt < MT; ++tt) acc[tt] = v4f32{0.f, 0.f, 0.f, 0.f};

  for (int i0 = 0; i0 < nq_pad; i0 += PF) {
    static_for<0, PF>([&](auto F) __attribute__((always_inline)) {
      Stage &cur = st[F];  // consumed, then refilled in place
      const GroupParam gp = make_group_param(scale_f32<SDT>(cur.s), tile_zero(cur.z, c16));
      const uint32_t qwords[4] = {cur.q.x, cur.q.y, cur.q.z, cur.q.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 b = dequant8<DT>(qwords[j], gp);
#pragma unroll
        for (int tt = 0; tt < MT; ++tt) {
          const uint4 xa = make_uint4(cur.x[tt][4 * j], cur.x[tt][4 * j + 1], cur.x[tt][4 * j + 2], cur.x[tt][4 * j + 3]);
          acc[tt] = mfma16x16x32<DT>(xa, b, acc[tt]);
        }
      }
      load(cur, wave + NW * (i0 + F + PF));
    });
  }

  // acc[tt][i] = row 16tt + 4*quad + i, column c16. Waves 1.. park their sums
  // in LDS behind one barrier; wave 0 adds them in wave order.
  __shared__ float red[NW - 1][MT * 16][TILE_N + 1];
  if (wave > 0) {
#pragma unroll
    for (int tt = 0; tt < MT; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave - 1][16 * tt + 4 * quad + i][c16] = acc[tt][i];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < NW - 1; ++w)
#pragma unroll
      for (int tt = 0; tt < MT; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[tt][i] += red[w][16 * tt + 4 * quad + i][c16];
  }
  if (wave != 0 || n >= p.N) return;
  const float bv = bias_at(p, n);
  wait_vmcnt<0>();  // the bias is in on every path: the stores below wait for nothing
#pragma unroll
  for (int tt = 0; tt < MT; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * tt + 4 * quad + i;
      if (row < M) store_c<DT>(p.c, static_cast<int64_t>(row) * p.ldc + n, acc[tt][i] + bv);
    }
}

// ---------------------------------------------------------------------------
// Weight access of the large-M kernel, per format.
template <int FMT>
__device__ __forceinline__ uint32_t load_word(const GemmParams &p, const void *qw, int tile, int ks, int quad,
                                              int c16) {
  if constexpr (FMT == FMT_GPTQ) {
    return static_cast<const uint32_t *>(qw)[((static_cast<int64_t>(tile) * p.KS + ks) * TILE_N + c16) * 4 + quad];
  } else {
    // Clamped like the RTN scale/zero rows: with N % 16 == 8 the upper lanes
    // of the last tile name rows past the weight (their results are unused).
    const int n = min(TILE_N * tile + c16, p.N - 1);
    const uint8_t *row = static_cast<const uint8_t *>(qw) + static_cast<int64_t>(n) * p.row_bytes;
    if constexpr (FMT == FMT_DSV4_2)  // 8 two-bit codes: 2 bytes
      return *reinterpret_cast<const uint16_t *>(row + 8 * ks + 2 * quad);
    else
      return *reinterpret_cast<const uint32_t *>(row + 16 * ks + 4 * quad);
  }
}

template <int DT>
__device__ __forceinline__ RtnParam rtn_param(const GemmParams &p, int g, int n) {
  const int64_t i = static_cast<int64_t>(n) * p.rtn_G + g;
  RtnParam r;
  r.zq = round_to<DT>(load_any_f32(p.zeros, i, p.zero_dtype));
  r.sq = round_to<DT>(load_any_f32(p.scales, i, p.scale_dtype));
  return r;
}

// Sum of the split-K partials in split order, plus bias, rounded once. A
// thread adds 4 adjacent outputs (N % 8 == 0 keeps them in one row); the
// partials of up to 8 splits are loaded together before the in-order sum.
// Partials are written once and read once, both non-temporally (padded
// gs26 M=256 K=1040 N=3072: 19.6 -> 18.7 us).
constexpr int REDUCE_UNROLL = 8;
template <int DT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmParams p) {
  const int64_t MN = static_cast<int64_t>(p.M) * p.N;
  const int64_t idx = 4 * (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x);
  if (idx >= MN) return;
  const int n = static_cast<int>(idx % p.N);
  const int row = static_cast<int>(idx / p.N);
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < p.ksplit; s0 += REDUCE_UNROLL) {
    float4 t[REDUCE_UNROLL];
#pragma unroll
    for (int j = 0; j < REDUCE_UNROLL; ++j) {  // clamped, not guarded: the loads go out together
      using f32x4 = __attribute__((ext_vector_type(4))) float;
      const f32x4 v = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4 *>(p.partials + min(s0 + j, p.ksplit - 1) * MN + idx));
      t[j] = make_float4(v[0], v[1], v[2], v[3]);
    }
#pragma unroll
    for (int j = 0; j < REDUCE_UNROLL; ++j) {
      if (s0 + j >= p.ksplit) break;
      v.x += t[j].x;
      v.y += t[j].y;
      v.z += t[j].z;
      v.w += t[j].w;
    }
  }
  const int64_t o = static_cast<int64_t>(row) * p.ldc + n;
  const float b0 = bias_at(p, n), b1 = bias_at(p, n + 1), b2 = bias_at(p, n + 2), b3 = bias_at(p, n + 3);
  wait_vmcnt<0>();  // every bias in before the first store
  store_c<DT>(p.c, o, v.x + b0);
  store_c<DT>(p.c, o + 1, v.y + b1);
  store_c<DT>(p.c, o + 2, v.z + b2);
  store_c<DT>(p.c, o + 3, v.w + b3);
}

// ---------------------------------------------------------------------------
// LDS-tiled kernel. BM = 16*WM rows, BN = 64*WN columns (4 waves x WN tiles),
// KG groups of 4 waves per workgroup splitting the workgroup's K steps into
// contiguous parts (each group its own LDS tiles; the groups' sums are added
// in group order at the end). One wave per SIMD leaves every latency of a
// step exposed; KG = 4 puts four independent steps on each SIMD.
// grid = (ceil(N/BN), ceil(M/BM), ksplit), 256 KG threads.
constexpr int A_LDS_STRIDE = 40;  // halves per LDS row: 32 data + 8 pad (80 B)

// RDT (RTN): the dtype of both scales and zeros when they share a 16-bit one
// (raw loads, converted at use), else 0 (any dtypes, converted as loaded).
template <int DT, int SDT, int WM, int WN, int FMT, int RDT, int KG>
__global__ __launch_bounds__(256 * KG) void gemm_tiled_kernel(GemmParams p) {
  // PF K steps in flight in registers (activation chunks, weight words and
  // group parameters of each step); the activation tile of the next step is
  // written to the other LDS buffer once its loads are in, and the step ends
  // with an LDS-only barrier, so the loads of later steps stay in flight.
  // Loads of steps past the range and of rows / columns past the matrix read
  // clamped (valid) addresses; their results are never used or stored.
  constexpr int BM = 16 * WM;
  constexpr int BN = 64 * WN;
  constexpr int PF = 2;  // measured on RTN M=512: 2 beats 4 and 8
  __shared__ __attribute__((aligned(16))) uint16_t As_all[KG][2][BM * A_LDS_STRIDE];
  const int tid = threadIdx.x & 255, grp = threadIdx.x >> 8;  // thread within its K group, the group
  auto &As = As_all[grp];
  const int wave = tid >> 6, lane = tid & 63;
  const int quad = lane >> 4, c16 = lane & 15;
  // The column blocks of one row block on one XCD (they share its activation
  // rows in that XCD's L2).
  const int blk = xcd_block(blockIdx.y * gridDim.x + blockIdx.x, gridDim.x * gridDim.y);
  const int bxx = blk % gridDim.x, byy = blk / gridDim.x;
  const int n0 = bxx * BN;
  const int tw = n0 / TILE_N + wave * WN;  // first tile of this wave
  const int last_tile = (p.N - 1) / TILE_N;
  const uint16_t *a = static_cast<const uint16_t *>(p.a);
  const int m0 = byy * BM;
  const int wg_begin = blockIdx.z * p.ksteps_per_split;
  const int wg_end = min(wg_begin + p.ksteps_per_split, p.KS);
  const int part = (max(wg_end - wg_begin, 0) + KG - 1) / KG;  // steps per K group (the last may have fewer)
  const int ks_begin = wg_begin + grp * part;
  const int ks_end = min(ks_begin + part, wg_end);
  const int nsteps = max(ks_end - ks_begin, 0);

  constexpr int A_CHUNKS = BM * 4;  // 16-byte chunks of an activation tile (a multiple of 256)
  constexpr int A_PER_THREAD = A_CHUNKS / 256;
  // Addressing: a uniform base per step (scalar registers) plus a lane
  // offset fixed for the kernel (32 bits), so a step's loads cost no vector
  // address arithmetic (64-bit per-lane index math per step measured ~300 of
  // ~1200 cycles per step on RTN M=512).
  const char *a_blk = reinterpret_cast<const char *>(a + static_cast<int64_t>(m0) * p.lda);
  uint32_t a_off[A_PER_THREAD];
#pragma unroll
  for (int i = 0; i < A_PER_THREAD; ++i) {
    const int ch = tid + 256 * i;
    a_off[i] = static_cast<uint32_t>((min(m0 + (ch >> 2), p.M - 1) - m0) * p.lda * 2 + 16 * (ch & 3));
  }
  // Weight, scale and zero lane offsets per column tile j (bytes; RTN scale
  // and zero ones in elements), and the tile's first 16-column tile.
  constexpr bool ROWS = fmt_rows(FMT);  // RTN / DSV4: one byte row per output column
  uint32_t q_off[WN], s_off[WN], z_off[WN];
  int tl_of[WN];
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int tl = min(tw + j, last_tile);
    tl_of[j] = tl;
    // Clamped like the RTN scale/zero rows: with N % 16 == 8 the upper lanes
    // of the last tile name rows past the weight (their results are unused).
    const int n = min(TILE_N * tl + c16, p.N - 1);
    if constexpr (FMT == FMT_GPTQ) {
      q_off[j] = static_cast<uint32_t>(c16 * 16 + quad * 4);
      s_off[j] = static_cast<uint32_t>(c16 * 2);
      z_off[j] = static_cast<uint32_t>((c16 >> 3) * 4);
    } else if constexpr (FMT == FMT_GPTQ8) {
      q_off[j] = static_cast<uint32_t>(c16 * 32 + quad * 8);
      s_off[j] = static_cast<uint32_t>(c16 * 2);
      z_off[j] = static_cast<uint32_t>((c16 >> 2) * 4);
    } else if constexpr (FMT == FMT_RTN_T) {
      q_off[j] = static_cast<uint32_t>(n * p.row_bytes + 4 * quad);
      s_off[j] = static_cast<uint32_t>((n / p.rtn_gs) * p.K_logical + 8 * quad);  // elements
      z_off[j] = s_off[j];
    } else {
      q_off[j] = static_cast<uint32_t>(n * p.row_bytes + (FMT == FMT_DSV4_2 ? 2 : 4) * quad);
      s_off[j] = static_cast<uint32_t>(n * p.sz_stride_n);  // elements
      z_off[j] = s_off[j];
    }
  }
  // Stage registers: per step in flight, the activation chunks, weight
  // words and group parameters (GPTQ: scale bits and zero word; RTN: scale
  // and zero as RDT bits, or as fp32 bits). Separate arrays indexed by
  // compile-time stage numbers stay in registers.
  uint32_t sa[PF][A_PER_THREAD * 4];
  uint32_t sq[PF][WN], ss[PF][WN], sz[PF][WN];
  uint32_t sq8[PF][WN];  // 8-bit: the second word of the lane's 8 codes
  uint32_t sst[PF][WN][4], szt[PF][WN][4];  // RTN_T: the 8 K rows' scales / zeros (16-bit pairs)
  const char *qb = static_cast<const char *>(p.qw);
  const char *sb = static_cast<const char *>(p.scales);
  const char *zb = static_cast<const char *>(p.zeros);
  auto load = [&](auto fc, int ks) __attribute__((always_inline)) {
    constexpr int f = decltype(fc)::value;
    ks = min(ks, max(ks_end - 1, 0));
    const char *ab = a_blk + 64 * static_cast<int64_t>(ks);
#pragma unroll
    for (int i = 0; i < A_PER_THREAD; ++i) {
      const uint4 v = *reinterpret_cast<const uint4 *>(ab + a_off[i]);
      sa[f][4 * i] = v.x;
      sa[f][4 * i + 1] = v.y;
      sa[f][4 * i + 2] = v.z;
      sa[f][4 * i + 3] = v.w;
    }
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int tl = tl_of[j];
      if constexpr (FMT == FMT_GPTQ8) {
        // Codes of K rows 8 quad .. 8 quad + 7: words 2 quad, 2 quad + 1.
        const uint2 v = *reinterpret_cast<const uint2 *>(qb + (static_cast<int64_t>(tl) * p.KS + ks) * 512 + q_off[j]);
        sq[f][j] = v.x;
        sq8[f][j] = v.y;
        const int64_t tgs = static_cast<int64_t>(tl) * p.G + group_of(p, ks);
        ss[f][j] = *reinterpret_cast<const uint16_t *>(sb + tgs * 32 + s_off[j]);
        sz[f][j] = *reinterpret_cast<const uint32_t *>(zb + tgs * 16 + z_off[j]);
      } else if constexpr (FMT == FMT_GPTQ) {
        sq[f][j] = *reinterpret_cast<const uint32_t *>(qb + (static_cast<int64_t>(tl) * p.KS + ks) * 256 + q_off[j]);
        const int64_t tgs = static_cast<int64_t>(tl) * p.G + group_of(p, ks);
        ss[f][j] = *reinterpret_cast<const uint16_t *>(sb + tgs * 32 + s_off[j]);
        sz[f][j] = *reinterpret_cast<const uint32_t *>(zb + tgs * 8 + z_off[j]);
      } else if constexpr (FMT == FMT_RTN_T) {
        sq[f][j] = *reinterpret_cast<const uint32_t *>(qb + 16 * static_cast<int64_t>(ks) + q_off[j]);
        // Scales / zeros of K rows 32 ks + 8 quad .. +7 in the group of column n.
        const uint4 sv = *reinterpret_cast<const uint4 *>(sb + 64 * static_cast<int64_t>(ks) + 2 * s_off[j]);
        const uint4 zv = *reinterpret_cast<const uint4 *>(zb + 64 * static_cast<int64_t>(ks) + 2 * z_off[j]);
        sst[f][j][0] = sv.x; sst[f][j][1] = sv.y; sst[f][j][2] = sv.z; sst[f][j][3] = sv.w;
        szt[f][j][0] = zv.x; szt[f][j][1] = zv.y; szt[f][j][2] = zv.z; szt[f][j][3] = zv.w;
      } else {
        if constexpr (FMT == FMT_DSV4_2)  // 8 two-bit codes: 2 bytes
          sq[f][j] = *reinterpret_cast<const uint16_t *>(qb + 8 * static_cast<int64_t>(ks) + q_off[j]);
        else
          sq[f][j] = *reinterpret_cast<const uint32_t *>(qb + 16 * static_cast<int64_t>(ks) + q_off[j]);
        // The group of K rows 32 ks + 8 quad .. + 7: a multiply-high by the
        // launch's reciprocal (exact for this layer's offsets), else a division.
        const uint32_t x = static_cast<uint32_t>(32 * ks + 8 * quad);
        uint32_t g;
        if (p.rtn_gs_magic != 0) g = __umulhi(x, p.rtn_gs_magic);
        else g = x / static_cast<uint32_t>(p.rtn_gs);
        const uint32_t i = s_off[j] + g * static_cast<uint32_t>(p.sz_stride_g);
        if constexpr (RDT != 0) {
          ss[f][j] = *reinterpret_cast<const uint16_t *>(sb + 2 * i);
          sz[f][j] = *reinterpret_cast<const uint16_t *>(zb + 2 * i);
        } else {
          ss[f][j] = __float_as_uint(load_any_f32(p.scales, i, p.scale_dtype));
          sz[f][j] = __float_as_uint(load_any_f32(p.zeros, i, p.zero_dtype));
        }
      }
    }
  };
  auto store_a = [&](int buf, auto fc) __attribute__((always_inline)) {
    constexpr int f = decltype(fc)::value;
#pragma unroll
    for (int i = 0; i < A_PER_THREAD; ++i) {
      const int ch = tid + 256 * i;
      *reinterpret_cast<uint4 *>(&As[buf][(ch >> 2) * A_LDS_STRIDE + 8 * (ch & 3)]) =
          make_uint4(sa[f][4 * i], sa[f][4 * i + 1], sa[f][4 * i + 2], sa[f][4 * i + 3]);
    }
  };

  // The prologue issues each step's loads in the loop's order.
  static_for<0, PF>([&](auto fc) __attribute__((always_inline)) {
    load(fc, ks_begin + decltype(fc)::value);
    __builtin_amdgcn_sched_barrier(0);
  });
  v4f32 acc[WM][WN];
#pragma unroll
  for (int t = 0; t < WM; ++t)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[t][j] = v4f32{0.f, 0.f, 0.f, 0.f};
  // RTN (16-bit activations): the exact single-rounding dequant when every
  // group parameter this workgroup reads allows it (checked once, the loads
  // overlapping the prologue's; the loop is built for both cases).
  constexpr bool RTN16 = FMT == FMT_RTN && DT != OC_DTYPE_F32;
  bool fast = false;
  if constexpr (RTN16) {
    const int k_lo = 32 * wg_begin, k_hi = 32 * max(wg_end, wg_begin + 1) - 1;
    const int g0 = k_lo / p.rtn_gs, ng = k_hi / p.rtn_gs - g0 + 1;
    bool ok = true;
    for (int i = tid; i < BN * ng; i += 256) {
      const int n = min(n0 + i / ng, p.N - 1);
      const int64_t e = n * p.sz_stride_n + static_cast<int64_t>(g0 + i % ng) * p.sz_stride_g;
      RtnParam rp;
      rp.sq = round_to<DT>(load_any_f32(p.scales, e, p.scale_dtype));
      rp.zq = round_to<DT>(load_any_f32(p.zeros, e, p.zero_dtype));
      ok = ok && rtn_fast_ok<DT>(rp);
    }
    fast = __syncthreads_and(ok) != 0;
  }
  if (nsteps > 0) store_a(0, ic<0>{});
  barrier_no_fence();

  const int nsteps_pad = (part + PF - 1) / PF * PF;  // the same in every group (one barrier per step)
  auto main_loop = [&](auto fastc) __attribute__((always_inline)) {
  constexpr bool FAST = decltype(fastc)::value;
  for (int i0 = 0; i0 < nsteps_pad; i0 += PF) {
    static_for<0, PF>([&](auto fc) __attribute__((always_inline)) {
      constexpr int f = decltype(fc)::value;
      const int i = i0 + f;  // step ks_begin + i sits in stage f; refilled once consumed
      if (i < nsteps) {      // uniform over the workgroup
        // A fragments first: their LDS latency overlaps the dequantization.
        uint4 av[WM];
#pragma unroll
        for (int t = 0; t < WM; ++t)
          av[t] = *reinterpret_cast<const uint4 *>(&As[i & 1][(16 * t + c16) * A_LDS_STRIDE + 8 * quad]);
        uint4 b[WN];
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          if constexpr (FMT == FMT_GPTQ) {
            b[j] = dequant8<DT>(sq[f][j], make_group_param(scale_f32<SDT>(ss[f][j]), tile_zero(sz[f][j], c16)));
          } else if constexpr (FMT == FMT_GPTQ8) {
            const float sv = scale_f32<SDT>(ss[f][j]);
            const float zv = static_cast<float>((sz[f][j] >> (8 * (c16 & 3))) & 0xFFu);
            b[j] = dequant8_u8<DT>(sq[f][j], sq8[f][j], sv, -sv * zv);
          } else if constexpr (FMT == FMT_RTN_T) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              RtnParam rp;
              rp.sq = round_to<DT>(half_to_f32<RDT>((sst[f][j][e >> 1] >> (16 * (e & 1))) & 0xFFFFu));
              rp.zq = round_to<DT>(half_to_f32<RDT>((szt[f][j][e >> 1] >> (16 * (e & 1))) & 0xFFFFu));
              v[e] = rtn_value<DT>(static_cast<int>((sq[f][j] >> (4 * e)) & 0xFu), rp);
            }
            b[j] = uint4{pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]), pack2<DT>(v[4], v[5]), pack2<DT>(v[6], v[7])};
          } else if constexpr (FMT == FMT_DSV4_4 || FMT == FMT_DSV4_2) {
            float sv, zv;
            if constexpr (RDT != 0) {
              sv = half_to_f32<RDT>(ss[f][j]);
              zv = half_to_f32<RDT>(sz[f][j]);
            } else {
              sv = __uint_as_float(ss[f][j]);
              zv = __uint_as_float(sz[f][j]);
            }
            b[j] = dsv4_dequant8<DT, FMT == FMT_DSV4_2 ? 2 : 4>(sq[f][j], sv, zv);
          } else {
            RtnParam rp;
            if constexpr (RDT != 0) {
              rp.sq = round_to<DT>(half_to_f32<RDT>(ss[f][j]));
              rp.zq = round_to<DT>(half_to_f32<RDT>(sz[f][j]));
            } else {
              rp.sq = round_to<DT>(__uint_as_float(ss[f][j]));
              rp.zq = round_to<DT>(__uint_as_float(sz[f][j]));
            }
            if constexpr (FAST) b[j] = rtn_dequant8_fast<DT>(sq[f][j], rp);
            else b[j] = rtn_dequant8<DT>(sq[f][j], rp);
          }
        }
#pragma unroll
        for (int t = 0; t < WM; ++t)
#pragma unroll
          for (int j = 0; j < WN; ++j) acc[t][j] = mfma16x16x32<DT>(av[t], b[j], acc[t][j]);
        if (i + 1 < nsteps) store_a((i + 1) & 1, ic<(f + 1) % PF>{});
      }
      load(fc, ks_begin + i + PF);
      barrier_no_fence();  // the next step's activations are in LDS; this step's reads are done
    });
  }
  };
  if (RTN16 && fast) main_loop(std::true_type{});
  else main_loop(std::false_type{});

  if constexpr (KG > 1) {
    // Groups 1.. park their sums; group 0 adds them in group order.
    __shared__ float red[KG > 1 ? (KG - 1) * BM * BN : 1];
    auto slot = [&](int g, int t, int j, int i) { return (((g * 4 + wave) * WM + t) * WN * 4 + j * 4 + i) * 64 + lane; };
    if (grp > 0) {
#pragma unroll
      for (int t = 0; t < WM; ++t)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) red[slot(grp - 1, t, j, i)] = acc[t][j][i];
    }
    __syncthreads();
    if (grp > 0) return;
    for (int g = 0; g < KG - 1; ++g)
#pragma unroll
      for (int t = 0; t < WM; ++t)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[t][j][i] += red[slot(g, t, j, i)];
  }
  // Epilogue. acc[t][j][i] = tile row 16t + 4*quad + i, column 16*(tw+j) + c16.
  if (p.ksplit == 1 && !p.out_f32) {
    // Every bias first and one wait on every path: bias loads behind dtype
    // branches mixed with the stores made the compiler wait for all memory
    // operations, the previous stores included, before each store.
    float bvs[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n = TILE_N * (tw + j) + c16;
      bvs[j] = n < p.N ? bias_at(p, n) : 0.f;
    }
    wait_vmcnt<0>();
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n = TILE_N * (tw + j) + c16;
      if (n >= p.N) continue;
      const float bv = bvs[j];
#pragma unroll
      for (int t = 0; t < WM; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = m0 + 16 * t + 4 * quad + i;
          if (r < p.M) store_c<DT>(p.c, static_cast<int64_t>(r) * p.ldc + n, acc[t][j][i] + bv);
        }
    }
  } else {
    // split-K (or fp32 output): fp32 partials; the caller's reduce sums them in split order
    float *part = p.partials + static_cast<int64_t>(blockIdx.z) * p.M * p.N;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n = TILE_N * (tw + j) + c16;
      if (n >= p.N) continue;
#pragma unroll
      for (int t = 0; t < WM; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = m0 + 16 * t + 4 * quad + i;
          if (r < p.M) __builtin_nontemporal_store(acc[t][j][i], part + static_cast<int64_t>(r) * p.N + n);
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Large-M GPTQ kernel. Workgroup tile 128 x (64 * WN): 4 waves split the
// columns (WN tiles of 16 each, 8 x WN MFMA tiles per wave). Every K step's
// operands (the 128 x 32 activation block, 8 KB, and the workgroup's weight
// words, scales and zeros) are copied global -> LDS by the DMA path
// (global_load_lds, no registers) into a ring of BIG_NS buffers, BIG_NS - 1
// steps ahead. Each wave dequantizes only its own columns, once per step,
// from LDS. WN = 3: two workgroups per CU; WN = 6: one, with half the LDS
// traffic per MFMA.
//
// DMA accounting: every wave issues the same DMA instructions each step, with
// no branch around them (see BigLayout: lanes and waves without a job copy a
// valid word into a pad; steps past the end reload the last step), and no
// other vector memory instruction in the loop. So "this wave's copies of
// step s have landed" is vmcnt <= DMA * (BIG_NS - 2), and a barrier then
// makes every wave's copies visible. The ring buffers are distinct LDS arrays, and every
// access names one of them (slot indices are compile-time constants).
// grid = (ceil(N / (64 WN)), ceil(M / 128), ksplit).
constexpr int BIG_NS = 4;   // LDS ring depth

// One weight ring slot, in dwords. Words are tile-major, 64 per tile, from 0.
// WN = 3: waves 0-2 copy tiles 4w..4w+3 to 256w, wave 3 the scales to SC;
//         every wave's 4-byte DMA lands at Z + 64w (wave 3's: the zero words).
// WN = 6: 16-byte DMA X of wave w copies tiles 4w..4w+3 to 256w; DMA Y of
//         waves 0-1 copies tiles 16 + 4w.. to 1024 + 256w, of wave 2 the
//         scales to SC (wave 3: a pad); the 4-byte DMA of wave 0 copies the
//         zero words to Z (waves 1-3: pads).
template <int WN>
struct BigLayout {
  static constexpr int TILES = 4 * WN;  // 16-column tiles per workgroup
  static constexpr int WDMA = WN == 3 ? 2 : 3;  // weight DMA instructions per wave per step
  static constexpr int SC = WN == 3 ? 768 : 1536;
  static constexpr int Z = WN == 3 ? 1024 : 2048;
  static constexpr int ZREAD = WN == 3 ? Z + 192 : Z;
  static constexpr int DW = Z + 256;
};


template <int DT, int SDT, int WM, int WN, int KPS, bool MOE, int NSX = (KPS == 1 ? 4 : 3)>
__global__ __launch_bounds__(256, MOE && NSX == 4 ? 3 : (WM <= 8 && WN == 3 && NSX <= 6 ? 2 : 1)) void gemm_big_kernel(GemmParams p) {
  // WM 16-row tiles per workgroup; KPS K steps per ring stage (one barrier
  // per stage); ring depth NS. MOE: grid z = expert; the workgroup walks its
  // expert's routed rows (expert_offsets / sorted_pairs) in blocks of 16 WM.
  using L = BigLayout<WN>;
  constexpr int BM = 16 * WM;
  constexpr int NS = NSX;  // ring depth: NS - 1 stages in flight
  static_assert(NS >= 3 && NS <= 8, "ring depth");
  constexpr int TILES = L::TILES;
  constexpr int AST = BM * 4;       // uint4 per K step of activations
  constexpr int ADMA = BM / 64;     // activation DMAs per wave per K step
  constexpr int DMA = ADMA + L::WDMA;
  static_assert((WM == 4 || WM == 8 || WM == 16) && (WN == 3 || WN == 6) && (KPS == 1 || KPS == 2),
                "DMA assignment");
  // One distinct LDS array per ring slot (the compiler's wait insertion tells
  // DMA targets apart by array); slots past NS are one element.
  constexpr int ASZ = KPS * AST, WSZ = KPS * L::DW;
  __shared__ __attribute__((aligned(1024))) uint4 A0[ASZ], A1[ASZ], A2[ASZ], A3[NS > 3 ? ASZ : 1],
      A4[NS > 4 ? ASZ : 1], A5[NS > 5 ? ASZ : 1], A6[NS > 6 ? ASZ : 1], A7[NS > 7 ? ASZ : 1];
  __shared__ __attribute__((aligned(1024))) uint32_t W0[WSZ], W1[WSZ], W2[WSZ], W3[NS > 3 ? WSZ : 1],
      W4[NS > 4 ? WSZ : 1], W5[NS > 5 ? WSZ : 1], W6[NS > 6 ? WSZ : 1], W7[NS > 7 ? WSZ : 1];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int quad = lane >> 4, c16 = lane & 15;
  const int nb = (p.N + 16 * TILES - 1) / (16 * TILES);
  const int flat = MOE ? static_cast<int>(blockIdx.x) : xcd_block(blockIdx.y * nb + blockIdx.x, nb * gridDim.y);
  const int bx = flat % nb, by = flat / nb;
  const int t0 = bx * TILES;  // first tile of the workgroup
  const int ks_begin = MOE ? 0 : blockIdx.z * p.ksteps_per_split;
  const int ks_end = MOE ? p.KS : min(ks_begin + p.ksteps_per_split, p.KS);
  const int tiles = (p.N + TILE_N - 1) / TILE_N;
  int row_begin = by * BM, row_end = p.M;
  const uint32_t *qw = static_cast<const uint32_t *>(p.qw);
  const uint16_t *sc = static_cast<const uint16_t *>(p.scales);
  const uint32_t *zw = static_cast<const uint32_t *>(p.zeros);
  if constexpr (MOE) {
    const int e = blockIdx.z;
    row_begin = p.expert_offsets[e];
    row_end = p.expert_offsets[e + 1];
    qw += e * p.qw_expert_stride;
    sc += e * p.s_expert_stride;
    zw += e * p.z_expert_stride;
  }
  const __amdgpu_buffer_rsrc_t rs_a = buffer_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rs_q = buffer_rsrc(qw, static_cast<int64_t>(tiles) * p.KS * 256);
  const __amdgpu_buffer_rsrc_t rs_s = buffer_rsrc(sc, static_cast<int64_t>(tiles) * p.G * 32);
  const __amdgpu_buffer_rsrc_t rs_z = buffer_rsrc(zw, static_cast<int64_t>(tiles) * p.G * 8);
  // Logical row -> activation row and output row.
  auto src_row = [&](int r) -> int64_t { return MOE ? p.sorted_pairs[r] / p.topk : r; };
  auto dst_row = [&](int r) -> int64_t { return MOE ? p.sorted_pairs[r] : r; };

  // One block of up to BM rows starting at m0 (all waves, whole K range).
  auto run = [&](int m0) {
    // Row tiles of this block holding rows (all of them unless grouped).
    const int active_tiles = MOE ? min(WM, (row_end - m0 + 15) / 16) : WM;
    // Activation sources: DMA i of wave w fills LDS rows 16 (ADMA w + i) + lane / 4,
    // 16-byte position lane % 4, which holds chunk (position ^ big_swz(row)) of
    // that row (rows past the end re-read the last row; never stored).
    uint32_t avo[ADMA];  // byte offsets into the activations
#pragma unroll
    for (int i = 0; i < ADMA; ++i) {
      const int l = 16 * (ADMA * wave + i) + (lane >> 2);
      const int r = min(m0 + l, row_end - 1);
      avo[i] = static_cast<uint32_t>(src_row(r) * p.lda * 2 + 16 * ((lane & 3) ^ big_swz(l)));
    }
    // Weight sources. Words: 16-byte DMAs copy 4 tiles each (lane: tile lane / 16,
    // 16 bytes lane % 16 of its 256). Scales (lane: tile lane / 2, 16 bytes
    // lane % 2 of its 32) and zero words (lane: tile lane / 2, word lane % 2).
    // Tiles past N re-read the last tile; lanes without a job re-read a valid word.
    const int tm = min(t0 + min(lane >> 1, TILES - 1), tiles - 1);  // metadata tile of this lane
    const bool meta_job = lane < 2 * TILES;
    const int tqx = min(t0 + 4 * wave + (lane >> 4), tiles - 1);
    const int tqy = min(t0 + 16 + 4 * wave + (lane >> 4), tiles - 1);
    // Which wave carries the scales (WN = 3: wave 3; WN = 6: wave 2, wave 3 a pad).
    const bool sc_wave = WN == 3 ? wave == 3 : wave >= 2;
    const int sc_dst = WN == 3 ? (wave == 3 ? L::SC : 256 * wave) : 1024 + 256 * wave;

    // Per-lane byte offsets of the weight copies (the K step / group part is
    // added as a scalar per step).
    const uint32_t vo_s = static_cast<uint32_t>(tm) * p.G * 32 + 16 * (lane & 1);
    const uint32_t vo_z = static_cast<uint32_t>(tm) * p.G * 8 + (meta_job ? 4 * (lane & 1) : 0);
    const uint32_t vo_qx = static_cast<uint32_t>(tqx) * p.KS * 256 + 16 * (lane & 15);
    const uint32_t vo_qy = static_cast<uint32_t>(tqy) * p.KS * 256 + 16 * (lane & 15);

    // The copies of one K step into one ring stage part.
    auto issue1 = [&](uint4 *ab, uint32_t *wb, int ks) {
      const int kk = min(ks, ks_end - 1);  // past the end: reload the last step
#pragma unroll
      for (int i = 0; i < ADMA; ++i) dma16(rs_a, avo[i], 64 * kk, ab + 64 * (ADMA * wave + i));
      const int g = group_of(p, kk);
      if constexpr (WN == 3) {
        if (sc_wave) dma16(rs_s, vo_s, 32 * g, wb + sc_dst);
        else dma16(rs_q, vo_qx, 256 * kk, wb + sc_dst);
      } else {
        dma16(rs_q, vo_qx, 256 * kk, wb + 256 * wave);
        if (sc_wave) dma16(rs_s, vo_s, 32 * g, wb + sc_dst);
        else dma16(rs_q, vo_qy, 256 * kk, wb + sc_dst);
      }
      dma4(rs_z, vo_z, 8 * g, wb + L::Z + 64 * wave);
    };
    auto issue = [&](uint4 *ab, uint32_t *wb, int stage) {
#pragma unroll
      for (int h = 0; h < KPS; ++h) issue1(ab + h * AST, wb + h * L::DW, ks_begin + KPS * stage + h);
    };

    v4f32 acc[WM][WN];
#pragma unroll
    for (int t = 0; t < WM; ++t)
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[t][j] = v4f32{0.f, 0.f, 0.f, 0.f};

    auto compute1 = [&](const uint4 *ab, const uint32_t *wb) {
      const uint16_t *sb = reinterpret_cast<const uint16_t *>(wb + L::SC);
      uint4 b[WN];
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int tj = WN * wave + j;  // tile within the workgroup
        const uint32_t q = wb[tj * 64 + c16 * 4 + quad];
        const float sv = scale_f32<SDT>(sb[tj * 16 + c16]);
        const int zv = tile_zero(wb[L::ZREAD + tj * 2 + (c16 >> 3)], c16);
        b[j] = dequant8<DT>(q, make_group_param(sv, zv));
      }
#pragma unroll
      for (int t = 0; t < WM; ++t) {
        // Grouped experts fill a block only partly (~64 of 128 routed rows):
        // row tiles past the expert's rows are skipped (a wave-uniform branch).
        if (MOE && t >= active_tiles) break;
        const int row = 16 * t + c16;
        const uint4 av = ab[row * 4 + (quad ^ big_swz(row))];
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[t][j] = mfma16x16x32<DT>(av, b[j], acc[t][j]);
      }
    };

    // One ring stage on slot U (a compile-time constant).
    auto slot_a = [&](auto U) -> uint4 * {
      constexpr int u = decltype(U)::value;
      if constexpr (u == 0) return A0;
      else if constexpr (u == 1) return A1;
      else if constexpr (u == 2) return A2;
      else if constexpr (u == 3) return A3;
      else if constexpr (u == 4) return A4;
      else if constexpr (u == 5) return A5;
      else if constexpr (u == 6) return A6;
      else return A7;
    };
    auto slot_w = [&](auto U) -> uint32_t * {
      constexpr int u = decltype(U)::value;
      if constexpr (u == 0) return W0;
      else if constexpr (u == 1) return W1;
      else if constexpr (u == 2) return W2;
      else if constexpr (u == 3) return W3;
      else if constexpr (u == 4) return W4;
      else if constexpr (u == 5) return W5;
      else if constexpr (u == 6) return W6;
      else return W7;
    };
    auto step = [&](auto U, int stage) {
      constexpr int u = decltype(U)::value;
      constexpr int un = (u + NS - 1) % NS;
      uint4 *ab = slot_a(U);
      uint32_t *wb = slot_w(U);
      uint4 *abn = slot_a(ic<un>{});
      uint32_t *wbn = slot_w(ic<un>{});
      wait_vmcnt<DMA * KPS * (NS - 2)>();  // this wave's copies of the stage landed ...
      barrier_no_fence();                      // ... and everyone's; slot un is free again
      issue(abn, wbn, stage + NS - 1);
#pragma unroll
      for (int h = 0; h < KPS; ++h)
        if (ks_begin + KPS * stage + h < ks_end) compute1(ab + h * AST, wb + h * L::DW);
    };
    // Ring cycle starting at stage s0 over slots 0 .. n-1 (n <= NS).
    auto cycle = [&](int s0, int n) {
      if (n > 0) step(ic<0>{}, s0);
      if (n > 1) step(ic<1>{}, s0 + 1);
      if (n > 2) step(ic<2>{}, s0 + 2);
      if constexpr (NS > 3) if (n > 3) step(ic<3>{}, s0 + 3);
      if constexpr (NS > 4) if (n > 4) step(ic<4>{}, s0 + 4);
      if constexpr (NS > 5) if (n > 5) step(ic<5>{}, s0 + 5);
      if constexpr (NS > 6) if (n > 6) step(ic<6>{}, s0 + 6);
      if constexpr (NS > 7) if (n > 7) step(ic<7>{}, s0 + 7);
    };

    issue(A0, W0, 0);
    issue(A1, W1, 1);
    if constexpr (NS > 3) issue(A2, W2, 2);
    if constexpr (NS > 4) issue(A3, W3, 3);
    if constexpr (NS > 5) issue(A4, W4, 4);
    if constexpr (NS > 6) issue(A5, W5, 5);
    if constexpr (NS > 7) issue(A6, W6, 6);
    const int nst = (ks_end - ks_begin + KPS - 1) / KPS;  // stages
    const int nfull = nst / NS * NS;
    for (int s0 = 0; s0 < nfull; s0 += NS) cycle(s0, NS);
    if (nst > nfull) cycle(nfull, nst - nfull);
    wait_vmcnt<0>();  // no DMA outlives the workgroup's LDS

    // Epilogue. acc[t][j][i] = row m0 + 16t + 4*quad + i, column 16*(t0 + WN wave + j) + c16.
    const int tw = t0 + WN * wave;
    if (MOE || p.ksplit == 1) {
      // Biases first, then per row tile its destination rows (grouped: loads
      // of the routing table), each time one wait on every path (loads mixed
      // with the stores made every store wait for the previous ones).
      float bvs[WN];
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int n = TILE_N * (tw + j) + c16;
        bvs[j] = n < p.N ? bias_at(p, n) : 0.f;
      }
      wait_vmcnt<0>();
#pragma unroll
      for (int t = 0; t < WM; ++t) {
        int drow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = m0 + 16 * t + 4 * quad + i;
          drow[i] = r < row_end ? static_cast<int>(dst_row(r)) : -1;
        }
        if constexpr (MOE) wait_vmcnt<0>();
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          const int n = TILE_N * (tw + j) + c16;
          if (n >= p.N) continue;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (drow[i] >= 0) store_c<DT>(p.c, static_cast<int64_t>(drow[i]) * p.ldc + n, acc[t][j][i] + bvs[j]);
        }
      }
    } else {
      float *part = p.partials + static_cast<int64_t>(blockIdx.z) * p.M * p.N;
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int n = TILE_N * (tw + j) + c16;
        if (n >= p.N) continue;
#pragma unroll
        for (int t = 0; t < WM; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = m0 + 16 * t + 4 * quad + i;
            if (r < p.M) __builtin_nontemporal_store(acc[t][j][i], part + static_cast<int64_t>(r) * p.N + n);
          }
      }
    }
  };
  if constexpr (MOE) {
    for (int m0 = row_begin; m0 < row_end; m0 += BM) {
      run(m0);
      __syncthreads();  // the next block's prologue reuses the ring
    }
  } else {
    if (row_begin < row_end) run(row_begin);
  }
}

// ---------------------------------------------------------------------------
// MoE routing: stable counting sort of (token, slot) pairs by expert.
// One workgroup of 256 threads; thread t owns the contiguous pair range
// [t*per, (t+1)*per), so ranks computed from per-thread prefix counts keep
// the original pair order inside every expert.
constexpr int ROUTE_WAVES = 16;
constexpr int ROUTE_THREADS = 64 * ROUTE_WAVES;

// Stable counting sort of the P = T * topk (token, slot) pairs by expert, in
// one workgroup. Wave w owns the pairs [w * chunk, (w + 1) * chunk), 64 at a
// time: the lanes of a batch that hold the same expert find each other with
// one ballot per expert-id bit, so a lane's rank among them is a popcount
// and the highest of them adds the batch's count to the wave's counter for
// that expert (no atomics; pair order is kept within and across batches).
// Expert totals, their exclusive scan (offsets) and per-wave bases follow;
// a second pass writes every pair at base + rank. Ids outside [0, E) are
// dropped.
__global__ __launch_bounds__(ROUTE_THREADS) void moe_route_kernel(const int64_t *__restrict__ ids, int P,
                                                                  int E, int32_t *__restrict__ offsets,
                                                                  int32_t *__restrict__ sorted) {
  extern __shared__ int32_t cnt[];  // [ROUTE_WAVES][E] per-wave counts (then bases), then [E] offsets
  __shared__ int32_t wave_tot[ROUTE_WAVES];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int32_t *eoff = cnt + ROUTE_WAVES * E;
  const int bits = 32 - __builtin_clz(static_cast<unsigned>(E));  // ids 0..E (E marks "dropped")
  const int chunk = (P + ROUTE_WAVES - 1) / ROUTE_WAVES;
  const int q_begin = min(w * chunk, P), q_end = min(q_begin + chunk, P);
  const uint64_t below = (uint64_t{1} << lane) - 1;
  for (int i = tid; i < (ROUTE_WAVES + 1) * E; i += ROUTE_THREADS) cnt[i] = 0;
  __syncthreads();

  // Expert of pair q (E: dropped or past the wave's pairs).
  auto expert_of = [&](int q) {
    const int64_t id = q < q_end ? ids[q] : -1;
    return id >= 0 && id < E ? static_cast<int>(id) : E;
  };
  // Same-expert lanes of a batch, this lane's rank among them and their count.
  auto match = [&](int e, int &rank, int &count) {
    uint64_t mask = __ballot(1);
    for (int b = 0; b < bits; ++b) {
      const uint64_t bb = __ballot((e >> b) & 1);
      mask &= ((e >> b) & 1) ? bb : ~bb;
    }
    rank = __popcll(mask & below);
    count = __popcll(mask);
  };
  int32_t *wc = cnt + w * E;
  // Rounds of RB batches: their id loads go out together.
  constexpr int RB = 8;
  for (int q0 = q_begin; q0 < q_end; q0 += 64 * RB) {
    int ex[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) ex[r] = expert_of(q0 + 64 * r + lane);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      if (q0 + 64 * r >= q_end) break;
      int rank, count;
      match(ex[r], rank, count);
      if (ex[r] < E && rank == count - 1) wc[ex[r]] += count;
    }
  }
  __syncthreads();

  // Expert totals, exclusive scan over experts (E <= ROUTE_THREADS: a scan
  // per wave, then over the wave totals).
  {
    const int e = tid;
    int tot = 0;
    if (e < E)
      for (int v = 0; v < ROUTE_WAVES; ++v) tot += cnt[v * E + e];
    int incl = tot;
    for (int d = 1; d < 64; d <<= 1) {
      const int up = __shfl_up(incl, d);
      if (lane >= d) incl += up;
    }
    if (lane == 63) wave_tot[w] = incl;
    __syncthreads();
    int before = 0;
    for (int v = 0; v < w; ++v) before += wave_tot[v];
    if (e < E) eoff[e] = before + incl - tot;  // exclusive offset of expert e
    __syncthreads();
  }
  // Per-wave bases: offset of the expert plus the counts of earlier waves.
  if (tid < E) {
    const int e = tid;
    offsets[e] = eoff[e];
    int run = eoff[e];
    for (int v = 0; v < ROUTE_WAVES; ++v) {
      const int c = cnt[v * E + e];
      cnt[v * E + e] = run;
      run += c;
    }
    if (e == E - 1) offsets[E] = run;  // pairs kept
  }
  __syncthreads();

  for (int q0 = q_begin; q0 < q_end; q0 += 64 * RB) {
    int ex[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) ex[r] = expert_of(q0 + 64 * r + lane);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      if (q0 + 64 * r >= q_end) break;
      const int e = ex[r];
      int rank, count;
      match(e, rank, count);
      // Every lane reads its base before the group's last lane advances it
      // (one wave's LDS accesses complete in program order).
      const int base = e < E ? wc[e] : 0;
      if (e < E) sorted[base + rank] = q0 + 64 * r + lane;
      if (e < E && rank == count - 1) wc[e] = base + count;
    }
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.

struct TileCfg {
  int wm, wn, kg;
};

// Shape of the LDS-tiled kernel: the largest tile whose grid fills the chip
// (want workgroups, one per CU), else 64 x 64 tiles. Those run K groups: two
// when their grid fills the chip, four (no K split) from half of it, and a
// K split over fp32 partials below that (each part of 16 or more steps when
// split_k allows it). Measured on MI355X, 64 x 64 tiles: RTN M=512 K=1024
// N=2048 (256 tiles) 15.1 / 12.5 / 13.2 us with 1 / 2 / 4 groups; padded
// gs26 M=256 K=1056 N=3072 (192 tiles) 18.9 us split in two, 15.0 us with
// four groups and no split.
int env_int(const char *name, int dflt);
TileCfg pick_tiles(int M, int N, int ksteps, int *ksplit, int *ksteps_per_split, bool split_k = true) {
  static const int want = std::max(1, env_int("ONECOMP_HIP_TILED_MIN_WGS", 256));
  static const TileCfg cfgs[] = {{16, 3, 1}, {8, 2, 1}, {4, 1, 1}};
  TileCfg pick = cfgs[2];
  // The largest tile whose grid fills at least 3/4 of the target (bigger
  // tiles re-read fewer activation and weight bytes: the packed Conv1d's RTN
  // GEMM, 7168 x 512 x 3584, 322 -> 257 us with 224 workgroups of 128 x 128
  // instead of 896 of 64 x 64).
  for (const TileCfg &c : cfgs) {
    if (4 * static_cast<int64_t>((M + 16 * c.wm - 1) / (16 * c.wm)) * ((N + 64 * c.wn - 1) / (64 * c.wn)) >=
        3 * static_cast<int64_t>(want)) {
      pick = c;
      break;
    }
  }
  const int64_t tiles = static_cast<int64_t>((M + 16 * pick.wm - 1) / (16 * pick.wm)) *
                        ((N + 64 * pick.wn - 1) / (64 * pick.wn));
  int ks = 1;
  if (pick.wm == 4) {
    if (tiles >= want) {
      pick.kg = ksteps >= 16 ? 2 : 1;
    } else if (2 * tiles >= want || !split_k) {
      pick.kg = ksteps >= 32 ? 4 : ksteps >= 16 ? 2 : 1;
    } else {
      ks = static_cast<int>(std::min<int64_t>(want / tiles, std::max(1, ksteps / 16)));
      const int per = (ksteps + ks - 1) / ks;
      pick.kg = per >= 32 ? 4 : per >= 16 ? 2 : 1;
    }
  }
  *ksteps_per_split = (ksteps + ks - 1) / ks;
  *ksplit = (ksteps + *ksteps_per_split - 1) / *ksteps_per_split;
  return pick;
}

int env_int(const char *name, int dflt) {
  const char *v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int s = 0;
  while ((1 << s) < v) ++s;
  return s;
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

// Decode launch shapes: waves per workgroup x tiles per workgroup.
enum { DOT_W8 = 0, DOT_W8_HALF = 1, DOT_W4 = 2 };

struct Plan {
  int regime;
  int mt;        // small-M kernel: row tiles of 16
  TileCfg tile;  // large-M kernel
  int ksplit;
  int ksteps_per_split;
  bool gather;   // activations gathered into physical order first (kmap, MFMA regimes)
  int waves;     // decode kernel: launch shape (DOT_W*)
  bool big;      // large M: gemm_big_kernel
  int wide_wn;   // large M: gemm_wide_kernel with this many tiles per wave (0: not used)
  bool legacy_dot;  // decode: whole-tile gemv_dot_kernel (else the split-item GEMV)
  GemvPlan gv;      // decode: split GEMV work items
  int stream_wgs;   // decode: balanced-range GEMV with this many workgroups (0: not used)
  bool stream_global;  // ... reading gathered activation rows from global memory
};

// Workspace layout: see COUNTER_BYTES (oc_internal.h).
constexpr int COUNTER_SLOTS = static_cast<int>(COUNTER_BYTES / sizeof(int));

// Compute units of the current device (cached per device).
int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (dev < 0 || dev >= 64) dev = 0;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Tiles per wave of the wide kernel for an M x N problem: the shape whose
// workgroups fill the compute units best (whole waves of workgroups over the
// CUs, times the useful fraction of the last column block). Ties go to 3
// tiles (192 columns), measured as fast as 4 on full grids and lighter on
// registers.
int pick_wide_wn(int M, int N) {
  static const int forced = env_int("ONECOMP_HIP_WIDE_WN", 0);
  if (forced == 3 || forced == 4) return forced;
  const int cus = device_cus();
  double best = -1.0;
  int pick = 3;
  for (int wn : {3, 4}) {
    const int64_t nbn = (N + 64 * wn - 1) / (64 * wn), nbm = (M + 255) / 256;
    const int64_t blocks = nbn * nbm;
    const double fill = static_cast<double>(blocks) / (static_cast<double>((blocks + cus - 1) / cus) * cus);
    const double useful = static_cast<double>(N) / (static_cast<double>(nbn) * 64 * wn);
    const double score = fill * useful;
    if (score > best + 0.02) {
      best = score;
      pick = wn;
    }
  }
  return pick;
}

// The decode kernel takes M <= 2, power-of-two groups of 32-row steps and its
// activation rows in (at most 128 KB of) LDS.
bool dot_eligible(int M, int K_phys, int group_rows) {
  (void)K_phys;
  return M >= 1 && M <= 2 && ilog2_exact(group_rows / 32) >= 0;
}
// The whole-tile kernel stages the entire activation row in LDS.
bool legacy_dot_fits(int M, int K_phys) { return dot_lds_bytes(M, K_phys / 32) <= 128 * 1024; }

Plan plan_gemm(int M, int N, int K_phys, int group_rows, bool has_kmap, int regime, bool has_kinv = true,
               int64_t lda_hint = 0) {
  Plan sp{};
  const int ksteps = K_phys / 32;
  // Tuning knobs, read once per process.
  static const bool dot_disabled = env_int("ONECOMP_HIP_DISABLE_DOT", 0) != 0;
  static const int want = std::max(1, env_int("ONECOMP_HIP_TILED_MIN_WGS", 256));
  const bool automatic = regime == OC_REGIME_AUTO;
  if (automatic) {
    if (!dot_disabled && dot_eligible(M, K_phys, group_rows)) regime = OC_REGIME_DOT;
    else regime = M <= 64 ? OC_REGIME_SPLITK : OC_REGIME_TILED;
  }
  sp.regime = regime;
  sp.ksplit = 1;
  sp.ksteps_per_split = ksteps;
  sp.gather = has_kmap && regime != OC_REGIME_DOT;
  if (regime == OC_REGIME_DOT) {
    // Balanced-range kernel (oc_gemv_stream.hip) for layers of one to six
    // tiles per compute unit whose activation rows fit in LDS: equal weight
    // bytes per compute unit and one staging each (measured 8-18 % faster
    // than whole tiles on 320 and 1088 tiles; a tie on 320 tiles of K=5120).
    // ONECOMP_HIP_GEMV_STREAM=0 (read per call) selects the kernels below.
    if (env_int("ONECOMP_HIP_GEMV_STREAM", 1) != 0) {
      sp.stream_wgs = gemv_stream_wgs(M, N, ksteps, device_cus(), COUNTER_BYTES);
      if (sp.stream_wgs > 0) return sp;
    }
    // Whole-tile kernel when it can run (measured faster or equal on the
    // decode shapes); the split-item kernel (oc_gemv.hip) gathers through
    // kmap without kinv and has no K limit. ONECOMP_HIP_GEMV_SPLIT=1 forces it.
    const bool split_forced = env_int("ONECOMP_HIP_GEMV_SPLIT", 0) != 0;  // read per call (tests switch it)
    if (split_forced || (has_kmap && !has_kinv) || !legacy_dot_fits(M, K_phys)) {
      // Balanced work items; K split when it evens the load.
      sp.gv = plan_gemv(M, N, ksteps, has_kmap, device_cus());
      const int tiles = (N + TILE_N - 1) / TILE_N;
      if (sp.gv.ksplit > 1 && (tiles + sp.gv.T - 1) / sp.gv.T > COUNTER_SLOTS)
        sp.gv = GemvPlan{sp.gv.T, (ksteps + 3) / 4 * 4, 1};
      sp.ksplit = sp.gv.ksplit;
      sp.ksteps_per_split = sp.gv.S;
      sp.gather = false;
      return sp;
    }
    sp.legacy_dot = true;
    static const int dot_shape = env_int("ONECOMP_HIP_DOT_SHAPE", -1);
    // 8 waves; half tiles (twice the workgroups) for narrow layers (N < 2048;
    // wider ones measured faster with whole tiles, which stage activations once
    // per 16 columns).
    // ONECOMP_HIP_DOT_SHAPE overrides (tuning only).
    const int tiles = (N + TILE_N - 1) / TILE_N;
    sp.waves = dot_shape >= DOT_W8 && dot_shape <= DOT_W4 ? dot_shape : (tiles < 128 ? DOT_W8_HALF : DOT_W8);
    return sp;
  }
  if (regime == OC_REGIME_SPLITK) {
    // Chosen automatically, batches of 3..16 rows take the balanced-range
    // kernel's MFMA form when their activation rows fit in LDS (it stages
    // act-order rows itself: no gather pass). ONECOMP_HIP_GEMV_STREAM=0
    // (read per call) keeps them on the whole-tile MFMA kernel below.
    // Not for layers the whole-tile kernel already spreads evenly and reads
    // without a gather (measured M = 8 K=N=4096: 6.7 us whole tiles, 7.7 us
    // staged; M = 16: 7.7 vs 9.3 us).
    const bool even_plain = !has_kmap && ((N + TILE_N - 1) / TILE_N) % device_cus() == 0;
    if (automatic && M >= 3 && M <= 16 && !even_plain && ilog2_exact(group_rows / 32) >= 0 &&
        env_int("ONECOMP_HIP_GEMV_STREAM", 1) != 0) {
      // ONECOMP_HIP_STREAM_GLOBAL=1 (read per call; tests) skips the staged form.
      const bool global_only = env_int("ONECOMP_HIP_STREAM_GLOBAL", 0) != 0;
      const int cus = device_cus();
      const int staged = global_only ? 0 : gemv_stream_wgs(M, N, ksteps, cus, COUNTER_BYTES);
      // Rows beyond LDS, or a narrow layer the staged form would run on under
      // half the CUs: the same ranges over rows read from global memory.
      const int global = staged >= cus / 2 ? 0 : gemv_stream_global_wgs(M, N, ksteps, cus, COUNTER_BYTES);
      if (global > staged) {
        sp.stream_wgs = global;
        sp.stream_global = true;
        return sp;  // sp.gather as planned: act-order rows are gathered first
      }
      if (staged > 0) {
        sp.stream_wgs = staged;
        sp.gather = false;
        return sp;
      }
    }
    sp.mt = std::max(1, (M + 15) / 16);
    return sp;
  }
  static const bool big_disabled = env_int("ONECOMP_HIP_DISABLE_BIG", 0) != 0;
  // The large-M kernel addresses its operands with 32-bit buffer offsets.
  const int64_t tiles16 = (N + TILE_N - 1) / TILE_N;
  const bool big_fits = static_cast<int64_t>(M) * std::max<int64_t>(lda_hint, K_phys) * 2 < (int64_t{1} << 31) &&
                        tiles16 * ksteps * 256 < (int64_t{1} << 31);
  static const int wide_min_m = env_int("ONECOMP_HIP_WIDE_MIN_M", 1024);
  if (M >= wide_min_m && wide_min_m > 0 && big_fits && ilog2_exact(group_rows / 32) >= 0) {
    // 256-row wave tiles, whole K per workgroup.
    sp.wide_wn = pick_wide_wn(M, N);
    return sp;
  }
  // Below 512 rows the 64 x 64 tiled kernel fills the chip better (measured
  // M = 256: K=1280 N=3072 16.9 vs 27.1 us, K=3072 N=12288 53.0 vs 56.3 us).
  if (M >= 512 && !big_disabled && big_fits) {
    // Pipelined 128 x 192 kernel; split K only when the grid cannot fill the chip.
    sp.big = true;
    const int blocks = ((M + 127) / 128) * ((N + 191) / 192);
    static const int min_steps = std::max(1, env_int("ONECOMP_HIP_SPLIT_MIN_STEPS", 16));
    int ksplit = 1;
    if (blocks < want) ksplit = std::min((want + blocks - 1) / blocks, std::max(1, ksteps / min_steps));
    sp.ksteps_per_split = (ksteps + ksplit - 1) / ksplit;
    sp.ksplit = (ksteps + sp.ksteps_per_split - 1) / sp.ksteps_per_split;
    return sp;
  }
  sp.tile = pick_tiles(M, N, ksteps, &sp.ksplit, &sp.ksteps_per_split);
  return sp;
}

// Workspace: [gathered activations (M x K_phys 16-bit)][split-K partials].
size_t gather_bytes(const Plan &sp, int M, int K_phys) {
  return sp.gather ? align256(static_cast<size_t>(M) * K_phys * 2) : 0;
}
size_t workspace_bytes(const Plan &sp, int M, int N, int K_phys) {
  size_t b = gather_bytes(sp, M, K_phys);
  if (sp.ksplit > 1) b += static_cast<size_t>(sp.ksplit) * M * N * sizeof(float);
  return b > 0 || sp.stream_wgs > 0 ? COUNTER_BYTES + b : 0;
}

template <int DT, int SDT, int MR, int XS, int WAVES, int CPW>
void launch_dot_t(const GemmParams &p, hipStream_t s) {
  auto kern = gemv_dot_kernel<DT, SDT, MR, XS, WAVES, CPW>;
  // Allow up to 128 KB of dynamic LDS, once per instantiation and device.
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  (void)hipGetDevice(&dev);
  const uint64_t bit = dev < 64 ? (uint64_t{1} << dev) : 0;
  if (!bit || !(attr_set.load(std::memory_order_relaxed) & bit)) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              128 * 1024);
    attr_set.fetch_or(bit, std::memory_order_relaxed);
  }
  const size_t lds = std::max(dot_lds_bytes(MR, p.KS), sizeof(float) * WAVES * MR * CPW);
  const int tiles = (p.N + TILE_N - 1) / TILE_N;
  hipLaunchKernelGGL(kern, dim3(tiles * (TILE_N / CPW)), dim3(64 * WAVES), lds, s, p);
}

template <int DT, int SDT, int MR, int XS>
void launch_dot_w(const GemmParams &p, int shape, hipStream_t s) {
  switch (shape) {
    case DOT_W8_HALF: launch_dot_t<DT, SDT, MR, XS, 8, 8>(p, s); break;
    case DOT_W4: launch_dot_t<DT, SDT, MR, XS, 4, 16>(p, s); break;
    default: launch_dot_t<DT, SDT, MR, XS, 8, 16>(p, s); break;
  }
}

template <int DT, int SDT>
void launch_dot(const GemmParams &p, const Plan &sp, hipStream_t s) {
  if (p.M == 1) {
    p.kinv ? launch_dot_w<DT, SDT, 1, XS_SCATTER>(p, sp.waves, s) : launch_dot_w<DT, SDT, 1, XS_CONTIG>(p, sp.waves, s);
  } else {
    p.kinv ? launch_dot_w<DT, SDT, 2, XS_SCATTER>(p, sp.waves, s) : launch_dot_w<DT, SDT, 2, XS_CONTIG>(p, sp.waves, s);
  }
}

template <int DT, int SDT, int MT, int NW>
void launch_mfma_t(const GemmParams &p, hipStream_t s) {
  // Quad-steps in flight (measured on MI355X): one when a wave has at most 4
  // (K = N = 4096, M = 16: 7.6 vs 8.2 us with 2 or 3), else two (K = 17408,
  // M = 8: 31.9 vs 34.5 us with one).
  const int per_wave = ((p.KS + 3) / 4 + NW - 1) / NW;
  const dim3 grid((p.N + TILE_N - 1) / TILE_N), block(64 * NW);
  if (per_wave <= 4) hipLaunchKernelGGL((gemv_mfma_kernel<DT, SDT, MT, NW, 1>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gemv_mfma_kernel<DT, SDT, MT, NW, 2>), grid, block, 0, s, p);
}

template <int DT, int SDT, int MT>
void launch_mfma_w(const GemmParams &p, int nw, hipStream_t s) {
  if (MT <= 2 && nw >= 8) launch_mfma_t<DT, SDT, MT, 8>(p, s);
  else launch_mfma_t<DT, SDT, MT, 4>(p, s);
}

// Waves per workgroup (measured on MI355X): 8 when there are few tiles and
// the per-lane state is small (M <= 32), else 4.
template <int DT, int SDT>
void launch_mfma(const GemmParams &p, int mt, hipStream_t s) {
  static const int env_nw = env_int("ONECOMP_HIP_MFMA_WAVES", 0);
  const int tiles = (p.N + TILE_N - 1) / TILE_N;
  const int nw = env_nw > 0 ? env_nw : (tiles <= 256 ? 8 : 4);
  switch (mt) {
    case 1: launch_mfma_w<DT, SDT, 1>(p, nw, s); break;
    case 2: launch_mfma_w<DT, SDT, 2>(p, nw, s); break;
    case 3: launch_mfma_w<DT, SDT, 3>(p, nw, s); break;
    default: launch_mfma_w<DT, SDT, 4>(p, nw, s); break;
  }
}

// ceil(2^32 / gs) when x * gs < 2^32 for every offset x < K (then
// umulhi(x, magic) = floor(x / gs): the error x (magic - 2^32 / gs) / 2^32 is
// below x / 2^32 < 1 / gs), else 0.
static uint32_t group_magic(int gs, int K) {
  if (gs < 2 || static_cast<uint64_t>(K) * static_cast<uint64_t>(gs) >= (uint64_t{1} << 32)) return 0;
  return static_cast<uint32_t>(((uint64_t{1} << 32) + gs - 1) / gs);
}

template <int DT, int SDT, int WM, int WN, int FMT, int KG>
void launch_tiled_t(const GemmParams &p_in, hipStream_t s) {
  GemmParams p = p_in;
  p.rtn_gs_magic = fmt_rows(FMT) ? group_magic(p.rtn_gs, p.K_phys) : 0;
  const dim3 grid((p.N + 64 * WN - 1) / (64 * WN), (p.M + 16 * WM - 1) / (16 * WM), p.ksplit);
  const bool same16 = fmt_rows(FMT) && p.scale_dtype == p.zero_dtype;
  if (same16 && p.scale_dtype == OC_DTYPE_F16)
    hipLaunchKernelGGL((gemm_tiled_kernel<DT, SDT, WM, WN, FMT, fmt_rows(FMT) ? OC_DTYPE_F16 : 0, KG>), grid,
                       dim3(256 * KG), 0, s, p);
  else if (same16 && p.scale_dtype == OC_DTYPE_BF16)
    hipLaunchKernelGGL((gemm_tiled_kernel<DT, SDT, WM, WN, FMT, fmt_rows(FMT) ? OC_DTYPE_BF16 : 0, KG>), grid,
                       dim3(256 * KG), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_tiled_kernel<DT, SDT, WM, WN, FMT, 0, KG>), grid, dim3(256 * KG), 0, s, p);
  if (p.ksplit > 1 && !p.out_f32) {
    const int64_t mn = static_cast<int64_t>(p.M) * p.N;
    hipLaunchKernelGGL(splitk_reduce_kernel<DT>, dim3(static_cast<unsigned>((mn / 4 + 255) / 256)), dim3(256), 0,
                       s, p);
  }
}

template <int DT, int SDT, int FMT>
void launch_tiled(const GemmParams &p, TileCfg c, hipStream_t s) {
  if (c.wm == 16 && c.wn == 3) launch_tiled_t<DT, SDT, 16, 3, FMT, 1>(p, s);
  else if (c.wm == 8 && c.wn == 2) launch_tiled_t<DT, SDT, 8, 2, FMT, 1>(p, s);
  else if (c.kg == 4) launch_tiled_t<DT, SDT, 4, 1, FMT, 4>(p, s);
  else if (c.kg == 2) launch_tiled_t<DT, SDT, 4, 1, FMT, 2>(p, s);
  else launch_tiled_t<DT, SDT, 4, 1, FMT, 1>(p, s);
}

// Launch shape: 128 x 192 tiles, one K step per stage (4-deep ring). Measured
// on MI355X against 128 x 384 (one workgroup per CU), 256 x 192 (one per CU)
// and two K steps per stage: this one is fastest on the M = 4096 shapes.
constexpr int BIG_WM = 8, BIG_WN = 3, BIG_KPS = 1;
// Grouped experts use the same 128-row blocks: measured faster than 64-row
// blocks, whose experts with more than 64 routed rows stream their weights twice.
constexpr int MOE_WM = BIG_WM;
// Ring depth of the grouped launch: 4, as the dense one (measured on the
// 64-expert top-8 workload: 6 stages no faster, 8 slower with one workgroup
// per CU). At depth 4 the kernel's launch bound asks for 3 waves per SIMD:
// the compiler does not reach it (191 registers, 2 workgroups per CU) but the
// schedule it makes for that target measured 217 -> 168 us on the workload;
// a hard cap at 168 registers (3 workgroups per CU, a small spill) measured
// the same. ONECOMP_HIP_MOE_NS (4, 6 or 8) overrides (tuning only).
constexpr int MOE_NS = 4;

template <int DT, int SDT>
void launch_moe(const GemmParams &p, dim3 grid, int ns, hipStream_t s) {
  if (ns == 4) hipLaunchKernelGGL((gemm_big_kernel<DT, SDT, MOE_WM, BIG_WN, BIG_KPS, true, 4>), grid, dim3(256), 0, s, p);
  else if (ns == 6) hipLaunchKernelGGL((gemm_big_kernel<DT, SDT, MOE_WM, BIG_WN, BIG_KPS, true, 6>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((gemm_big_kernel<DT, SDT, MOE_WM, BIG_WN, BIG_KPS, true, 8>), grid, dim3(256), 0, s, p);
}

template <int DT, int SDT>
void launch_big(const GemmParams &p, hipStream_t s) {
  const dim3 grid((p.N + 64 * BIG_WN - 1) / (64 * BIG_WN), (p.M + 16 * BIG_WM - 1) / (16 * BIG_WM), p.ksplit);
  hipLaunchKernelGGL((gemm_big_kernel<DT, SDT, BIG_WM, BIG_WN, BIG_KPS, false>), grid, dim3(256), 0, s, p);
  if (p.ksplit > 1) {
    const int64_t mn = static_cast<int64_t>(p.M) * p.N;
    hipLaunchKernelGGL(splitk_reduce_kernel<DT>, dim3(static_cast<unsigned>((mn / 4 + 255) / 256)), dim3(256), 0,
                       s, p);
  }
}

template <int DT, int SDT>
void launch_gptq(const GemmParams &p, const Plan &sp, hipStream_t s) {
  if (sp.regime == OC_REGIME_DOT) launch_dot<DT, SDT>(p, sp, s);
  else if (sp.regime == OC_REGIME_SPLITK) launch_mfma<DT, SDT>(p, sp.mt, s);
  else if (sp.big) launch_big<DT, SDT>(p, s);
  else launch_tiled<DT, SDT, FMT_GPTQ>(p, sp.tile, s);
}

// 8-bit GPTQ and DSV4 layers run the LDS-tiled kernel at every M: the largest tile shape
// whose grid fills the chip, K split over fp32 partials when even 64 x 64
// tiles leave it short (act-order rows gathered into the workspace first).
Plan plan_tiled_only(int M, int N, int K_phys, bool has_kmap) {
  Plan sp{};
  sp.regime = OC_REGIME_TILED;
  sp.tile = pick_tiles(M, N, K_phys / 32, &sp.ksplit, &sp.ksteps_per_split);
  sp.gather = has_kmap;
  return sp;
}

// 8-bit GPTQ: batches of up to 16 rows on the balanced-range kernel's global
// form (exact dequantization, MFMA; act-order rows gathered first) where it
// applies (power-of-two group steps; ONECOMP_HIP_GEMV_STREAM=0, read per
// call, keeps them on the tiled kernel), else the tiled kernel.
Plan plan_int8(int M, int N, int K_phys, int group_rows, bool has_kmap) {
  Plan sp = plan_tiled_only(M, N, K_phys, has_kmap);
  if (M <= 16 && ilog2_exact(group_rows / 32) >= 0 && env_int("ONECOMP_HIP_GEMV_STREAM", 1) != 0) {
    const int nwg = gemv_stream_global8_wgs(M, N, K_phys / 32, device_cus(), COUNTER_BYTES);
    if (nwg > 0) {
      sp.regime = OC_REGIME_SPLITK;
      sp.stream_wgs = nwg;
      sp.stream_global = true;
      sp.ksplit = 1;
      sp.ksteps_per_split = K_phys / 32;
    }
  }
  return sp;
}

void plan_tiled(int M, int N, int K, int *wm, int *wn, int *kg, int *ksplit, int *ksteps_per_split) {
  const Plan sp = plan_tiled_only(M, N, K, false);
  *wm = sp.tile.wm;
  *wn = sp.tile.wn;
  *kg = sp.tile.kg;
  *ksplit = sp.ksplit;
  *ksteps_per_split = sp.ksteps_per_split;
}

void launch_rtn_tiled(const GemmParams &p, int x_dtype, bool transposed, int wm, int wn, int kg, hipStream_t s) {
  const TileCfg c{wm, wn, kg};
  const bool bf = x_dtype == OC_DTYPE_BF16;
  if (transposed) {
    if (bf) launch_tiled<OC_DTYPE_BF16, OC_DTYPE_F16, FMT_RTN_T>(p, c, s);
    else launch_tiled<OC_DTYPE_F16, OC_DTYPE_F16, FMT_RTN_T>(p, c, s);
  } else {
    if (bf) launch_tiled<OC_DTYPE_BF16, OC_DTYPE_F16, FMT_RTN>(p, c, s);
    else launch_tiled<OC_DTYPE_F16, OC_DTYPE_F16, FMT_RTN>(p, c, s);
  }
}

}  // namespace oc

using namespace oc;

extern "C" {

size_t oc_int8_gemm_workspace_bytes(int32_t M, int32_t N, int32_t K_phys, int32_t group_rows, int32_t has_kmap) {
  if (M <= 0 || N <= 0 || K_phys <= 0 || group_rows <= 0) return 0;
  return workspace_bytes(plan_int8(M, N, K_phys, group_rows, has_kmap != 0), M, N, K_phys);
}

int oc_int8_gemm(const void *a, int64_t lda, int32_t a_dtype, int32_t M, int32_t K_logical, const int32_t *qt,
                 const void *st, int32_t scale_dtype, const int32_t *zt, int32_t N, int32_t K_phys,
                 int32_t group_rows, const int32_t *kmap, const uint16_t *kinv, const void *bias,
                 int32_t bias_dtype, void *c, int64_t ldc, void *workspace, size_t workspace_bytes_given,
                 void *stream) {
  clear_error();
  if (M < 0 || N <= 0 || K_phys <= 0 || K_logical <= 0)
    return fail(OC_ERR_SHAPE, "bad shape M=%d N=%d K_logical=%d K_phys=%d", M, N, K_logical, K_phys);
  if (M == 0) return OC_OK;
  if (!a || !qt || !st || !zt || !c) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(a_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "a_dtype must be F16 or BF16");
  if (!is_half_dtype(scale_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "scale_dtype must be F16 or BF16");
  if (bias && !is_float_dtype(bias_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "bad bias dtype");
  if (N % 4 != 0) return fail(OC_ERR_SHAPE, "N must be a multiple of 4 (8-bit qzeros packing), got N=%d", N);
  if (K_phys % 32 != 0 || group_rows <= 0 || group_rows % 32 != 0 || K_phys % group_rows != 0)
    return fail(OC_ERR_SHAPE, "K_phys=%d / group_rows=%d must be multiples of 32 with K_phys %% group_rows == 0",
                K_phys, group_rows);
  if (!kmap && K_logical != K_phys)
    return fail(OC_ERR_SHAPE, "K_logical=%d != K_phys=%d requires a kmap", K_logical, K_phys);
  if (lda < K_logical || ldc < N) return fail(OC_ERR_SHAPE, "lda/ldc smaller than the row length");
  if (lda % 8 != 0 || !aligned(a, 16))
    return fail(OC_ERR_SHAPE, "activations need 16-byte aligned rows (lda %% 8 == 0)");
  if (!aligned(qt, 16) || !aligned(kmap, 16) || !aligned(kinv, 16))
    return fail(OC_ERR_SHAPE, "qweight, kmap and kinv must be 16-byte aligned");
  const int64_t tiles = (N + TILE_N - 1) / TILE_N;
  if (tiles * (K_phys / 32) * 512 >= (1LL << 31))
    return fail(OC_ERR_UNSUPPORTED, "layer too large: packed words of 2 GiB or more");
  Plan sp = plan_int8(M, N, K_phys, group_rows, kmap != nullptr);
  // The global form addresses activation rows with 32-bit offsets.
  if (sp.stream_wgs > 0 && (static_cast<int64_t>(M) - 1) * (kmap ? K_phys : lda) * 2 + K_phys * 2 >= (int64_t{1} << 31))
    sp = plan_tiled_only(M, N, K_phys, kmap != nullptr);
  const size_t need = workspace_bytes(sp, M, N, K_phys);
  if (need > 0) {
    if (!workspace || workspace_bytes_given < need)
      return fail(OC_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                  workspace ? workspace_bytes_given : static_cast<size_t>(0));
    if (!aligned(workspace, 256)) return fail(OC_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  GemmParams p{};
  p.a = a;
  p.lda = lda;
  p.M = M;
  p.K_logical = K_logical;
  p.qw = qt;
  p.scales = st;
  p.zeros = zt;
  p.N = N;
  p.K_phys = K_phys;
  p.KS = K_phys / 32;
  p.G = K_phys / group_rows;
  p.group_rows = group_rows;
  p.gshift = ilog2_exact(group_rows / 32);
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.c = c;
  p.ldc = ldc;
  p.ksplit = sp.ksplit;
  p.ksteps_per_split = sp.ksteps_per_split;
  char *ws_after_counters = need > 0 ? static_cast<char *>(workspace) + COUNTER_BYTES : nullptr;
  if (sp.gather) {
    launch_gather_cols(a, lda, M, K_logical, kmap, kinv, K_phys, ws_after_counters, stream);
    p.a = ws_after_counters;
    p.lda = K_phys;
  }
  if (sp.ksplit > 1) p.partials = reinterpret_cast<float *>(ws_after_counters + gather_bytes(sp, M, K_phys));
  const bool bf = a_dtype == OC_DTYPE_BF16, sbf = scale_dtype == OC_DTYPE_BF16;
  if (sp.stream_wgs > 0) {
    p.a_bytes = (static_cast<int64_t>(M) - 1) * p.lda * 2 + static_cast<int64_t>(sp.gather ? K_phys : K_logical) * 2;
    p.counters = static_cast<int *>(workspace);
    launch_gptq8_gemv_stream(p, a_dtype, scale_dtype, sp.stream_wgs, s);
  } else if (bf && sbf) launch_tiled<OC_DTYPE_BF16, OC_DTYPE_BF16, FMT_GPTQ8>(p, sp.tile, s);
  else if (bf) launch_tiled<OC_DTYPE_BF16, OC_DTYPE_F16, FMT_GPTQ8>(p, sp.tile, s);
  else if (sbf) launch_tiled<OC_DTYPE_F16, OC_DTYPE_BF16, FMT_GPTQ8>(p, sp.tile, s);
  else launch_tiled<OC_DTYPE_F16, OC_DTYPE_F16, FMT_GPTQ8>(p, sp.tile, s);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

size_t oc_dsv4_gemm_workspace_bytes(int32_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 32 != 0) return 0;
  return workspace_bytes(plan_tiled_only(M, N, K, false), M, N, K);
}

int oc_dsv4_gemm(const void *x, int64_t ldx, int32_t x_dtype, int32_t M, int32_t K, const uint8_t *qweight,
                 int32_t row_bytes, int32_t wbits, const void *scales, int32_t scale_dtype, const void *zeros,
                 int32_t zero_dtype, int32_t groupsize, int64_t sz_stride_n, int64_t sz_stride_g, int32_t N,
                 const void *bias, int32_t bias_dtype, void *c, int64_t ldc, void *workspace,
                 size_t workspace_bytes_given, void *stream) {
  clear_error();
  if (M < 0 || N <= 0 || K <= 0) return fail(OC_ERR_SHAPE, "bad shape M=%d N=%d K=%d", M, N, K);
  if (M == 0) return OC_OK;
  if (!x || !qweight || !scales || !zeros || !c) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (wbits != 2 && wbits != 4) return fail(OC_ERR_INVALID_ARGUMENT, "wbits must be 2 or 4, got %d", wbits);
  if (!is_half_dtype(x_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "x_dtype must be F16 or BF16");
  if (!is_float_dtype(scale_dtype) || !is_float_dtype(zero_dtype))
    return fail(OC_ERR_INVALID_ARGUMENT, "scales and zeros must be F16, BF16 or F32");
  if (bias && !is_float_dtype(bias_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "bad bias dtype");
  const int per = 8 / wbits;
  if (K % 32 != 0 || (groupsize > 0 && groupsize % 8 != 0) || row_bytes < K / per)
    return fail(OC_ERR_UNSUPPORTED,
                "fused DSV4 GEMM needs K %% 32 == 0, groupsize %% 8 == 0 (or per row) and rows of K / %d bytes "
                "(K=%d groupsize=%d row_bytes=%d)", per, K, groupsize, row_bytes);
  if (row_bytes % (wbits == 4 ? 4 : 2) != 0 || !aligned(qweight, 4))
    return fail(OC_ERR_SHAPE, "qweight rows must be %d-byte aligned", wbits == 4 ? 4 : 2);
  if (ldx % 8 != 0 || !aligned(x, 16) || ldx < K || ldc < N)
    return fail(OC_ERR_SHAPE, "x needs 16-byte aligned rows (ldx %% 8 == 0)");
  const Plan sp = plan_tiled_only(M, N, K, false);
  const size_t need = workspace_bytes(sp, M, N, K);
  if (need > 0) {
    if (!workspace || workspace_bytes_given < need)
      return fail(OC_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                  workspace ? workspace_bytes_given : static_cast<size_t>(0));
    if (!aligned(workspace, 256)) return fail(OC_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  }
  GemmParams p{};
  p.a = x;
  p.lda = ldx;
  p.M = M;
  p.K_logical = K;
  p.qw = qweight;
  p.scales = scales;
  p.zeros = zeros;
  p.scale_dtype = scale_dtype;
  p.zero_dtype = zero_dtype;
  p.rtn_gs = groupsize > 0 ? groupsize : K;  // per row: one group spanning K
  p.row_bytes = row_bytes;
  p.sz_stride_n = sz_stride_n;
  p.sz_stride_g = groupsize > 0 ? sz_stride_g : 0;
  p.N = N;
  p.K_phys = K;
  p.KS = K / 32;
  p.group_rows = 32;
  p.gshift = 0;
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.c = c;
  p.ldc = ldc;
  p.ksplit = sp.ksplit;
  p.ksteps_per_split = sp.ksteps_per_split;
  if (sp.ksplit > 1) p.partials = reinterpret_cast<float *>(static_cast<char *>(workspace) + COUNTER_BYTES);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf = x_dtype == OC_DTYPE_BF16;
  if (rows_gemv_applies(M, K, p.rtn_gs, wbits, scale_dtype, zero_dtype, row_bytes, qweight)) {
    launch_rows_gemv(p, x_dtype, wbits == 4 ? FMT_DSV4_4 : FMT_DSV4_2, s);
  } else if (wbits == 4) {
    if (bf) launch_tiled<OC_DTYPE_BF16, OC_DTYPE_F16, FMT_DSV4_4>(p, sp.tile, s);
    else launch_tiled<OC_DTYPE_F16, OC_DTYPE_F16, FMT_DSV4_4>(p, sp.tile, s);
  } else {
    if (bf) launch_tiled<OC_DTYPE_BF16, OC_DTYPE_F16, FMT_DSV4_2>(p, sp.tile, s);
    else launch_tiled<OC_DTYPE_F16, OC_DTYPE_F16, FMT_DSV4_2>(p, sp.tile, s);
  }
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

size_t oc_int4_gemm_workspace_bytes(int32_t M, int32_t N, int32_t K_phys, int32_t group_rows, int32_t has_kmap,
                                    int32_t regime) {
  if (M <= 0 || N <= 0 || K_phys <= 0 || group_rows <= 0) return 0;
  // With a kmap the plan depends on whether kinv is given: cover both.
  const size_t with_kinv = workspace_bytes(plan_gemm(M, N, K_phys, group_rows, has_kmap != 0, regime), M, N, K_phys);
  if (!has_kmap) return with_kinv;
  return std::max(with_kinv, workspace_bytes(plan_gemm(M, N, K_phys, group_rows, true, regime, false), M, N, K_phys));
}

}  // extern "C"

namespace oc {

int gemm_impl(const void *a, int64_t lda, int32_t a_dtype, int32_t M, int32_t K_logical, const int32_t *qt,
              const void *st, int32_t scale_dtype, const int32_t *zt, int32_t N, int32_t K_phys,
              int32_t group_rows, const int32_t *kmap, const uint16_t *kinv, const void *bias,
              int32_t bias_dtype, void *c, int64_t ldc, WorkspaceArg ws, int32_t regime, void *stream) {
  void *workspace = ws.ptr;
  const size_t workspace_bytes_given = ws.bytes;
  if (M < 0 || N <= 0 || K_phys <= 0 || K_logical <= 0)
    return fail(OC_ERR_SHAPE, "bad shape M=%d N=%d K_logical=%d K_phys=%d", M, N, K_logical, K_phys);
  if (M == 0) return OC_OK;
  if (!a || !qt || !st || !zt || !c) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(a_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "a_dtype must be F16 or BF16");
  if (!is_half_dtype(scale_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "scale_dtype must be F16 or BF16");
  if (bias && !is_float_dtype(bias_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "bad bias dtype");
  if (regime < OC_REGIME_AUTO || regime > OC_REGIME_DOT)
    return fail(OC_ERR_INVALID_ARGUMENT, "unknown regime %d", regime);
  if (N % 8 != 0) return fail(OC_ERR_SHAPE, "N must be a multiple of 8 (qzeros packing), got N=%d", N);
  if (K_phys % 32 != 0 || group_rows <= 0 || group_rows % 32 != 0 || K_phys % group_rows != 0)
    return fail(OC_ERR_SHAPE, "K_phys=%d / group_rows=%d must be multiples of 32 with K_phys %% group_rows == 0",
                K_phys, group_rows);
  if (!kmap && K_logical != K_phys)
    return fail(OC_ERR_SHAPE, "K_logical=%d != K_phys=%d requires a kmap", K_logical, K_phys);
  if (lda < K_logical || ldc < N) return fail(OC_ERR_SHAPE, "lda/ldc smaller than the row length");
  if (lda % 8 != 0 || !aligned(a, 16))
    return fail(OC_ERR_SHAPE, "activations need 16-byte aligned rows (lda %% 8 == 0)");
  if (!aligned(qt, 16) || !aligned(kmap, 16) || !aligned(kinv, 16))
    return fail(OC_ERR_SHAPE, "qweight, kmap and kinv must be 16-byte aligned");
  const int64_t tiles = (N + TILE_N - 1) / TILE_N;
  if (tiles * (K_phys / 32) * 256 >= (1LL << 31))  // kernels address the words with 32-bit byte offsets
    return fail(OC_ERR_UNSUPPORTED, "layer too large: packed words of 2 GiB or more");
  if (regime == OC_REGIME_SPLITK && M > 64)
    return fail(OC_ERR_UNSUPPORTED, "small-M regime supports M <= 64, got M=%d", M);
  if (regime == OC_REGIME_DOT && !dot_eligible(M, K_phys, group_rows))
    return fail(OC_ERR_UNSUPPORTED, "decode regime needs M <= 2 and group_rows/32 a power of two (M=%d group_rows=%d)",
                M, group_rows);

  const Plan sp = plan_gemm(M, N, K_phys, group_rows, kmap != nullptr, regime, kinv != nullptr, lda);
  const size_t need = workspace_bytes(sp, M, N, K_phys);
  if (ws.scratch_cap > 0 && need > ws.scratch_cap)
    return fail(OC_ERR_WORKSPACE, "this call needs %zu bytes of scratch; the static scratch holds %zu", need,
                ws.scratch_cap);
  if (need > 0) {
    if (!workspace || workspace_bytes_given < need)
      return fail(OC_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                  workspace ? workspace_bytes_given : static_cast<size_t>(0));
    if (!aligned(workspace, 256)) return fail(OC_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  GemmParams p{};
  p.a = a;
  p.lda = lda;
  p.M = M;
  p.K_logical = K_logical;
  p.qw = qt;
  p.scales = st;
  p.zeros = zt;
  p.N = N;
  p.K_phys = K_phys;
  p.KS = K_phys / 32;
  p.G = K_phys / group_rows;
  p.group_rows = group_rows;
  p.gshift = ilog2_exact(group_rows / 32);
  p.kinv = (sp.regime == OC_REGIME_DOT || (sp.stream_wgs > 0 && !sp.stream_global)) && kmap ? kinv : nullptr;
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.c = c;
  p.ldc = ldc;
  p.ksplit = sp.ksplit;
  p.ksteps_per_split = sp.ksteps_per_split;
  char *ws_after_counters = need > 0 ? static_cast<char *>(workspace) + COUNTER_BYTES : nullptr;
  if (sp.gather) {
    launch_gather_cols(a, lda, M, K_logical, kmap, kinv, K_phys, ws_after_counters, stream);
    p.a = ws_after_counters;
    p.lda = K_phys;
  }
  p.a_bytes = (static_cast<int64_t>(M) - 1) * p.lda * 2 + static_cast<int64_t>(sp.gather ? K_phys : K_logical) * 2;
  // The whole-tile MFMA kernel addresses activation rows with 32-bit offsets.
  if (sp.regime == OC_REGIME_SPLITK && (sp.stream_wgs == 0 || sp.stream_global) && p.a_bytes >= (int64_t{1} << 31))
    return fail(OC_ERR_SHAPE, "activation rows span %lld bytes (2 GiB or more): pass a compact copy",
                static_cast<long long>(p.a_bytes));
  if (sp.ksplit > 1) p.partials = reinterpret_cast<float *>(ws_after_counters + gather_bytes(sp, M, K_phys));
  p.kmap = kmap;
  p.counters = need > 0 ? static_cast<int *>(workspace) : nullptr;
  const bool bf = a_dtype == OC_DTYPE_BF16, sbf = scale_dtype == OC_DTYPE_BF16;
  if (sp.stream_wgs > 0) launch_gptq_gemv_stream(p, a_dtype, scale_dtype, sp.stream_wgs, sp.stream_global, s);
  else if (sp.regime == OC_REGIME_DOT && !sp.legacy_dot) launch_gptq_gemv(p, a_dtype, scale_dtype, sp.gv.T, s);
  else if (sp.wide_wn) launch_gptq_wide(p, a_dtype, scale_dtype, sp.wide_wn, s);
  else if (bf && sbf) launch_gptq<OC_DTYPE_BF16, OC_DTYPE_BF16>(p, sp, s);
  else if (bf) launch_gptq<OC_DTYPE_BF16, OC_DTYPE_F16>(p, sp, s);
  else if (sbf) launch_gptq<OC_DTYPE_F16, OC_DTYPE_BF16>(p, sp, s);
  else launch_gptq<OC_DTYPE_F16, OC_DTYPE_F16>(p, sp, s);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

}  // namespace oc

extern "C" {

int oc_int4_gemm(const void *a, int64_t lda, int32_t a_dtype, int32_t M, int32_t K_logical, const int32_t *qt,
                 const void *st, int32_t scale_dtype, const int32_t *zt, int32_t N, int32_t K_phys,
                 int32_t group_rows, const int32_t *kmap, const uint16_t *kinv, const void *bias,
                 int32_t bias_dtype, void *c, int64_t ldc, void *workspace, size_t workspace_bytes_given,
                 int32_t regime, void *stream) {
  clear_error();
  return gemm_impl(a, lda, a_dtype, M, K_logical, qt, st, scale_dtype, zt, N, K_phys, group_rows, kmap, kinv,
                   bias, bias_dtype, c, ldc, WorkspaceArg{workspace, workspace_bytes_given, 0}, regime, stream);
}

int oc_rtn_linear(const void *x, int64_t ldx, int32_t x_dtype, int32_t M, int32_t K, const uint8_t *qweight_u8,
                  int32_t row_bytes, const void *scales, int32_t scale_dtype, const void *zeros, int32_t zero_dtype,
                  int32_t G, int32_t N, const void *bias, int32_t bias_dtype, void *c, int64_t ldc, void *stream) {
  clear_error();
  if (M < 0 || N <= 0 || K <= 0 || G <= 0) return fail(OC_ERR_SHAPE, "bad shape M=%d N=%d K=%d G=%d", M, N, K, G);
  if (M == 0) return OC_OK;
  if (!x || !qweight_u8 || !scales || !zeros || !c) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(x_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "x_dtype must be F16 or BF16");
  if (!is_float_dtype(scale_dtype) || dtype_bytes(zero_dtype) == 0)
    return fail(OC_ERR_INVALID_ARGUMENT, "unsupported scale/zero dtype");
  if (bias && !is_float_dtype(bias_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "bad bias dtype");
  if (K % G != 0) return fail(OC_ERR_SHAPE, "in_features=%d not divisible by num_groups=%d", K, G);
  if (K % 32 != 0 || (K / G) % 8 != 0 || row_bytes < K / 2 || row_bytes % 4 != 0 || N % 8 != 0)
    return fail(OC_ERR_UNSUPPORTED,
                "fused RTN linear needs K %% 32 == 0, (K/G) %% 8 == 0, N %% 8 == 0 and 4-byte rows "
                "(K=%d G=%d N=%d row_bytes=%d)",
                K, G, N, row_bytes);
  if (ldx % 8 != 0 || !aligned(x, 16) || !aligned(qweight_u8, 4) || ldx < K || ldc < N)
    return fail(OC_ERR_SHAPE, "x needs 16-byte aligned rows and qweight 4-byte aligned rows");

  // Bias is rounded to the activation type first (`bias.to(x.dtype)`); the
  // kernel adds it in fp32, which is exact for a 16-bit value.
  int rtn_ksplit = 1, rtn_kps = K / 32;  // no K split: the layer writes its output directly
  const TileCfg pick = pick_tiles(M, N, K / 32, &rtn_ksplit, &rtn_kps, false);
  GemmParams p{};
  p.a = x;
  p.lda = ldx;
  p.M = M;
  p.K_logical = K;
  p.qw = qweight_u8;
  p.scales = scales;
  p.zeros = zeros;
  p.scale_dtype = scale_dtype;
  p.zero_dtype = zero_dtype;
  p.rtn_G = G;
  p.rtn_gs = K / G;
  p.row_bytes = row_bytes;
  p.sz_stride_n = G;
  p.sz_stride_g = 1;
  p.N = N;
  p.K_phys = K;
  p.KS = K / 32;
  p.group_rows = 32;
  p.gshift = 0;
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.c = c;
  p.ldc = ldc;
  p.ksplit = 1;
  p.ksteps_per_split = K / 32;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (rows_gemv_applies(M, K, K / G, 4, scale_dtype, zero_dtype, row_bytes, qweight_u8))
    launch_rows_gemv(p, x_dtype, FMT_RTN, s);
  else if (x_dtype == OC_DTYPE_BF16) launch_tiled<OC_DTYPE_BF16, OC_DTYPE_F16, FMT_RTN>(p, pick, s);
  else launch_tiled<OC_DTYPE_F16, OC_DTYPE_F16, FMT_RTN>(p, pick, s);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_moe_route(const int64_t *topk_ids, int32_t T, int32_t topk, int32_t E, int32_t *expert_offsets,
                 int32_t *sorted_pairs, void *stream) {
  clear_error();
  if (!topk_ids || !expert_offsets || !sorted_pairs) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (T < 0 || topk <= 0 || E <= 0 || E > 1024 || static_cast<int64_t>(T) * topk > 65536)
    return fail(OC_ERR_SHAPE, "unsupported routing shape T=%d topk=%d E=%d", T, topk, E);
  const size_t lds = sizeof(int32_t) * (ROUTE_WAVES + 1) * E;
  if (lds > 128 * 1024) return fail(OC_ERR_UNSUPPORTED, "too many experts for one workgroup (E=%d)", E);
  if (lds > 64 * 1024)
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(moe_route_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(ROUTE_THREADS), lds, static_cast<hipStream_t>(stream), topk_ids,
                     T * topk, E, expert_offsets, sorted_pairs);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_int4_moe_gemm(const void *x, int64_t ldx, int32_t x_dtype, int32_t T, int32_t topk, int32_t K,
                     const int32_t *qt, const void *st, int32_t scale_dtype, const int32_t *zt, int32_t group_rows,
                     int32_t E, int32_t N, const int32_t *expert_offsets, const int32_t *sorted_pairs, void *y,
                     int64_t ldy, void *stream) {
  clear_error();
  if (T < 0 || topk <= 0 || K <= 0 || E <= 0 || N <= 0) return fail(OC_ERR_SHAPE, "bad shape");
  if (T == 0) return OC_OK;
  if (!x || !qt || !st || !zt || !expert_offsets || !sorted_pairs || !y)
    return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(x_dtype) || !is_half_dtype(scale_dtype))
    return fail(OC_ERR_INVALID_ARGUMENT, "x and scales must be F16 or BF16");
  if (K % 32 != 0 || group_rows <= 0 || group_rows % 32 != 0 || K % group_rows != 0 || N % 64 != 0)
    return fail(OC_ERR_SHAPE, "need K %% 32 == 0, group_rows | K (multiple of 32), N %% 64 == 0");
  if (ldx % 8 != 0 || !aligned(x, 16) || ldx < K || ldy < N) return fail(OC_ERR_SHAPE, "x needs 16-byte aligned rows");
  const int64_t tiles = N / TILE_N;
  if (static_cast<int64_t>(T) * ldx * 2 >= (int64_t{1} << 31) || tiles * (K / 32) * 256 >= (int64_t{1} << 31))
    return fail(OC_ERR_UNSUPPORTED, "grouped GEMM operands exceed 2 GiB per expert / activation block");
  GemmParams p{};
  p.a = x;
  p.lda = ldx;
  p.a_bytes = (static_cast<int64_t>(T) - 1) * ldx * 2 + static_cast<int64_t>(K) * 2;
  p.M = T * topk;
  p.K_logical = K;
  p.qw = qt;
  p.scales = st;
  p.zeros = zt;
  p.N = N;
  p.K_phys = K;
  p.KS = K / 32;
  p.G = K / group_rows;
  p.group_rows = group_rows;
  p.gshift = ilog2_exact(group_rows / 32);
  p.c = y;
  p.ldc = ldy;
  p.ksplit = 1;
  p.ksteps_per_split = K / 32;
  p.expert_offsets = expert_offsets;
  p.sorted_pairs = sorted_pairs;
  p.topk = topk;
  p.qw_expert_stride = tiles * p.KS * 64;
  p.s_expert_stride = tiles * p.G * TILE_N;
  p.z_expert_stride = tiles * p.G * 2;
  const dim3 grid((N + 64 * BIG_WN - 1) / (64 * BIG_WN), 1, E);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf = x_dtype == OC_DTYPE_BF16, sbf = scale_dtype == OC_DTYPE_BF16;
  static const int moe_ns = env_int("ONECOMP_HIP_MOE_NS", MOE_NS);
  if (bf && sbf) launch_moe<OC_DTYPE_BF16, OC_DTYPE_BF16>(p, grid, moe_ns, s);
  else if (bf) launch_moe<OC_DTYPE_BF16, OC_DTYPE_F16>(p, grid, moe_ns, s);
  else if (sbf) launch_moe<OC_DTYPE_F16, OC_DTYPE_BF16>(p, grid, moe_ns, s);
  else launch_moe<OC_DTYPE_F16, OC_DTYPE_F16>(p, grid, moe_ns, s);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

}  // extern "C"
