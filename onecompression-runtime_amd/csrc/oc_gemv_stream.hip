// Small-batch GEMV (M <= 16) as one balanced weight stream per workgroup, for gfx950.
//
// A layer's packed weights are U = tiles x QT units of 1 KB: one 16-column
// tile by four 32-row K steps (QT = ceil(KS / 4) units per tile), stored
// contiguously in unit order by the tile16 layout. Workgroup b of an n-wide
// launch (one per compute unit) owns a contiguous range of floor(U / n) or
// one more units and streams it with 16 waves: wave w takes every 16th unit
// from w, each
// lane one 16-byte load (column c, K step 4 q + h), PF units ahead of use.
// Every compute unit therefore reads the same number of bytes whatever the
// tile count (whole-tile launches leave 320 tiles on 256 CUs doubly loaded),
// and the activation rows are staged into LDS once per workgroup: copied,
// scattered through kinv (act-order, logical -> physical) or gathered
// through kmap (physical -> logical).
//
// A wave accumulates one tile at a time and parks each finished tile's column
// sums in LDS ([tile slot][wave]); after the stream the workgroup adds the
// waves in order and stores the tiles that lie wholly inside its range. The
// host launches at most one workgroup per tile, so every range spans at least
// one tile and a tile cut by a range boundary has exactly two contributors
// (the lower and the upper workgroup). Each hands its fp32 partial to the
// other through one 64-bit atomic swap per value (a presence flag above the
// float's bits) in the workspace's counter area: the second to arrive gets
// the first's partial back, stores lower + upper (the same bits whichever
// arrives first) and clears the cell. One round trip, no ordering waits; the
// cells are zero between calls and across HIP graph replays.
//
// Inner product (as in the whole-tile kernel): scale and zero are factored
// out of each 32-row group,
//   sum_k x_k s (w_k - z) = s (sum_k x_k (B + w_k) - (B + z) sum_k x_k),
// with B + w_k the exact 16-bit number made by OR-ing the code into the
// mantissa of B (bf16 128.0, fp16 1024.0) and the second sum from per-step
// activation sums staged beside the activation pairs. The first sum:
//  * M <= 2: v_dot2_f32_{bf16,f16} per lane against activation pairs in LDS;
//  * 3 <= M <= 16 (MR = 4, 8 or 16 staged rows): one v_mfma_f32_16x16x32 per
//    K step. Lane (g, c) loads octet g of each of the unit's four steps
//    (four 4-byte loads; a wave instruction reads 256 consecutive bytes),
//    which is the B operand layout of one MFMA per step (column c, K rows
//    8 g .. 8 g + 7), against the A operand of lane (g, r): row r's pairs of
//    octet g; output lane (g, c) holds rows 4 g + i. Each step's sum is
//    scaled once per output; the zero term of all four steps is one
//    v_mfma_f32_16x16x4_f32 (lane (g, c) holds the activation sum of row c
//    over step g and -s (B + z) of column c at step g), accumulated apart
//    and added when the tile is parked.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "oc_gemm_common.h"

namespace oc {

namespace {

constexpr int SW = 16;        // waves per workgroup
constexpr int SNT = 64 * SW;  // threads per workgroup
constexpr int SNTL = 8;       // tiles one workgroup's range may touch

// Activation rows: staged into LDS (copied, scattered through kinv, gathered
// through kmap), or read from global memory per unit (SX_GLOBAL: rows already
// in physical order; MFMA form with exact dequantization).
enum { SX_CONTIG = 0, SX_SCATTER = 1, SX_GATHER = 2, SX_GLOBAL = 3 };

// Balanced ranges: U = nwg q + r units; workgroups b < r own q + 1 units,
// the others q (q >= QT: the host launches at most one workgroup per tile).
__host__ __device__ __forceinline__ int range_start(int b, int q, int r) { return b * q + (b < r ? b : r); }

// Rows staged per launch: M itself for the dot2 path, else the next of 4, 8, 16.
int stream_rows(int M) { return M <= 2 ? M : M <= 4 ? 4 : M <= 8 ? 8 : M <= 16 ? 16 : 0; }

// Most tiles any workgroup's range touches (its LDS tile slots).
int stream_slots(int64_t tiles, int QT, int nwg) {
  const int U = static_cast<int>(tiles * QT), q = U / nwg, r = U % nwg;
  int most = 0;
  for (int b = 0; b < nwg; ++b) {
    const int u0 = range_start(b, q, r), u1 = range_start(b + 1, q, r);
    most = std::max(most, (u1 - 1) / QT - u0 / QT + 1);
  }
  return most;
}

}  // namespace

// AL: K steps per tile a multiple of 4, so unit u starts at byte 1024 u of
// the tile16 words (2048 u for 8-bit) and at group (4 u) >> gshift of the
// scales and zeros. WB: code bits, 4 (tile16) or 8 (tile16x8: global form
// only; a column's K step is 8 words, 32 bytes, 4 zero bytes per word).
template <int DT, int SDT, int MR, int SX, int PF, bool AL, int WB = 4>
__global__ __launch_bounds__(SNT) void gemv_stream_kernel(GemmParams p) {
  constexpr uint32_t MAGIC = DT == OC_DTYPE_BF16 ? 0x43004300u : 0x64006400u;
  constexpr bool MF = MR > 2;     // MFMA inner product (rows 4 g + i of lane (g, c))
  constexpr bool GL = SX == SX_GLOBAL;  // activations from global memory, nothing staged
  constexpr int SB = MF ? 1 : 3;  // staged octets per thread per batch
  static_assert(!MF || MR == 4 || MR == 8 || MR == 16, "MFMA rows");
  static_assert(!GL || MF, "global activation rows take the MFMA form");
  static_assert(WB == 4 || (WB == 8 && GL), "8-bit codes take the global form");
  constexpr uint32_t STEPB = WB == 8 ? 512u : 256u;  // bytes of one tile and K step
  constexpr uint32_t ZSTR = WB == 8 ? 16u : 8u;      // zero bytes of one tile and group
  extern __shared__ __attribute__((aligned(16))) uint4 sx_lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, h = lane >> 4;
  const int KS = p.KS, QT = (KS + 3) >> 2, KS4 = 4 * QT;  // LDS rows padded to whole units
  const int M = p.M;
  const int tiles = (p.N + TILE_N - 1) / TILE_N;
  const int U = tiles * QT;  // < 2^21 (host: packed words below 2 GiB)
  const int nwg = gridDim.x, b = blockIdx.x;
  const int rq = U / nwg, rm = U % nwg;
  const int u0 = range_start(b, rq, rm), u1 = range_start(b + 1, rq, rm);
  const int t_first = u0 / QT, t_last = (u1 - 1) / QT;
  const int nslots = p.stream_slots;                                 // tiles a range touches, at most
  // Row stride of the staged pairs, in 16-byte chunks: the MFMA form reads
  // 16 rows at once and pads each row by one chunk (distinct banks).
  const int RS = GL ? 0 : 4 * KS4 + (MF ? 1 : 0);
  uint4 *xpairs = sx_lds;                                          // [MR][RS]
  float2 *xsum = reinterpret_cast<float2 *>(sx_lds + MR * RS);  // dot2: [MR][KS4] (sum, B * sum)
  float *xst = reinterpret_cast<float *>(sx_lds + MR * RS);     // MFMA: [KS4][MR] sums
  float *red = MF ? xst + (GL ? 0 : KS4 * MR) : reinterpret_cast<float *>(xsum + MR * KS4);  // [nslots][SW][MR][16]
  // 16-bit slot that takes the scatter's writes for rows without a place.
  const int trash16 = static_cast<int>(reinterpret_cast<uint16_t *>(red + nslots * SW * MR * 16) -
                                       reinterpret_cast<uint16_t *>(xpairs));
  // Step sum of row m, K step ks.
  auto put_sum = [&](int m, int ks, float sum) {
    if constexpr (MF) xst[ks * MR + m] = sum;
    else xsum[m * KS4 + ks] = make_float2(sum, dot_base<DT>() * sum);
  };

  // ---- activation staging, batch by batch, before the weight stream ----
  const uint16_t *a = static_cast<const uint16_t *>(p.a);
  const int n_items = GL ? 0 : SX == SX_SCATTER ? (p.K_logical >> 3) : KS * 4;  // octets to stage
  const uint4 *kinv4 = reinterpret_cast<const uint4 *>(p.kinv);
  uint4 xr[MR][SB];
  uint4 rr[SB];
  auto stage_load = [&](int base) {
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      // Waves wholly past the end load nothing (their registers are never
      // stored); the lanes of a wave past the end read the last octet.
      // (Every workgroup stages the same rows at once: whole waves of
      // redundant loads of one line queue on one L2 channel. Measured on the
      // K = 5120 decode layers, 640 octets in 3 x 1024 slots: -0.3 us.)
      if (base + SNT * u + (tid & ~63) >= n_items) {
#pragma unroll
        for (int m = 0; m < MR; ++m) xr[m][u] = make_uint4(0, 0, 0, 0);
        rr[u] = make_uint4(0, 0, 0, 0);
        continue;
      }
      const int ic = min(base + SNT * u + tid, n_items - 1);
      if constexpr (SX == SX_GATHER) {
        const int4 k0 = *reinterpret_cast<const int4 *>(p.kmap + 8 * ic);
        const int4 k1 = *reinterpret_cast<const int4 *>(p.kmap + 8 * ic + 4);
        const int kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const uint16_t *arow = a + static_cast<int64_t>(min(m, M - 1)) * p.lda;
          uint32_t v[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = arow[max(kk[i], 0)];
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (kk[i] < 0) v[i] = 0u;  // padding row
          xr[m][u] = make_uint4(v[0] | v[1] << 16, v[2] | v[3] << 16, v[4] | v[5] << 16, v[6] | v[7] << 16);
        }
      } else {
        if constexpr (SX == SX_SCATTER) rr[u] = kinv4[ic];
#pragma unroll
        for (int m = 0; m < MR; ++m)
          xr[m][u] = reinterpret_cast<const uint4 *>(a + static_cast<int64_t>(min(m, M - 1)) * p.lda)[ic];
      }
    }
  };
  auto stage_store = [&](int base) {
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int i = base + SNT * u + tid;
      if constexpr (SX == SX_SCATTER) {
        // Branch-free within a wave: an octet past the end or a row without
        // a physical place writes the trash slot; waves wholly past the end
        // skip the slot.
        if (base + SNT * u + (tid & ~63) >= n_items) continue;
        uint16_t *x16 = reinterpret_cast<uint16_t *>(xpairs);
        const int K_phys = i < n_items ? p.K_phys : 0;
        const uint32_t rw[4] = {rr[u].x, rr[u].y, rr[u].z, rr[u].w};
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const uint32_t xw[4] = {xr[m][u].x, xr[m][u].y, xr[m][u].z, xr[m][u].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r0 = static_cast<int>(rw[j] & 0xFFFFu), r1 = static_cast<int>(rw[j] >> 16);
            x16[r0 < K_phys ? xpair_slot(m, 8 * RS, r0) : trash16] = static_cast<uint16_t>(xw[j]);
            x16[r1 < K_phys ? xpair_slot(m, 8 * RS, r1) : trash16] = static_cast<uint16_t>(xw[j] >> 16);
          }
        }
      } else {
        // The 4 octets of a K step sit in 4 consecutive lanes, which add up the step's sum.
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          float sum;
          const uint4 pr = octet_pairs<DT>(xr[m][u], sum);
          sum += __shfl_xor(sum, 1);
          sum += __shfl_xor(sum, 2);
          if (i < n_items) {
            xpairs[m * RS + i] = pr;
            if ((i & 3) == 0) put_sum(m, i >> 2, sum);
          }
        }
      }
    }
  };
  auto scatter_tail = [&]() {  // act-order rows beyond the last whole octet, one by one
    if constexpr (SX == SX_SCATTER) {
      uint16_t *x16 = reinterpret_cast<uint16_t *>(xpairs);
      for (int k = 8 * n_items + tid; k < p.K_logical; k += SNT) {
        const int r = p.kinv[k];
        if (r < p.K_phys) {
#pragma unroll
          for (int m = 0; m < MR; ++m)
            x16[xpair_slot(m, 8 * RS, r)] = a[static_cast<int64_t>(min(m, M - 1)) * p.lda + k];
        }
      }
    }
  };
  // One batch covers the rows (the common case): its loads go out first, the
  // LDS zeroing below runs while they are in flight, and they are stored
  // before the weight prefetch is issued. Longer or ragged rows are staged
  // batch by batch.
  const bool one_batch = n_items <= SNT * SB && (SX != SX_SCATTER || (p.K_logical & 7) == 0);
  if (one_batch && n_items > 0) stage_load(0);

  // Zeros (while the activations load): the parked tile sums, and the
  // padding steps [KS, KS4) of every row (a unit's lanes past the last K
  // step multiply zeros).
  for (int i = tid; i < nslots * SW * MR * 16; i += SNT) red[i] = 0.f;
  if constexpr (!GL) {
    const int pad = 4 * (KS4 - KS);
    for (int i = tid; i < MR * pad; i += SNT) {
      const int m = i / pad, j = i - m * pad;
      xpairs[m * RS + KS * 4 + j] = make_uint4(0, 0, 0, 0);
      if (j < KS4 - KS) put_sum(m, KS + j, 0.f);
    }
  }
  if constexpr (SX == SX_SCATTER) {
    if (p.K_logical != p.K_phys) {  // physical rows without a source stay zero
      for (int i = tid; i < MR * RS; i += SNT) xpairs[i] = make_uint4(0, 0, 0, 0);
      barrier_no_fence();
    }
  }
  if (!one_batch) {
    for (int base = 0; base < n_items; base += SNT * SB) {
      stage_load(base);
      stage_store(base);
    }
    scatter_tail();
  }

  // ---- weight stream: producer position (wave-uniform) and its prefetch ----
  // dot2 form: lane (h, c) loads the four octets of K step 4 q + h of
  // column c (16 bytes) and that step's scale and zero word. MFMA form: lane
  // (h, c) loads octet h of each of the four steps (four 4-byte loads, each
  // wave instruction 256 consecutive bytes), the four steps' scales of
  // column c, and the zero word of its own step h (for the zero term).
  struct StageDot {
    uint4 q;
    uint32_t s;
    uint32_t z;
  };
  struct StageMf {
    uint32_t q[4];
    uint32_t s[4];
    uint32_t z;
  };
  // Global form: the dot2 form's weight loads (8-bit: two 16-byte loads, the
  // column's 8 words of the step) plus the A operand of lane (h, r): row r's
  // 32 activations of K step 4 q + h (four 16-byte loads).
  struct StageGl {
    uint4 q;
    uint4 q2;
    uint32_t s;
    uint32_t z;
    uint32_t x[16];
  };
  using Stage = std::conditional_t<GL, StageGl, std::conditional_t<MF, StageMf, StageDot>>;
  // Buffer loads: a wave-uniform unit offset plus a fixed per-lane offset.
  // Lanes past a tile's last K step read the next tile (or past the end:
  // zero), which meets the zero padding of the staged activations; units
  // past the wave's range get an offset beyond every buffer (zero, no
  // memory access).
  const int G = p.G, gshift = p.gshift, gs2 = min(gshift, 2);
  const __amdgpu_buffer_rsrc_t q_rs = buffer_rsrc(p.qw, static_cast<int64_t>(tiles) * KS * STEPB);
  const __amdgpu_buffer_rsrc_t s_rs = buffer_rsrc(p.scales, static_cast<int64_t>(tiles) * G * 32);
  const __amdgpu_buffer_rsrc_t z_rs = buffer_rsrc(p.zeros, static_cast<int64_t>(tiles) * G * ZSTR);
  constexpr bool MFL = MF && !GL;  // per-octet weight loads (staged MFMA form)
  const uint32_t q_lane = MFL ? static_cast<uint32_t>(c * 16 + 4 * h)
                              : WB == 8 ? static_cast<uint32_t>(512 * h + 32 * c) : lane * 16u;  // + 256 j (MFMA form)
  const uint32_t s_lane = MFL ? static_cast<uint32_t>(c) * 2u                          // + 32 (j >> gs2)
                              : static_cast<uint32_t>((h >> gs2) * 16 + c) * 2u;      // group of K step 4 q + h
  // Global form: row c of the activations (rows past M read nowhere).
  const __amdgpu_buffer_rsrc_t a_rs = buffer_rsrc(p.a, GL ? p.a_bytes : 0);
  const uint32_t a_row = GL && c < M ? static_cast<uint32_t>(c * p.lda * 2) : 0xFFFFF000u;
  const uint32_t z_lane = WB == 8 ? static_cast<uint32_t>((h >> gs2) * 4 + (c >> 2)) * 4u
                                  : static_cast<uint32_t>((h >> gs2) * 2 + (c >> 3)) * 4u;
  constexpr uint32_t NOWHERE = 0xFFFFF000u;
  const int w_u0 = u0 + wave;  // this wave's first unit; it takes every SW-th from there
  int pu = w_u0;               // producer: next unit to load
  auto load = [&](Stage &S) {
    uint32_t qb, gb;
    if constexpr (AL) {
      qb = static_cast<uint32_t>(pu) * (4 * STEPB);
      gb = static_cast<uint32_t>(4 * pu) >> gshift;
    } else {
      const int tt = pu / QT, qq = pu - tt * QT;
      qb = static_cast<uint32_t>(tt * KS + 4 * qq) * STEPB;
      gb = static_cast<uint32_t>(tt * G + ((4 * qq) >> gshift));
    }
    const bool in = pu < u1;
    const uint32_t qo = q_lane + (in ? qb : NOWHERE), so = s_lane + (in ? gb * 32u : NOWHERE);
    if constexpr (GL) {
      const auto q = __builtin_amdgcn_raw_buffer_load_b128(q_rs, qo, 0,CPOL_WEIGHT_STREAM);
      S.q = make_uint4(q[0], q[1], q[2], q[3]);
      if constexpr (WB == 8) {
        const auto q2 = __builtin_amdgcn_raw_buffer_load_b128(q_rs, qo, 16, CPOL_WEIGHT_STREAM);
        S.q2 = make_uint4(q2[0], q2[1], q2[2], q2[3]);
      } else {
        S.q2 = make_uint4(0, 0, 0, 0);
      }
      S.s = __builtin_amdgcn_raw_buffer_load_b16(s_rs, so, 0,CPOL_WEIGHT_STREAM);
      const int ks = 4 * (pu % QT) + h;  // this lane's K step (steps past KS read zeros)
      const bool a_in = in && ks < KS && a_row != NOWHERE;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(a_rs, a_in ? a_row + 64u * ks + 16u * j : NOWHERE, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) S.x[4 * j + e] = v[e];
      }
    } else if constexpr (MF) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        S.q[j] = __builtin_amdgcn_raw_buffer_load_b32(q_rs, qo + 256u * j, 0,CPOL_WEIGHT_STREAM);
        S.s[j] = __builtin_amdgcn_raw_buffer_load_b16(s_rs, so, 32 * (j >> gs2),CPOL_WEIGHT_STREAM);
      }
    } else {
      const auto q = __builtin_amdgcn_raw_buffer_load_b128(q_rs, qo, 0,CPOL_WEIGHT_STREAM);
      S.q = make_uint4(q[0], q[1], q[2], q[3]);
      S.s = __builtin_amdgcn_raw_buffer_load_b16(s_rs, so, 0,CPOL_WEIGHT_STREAM);
    }
    S.z = __builtin_amdgcn_raw_buffer_load_b32(z_rs, z_lane + (in ? gb * ZSTR : NOWHERE), 0,CPOL_WEIGHT_STREAM);
    pu += SW;
  };
  // Activations are staged before the weight prefetch goes out: memory
  // waits count in issue order, so staging after it would also wait for
  // the prefetch.
  if (one_batch && n_items > 0) stage_store(0);
  // The prologue issues each stage's loads in the loop's order (no
  // regrouping by the scheduler): the loop's wait counts assume it.
  Stage st[PF];
#pragma unroll
  for (int f = 0; f < PF; ++f) {
    load(st[f]);
    __builtin_amdgcn_sched_barrier(0);
  }

  if constexpr (SX == SX_SCATTER) {
    // Step sums from the staged pairs.
    barrier_no_fence();
    const uint32_t ones = DT == OC_DTYPE_BF16 ? 0x3F803F80u : 0x3C003C00u;
    for (int i = tid; i < MR * KS; i += SNT) {
      const int m = i / KS, ks = i - m * KS;
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint4 pr = xpairs[m * RS + ks * 4 + w];
        sum = dot2acc<DT>(pr.x, ones, sum);
        sum = dot2acc<DT>(pr.y, ones, sum);
        sum = dot2acc<DT>(pr.z, ones, sum);
        sum = dot2acc<DT>(pr.w, ones, sum);
      }
      put_sum(m, ks, sum);
    }
  }
  barrier_no_fence();  // LDS only: the weight loads stay in flight

  // ---- consume: one tile at a time per wave, finished tiles parked in LDS ----
  const int nu = w_u0 < u1 ? (u1 - w_u0 + SW - 1) / SW : 0;
  int cu = w_u0, ct = w_u0 / QT;  // consumer: unit and its tile
  int t_end = (ct + 1) * QT;      // first unit of the next tile
  int cur_t = ct;                 // tile being accumulated
  constexpr int NACC = MF ? 4 : MR;
  float acc[NACC];  // dot2: row m, lane's K step; MFMA: row 4 h + i, column c
#pragma unroll
  for (int m = 0; m < NACC; ++m) acc[m] = 0.f;
  // MFMA form: the zero term of the tile, accumulated by the matrix core
  // alone and added to acc when the tile is parked. (Chaining it through
  // acc, whose values the VALU writes, gave wrong sums for 16 rows.)
  v4f32 zacc = {0.f, 0.f, 0.f, 0.f};
  auto flush = [&]() {
    float *slot_red = red + ((cur_t - t_first) * SW + wave) * MR * 16;
    if constexpr (MF) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (4 * h + i < MR) slot_red[(4 * h + i) * 16 + c] = acc[i] + zacc[i];
        acc[i] = 0.f;
        zacc[i] = 0.f;
      }
    } else {
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        float v = acc[m];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (h == 0) slot_red[m * 16 + c] = v;
        acc[m] = 0.f;
      }
    }
  };
  const int nu_pad = (nu + PF - 1) / PF * PF;
  for (int i0 = 0; i0 < nu_pad; i0 += PF) {
#pragma unroll
    for (int f = 0; f < PF; ++f) {
      const bool valid = i0 + f < nu;
      Stage &cur = st[f];  // refilled once consumed (below): fixed registers per stage
      if (valid && cu >= t_end) {
        flush();
        ct = cu / QT;
        t_end = (ct + 1) * QT;
        cur_t = ct;
      }
      const int qq = min(cu - ct * QT, QT - 1);  // unit within the tile; K steps 4 qq .. 4 qq + 3 < KS4
      if constexpr (GL) {
        // Exact dequantization (the scale inside B), so the unit's MFMAs
        // accumulate across its four K steps: MFMA j takes word j of every
        // lane (octet j of K step 4 qq + h) against row r's matching octet.
        const uint32_t qw[8] = {cur.q.x, cur.q.y, cur.q.z, cur.q.w, cur.q2.x, cur.q2.y, cur.q2.z, cur.q2.w};
        v4f32 av = {acc[0], acc[1], acc[2], acc[3]};
        const float s8 = scale_f32<SDT>(cur.s);
        const float zs8 = -s8 * static_cast<float>((cur.z >> (8 * (c & 3))) & 0xFFu);
        const GroupParam gp = make_group_param(scale_f32<SDT>(cur.s), tile_zero(cur.z, c));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // 8-bit: words 2j, 2j + 1 hold the K rows 8j .. 8j + 7 (4 codes each)
          const uint4 b = WB == 8 ? dequant8_u8<DT>(qw[2 * j], qw[2 * j + 1], s8, zs8) : dequant8<DT>(qw[j], gp);
          const uint4 xa = make_uint4(cur.x[4 * j], cur.x[4 * j + 1], cur.x[4 * j + 2], cur.x[4 * j + 3]);
          av = mfma16x16x32<DT>(xa, b, av);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = av[i];
      } else if constexpr (MF) {
        // LDS operands first (their latency overlaps the decode): A =
        // row c's pairs of octet h of each step (rows past MR read row
        // MR - 1 and feed output rows that are never stored), and row c's
        // activation sum over K step 4 qq + h.
        const int arow = MR == 16 ? c : min(c, MR - 1);
        const uint4 *xrow = xpairs + arow * RS + 16 * qq + h;
        uint4 xa[4];
        static_for<0, 4>([&](auto J) __attribute__((always_inline)) { xa[J] = xrow[4 * J]; });
        const float xz = xst[(4 * qq + h) * MR + arow];
        // Zero term of the unit's four steps on the matrix core: lane (h, c)
        // holds A[c][h] = that sum and B[h][c] = -s (B + z) of its own step
        // and column, so zacc[i] += sum_h X[4 g + i][h] * (-s (B + z))[h][c].
        // Scale of the lane's own step h, selected without branches (a branch
        // per case would wait for each load on its own path).
        const uint32_t m1 = 0u - static_cast<uint32_t>(h == 1), m2 = 0u - static_cast<uint32_t>(h == 2),
                       m3 = 0u - static_cast<uint32_t>(h == 3);
        const uint32_t s_own = cur.s[0] ^ ((cur.s[0] ^ cur.s[1]) & m1) ^ ((cur.s[0] ^ cur.s[2]) & m2) ^
                               ((cur.s[0] ^ cur.s[3]) & m3);
        const float bz = -scale_f32<SDT>(s_own) * (dot_base<DT>() + static_cast<float>(tile_zero(cur.z, c)));
        zacc = __builtin_amdgcn_mfma_f32_16x16x4f32(xz, bz, zacc, 0, 0, 0);
        v4f32 av = {acc[0], acc[1], acc[2], acc[3]};
        const uint32_t *oct = cur.q, *sj = cur.s;  // octet h of K step j, scale of K step j (column c)
        // Units past the range load zero scales: they add exactly zero (finite
        // activations), so no per-value select is needed.
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t q = oct[j];
          const uint4 bq = make_uint4(and_or(q, 0x000F000Fu, MAGIC), and_or(q >> 4, 0x000F000Fu, MAGIC),
                                      and_or(q >> 8, 0x000F000Fu, MAGIC), and_or(q >> 12, 0x000F000Fu, MAGIC));
          const v4f32 d = mfma16x16x32<DT>(xa[j], bq, v4f32{0.f, 0.f, 0.f, 0.f});
          const float s = scale_f32<SDT>(sj[j]);
#pragma unroll
          for (int i = 0; i < 4; ++i) av[i] = __builtin_fmaf(s, d[i], av[i]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = av[i];
      } else {
        const int ks = 4 * qq + h;
        float d[MR][2];
#pragma unroll
        for (int m = 0; m < MR; ++m) d[m][0] = d[m][1] = 0.f;
        const uint32_t qs[4] = {cur.q.x, cur.q.y, cur.q.z, cur.q.w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t q = qs[w];
          const uint32_t b0 = and_or(q, 0x000F000Fu, MAGIC);
          const uint32_t b1 = and_or(q >> 4, 0x000F000Fu, MAGIC);
          const uint32_t b2 = and_or(q >> 8, 0x000F000Fu, MAGIC);
          const uint32_t b3 = and_or(q >> 12, 0x000F000Fu, MAGIC);
#pragma unroll
          for (int m = 0; m < MR; ++m) {
            const uint4 xp = xpairs[m * RS + ks * 4 + w];
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
          const float2 xs = xsum[m * KS4 + ks];
          const float v = __builtin_fmaf(s, __builtin_fmaf(-zf, xs.x, (d[m][0] + d[m][1]) - xs.y), acc[m]);
          acc[m] = valid ? v : acc[m];
        }
      }
      load(cur);
      cu += SW;
    }
  }
  if (nu > 0) flush();
  __syncthreads();

  // ---- tiles of the range: waves added in order; cut tiles through the workspace ----
  const int ntl = t_last - t_first + 1;
  const int m = (tid >> 4) % MR, cc = tid & 15;
  for (int slot = tid / (16 * MR); slot < ntl; slot += SNT / (16 * MR)) {
    const int t = t_first + slot;
    const int n = TILE_N * t + cc;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < SW; ++w) v += red[((slot * SW + w) * MR + m) * 16 + cc];
    const bool out_ok = m < M && n < p.N;
    if (t * QT >= u0 && (t + 1) * QT <= u1) {  // wholly inside the range
      if (out_ok) store_c<DT>(p.c, static_cast<int64_t>(m) * p.ldc + n, v + bias_at(p, n));
      continue;
    }
    // A cut tile has two contributors: this workgroup is the upper one when
    // the tile starts before its range, else the lower. Its cell: [lower
    // workgroup][m][column].
    const bool upper = t * QT < u0;
    const int lower_b = upper ? b - 1 : b;
    unsigned long long *cell = reinterpret_cast<unsigned long long *>(p.counters) + (lower_b * MR + m) * 16 + cc;
    const unsigned long long mine = (1ull << 32) | __float_as_uint(v);
    const unsigned long long old = __hip_atomic_exchange(cell, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old >> 32) {  // the other half is in: this workgroup finishes the tile
      const float other = __uint_as_float(static_cast<uint32_t>(old));
      const float sum = upper ? other + v : v + other;  // lower + upper
      if (out_ok) store_c<DT>(p.c, static_cast<int64_t>(m) * p.ldc + n, sum + bias_at(p, n));
      __hip_atomic_store(cell, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

size_t gemv_stream_lds_bytes(int MR, int KS, int nslots, bool global_rows) {
  const size_t KS4 = static_cast<size_t>(KS + 3) / 4 * 4;
  const size_t sums = MR > 2 ? sizeof(float) : sizeof(float2), pad = MR > 2 ? sizeof(uint4) : 0;
  const size_t staged = global_rows ? 0 : static_cast<size_t>(MR) * (KS4 * (4 * sizeof(uint4) + sums) + pad);
  return staged + static_cast<size_t>(nslots) * SW * MR * 16 * sizeof(float) + 16;  // + the scatter's trash slot
}

int gemv_stream_wgs(int M, int N, int KS, int cus, size_t cell_bytes) {
  static const int wpc = std::max(1, env_int("ONECOMP_HIP_STREAM_WPC", 1));  // tuning only
  const int MR = M >= 1 ? stream_rows(M) : 0;
  if (MR == 0) return 0;
  const int64_t tiles = (N + TILE_N - 1) / TILE_N, QT = (KS + 3) / 4;
  int64_t nwg = static_cast<int64_t>(cus) * wpc;
  // The MFMA form also runs narrow layers, one workgroup per tile.
  if (MR > 2) nwg = std::min(nwg, tiles);
  // At least a tile per workgroup (a cut tile then has two contributors), at
  // most SNTL tiles touched by a range, the activation rows and tile slots
  // in LDS, and a swap cell per cut value.
  if (tiles < nwg) return 0;
  // Staging pays off when a workgroup streams at least half as many weight
  // bytes as it stages activation bytes (measured: M = 16, K = N = 4096, one
  // tile per workgroup, stages 128 KB for 32 KB of weights and loses to the
  // whole-tile kernel, which reads its activations in the stream).
  if (MR > 2 && tiles * QT / nwg * 1024 < static_cast<int64_t>(MR) * KS * 32) return 0;
  const int64_t q1 = tiles * QT / nwg + 1;  // longest range, in units
  if ((q1 + QT - 1) / QT + 1 > SNTL) return 0;
  const int nslots = stream_slots(tiles, static_cast<int>(QT), static_cast<int>(nwg));
  if (gemv_stream_lds_bytes(MR, KS, nslots, false) > 160 * 1024 - 64) return 0;
  if (static_cast<size_t>(nwg) * MR * 16 * sizeof(unsigned long long) > cell_bytes) return 0;
  return static_cast<int>(nwg);
}

int gemv_stream_global_wgs(int M, int N, int KS, int cus, size_t cell_bytes) {
  if (M < 3 || M > 16) return 0;
  const int MR = stream_rows(M);
  const int64_t tiles = (N + TILE_N - 1) / TILE_N, QT = (KS + 3) / 4;
  int64_t nwg = cus;
  if (tiles < cus) {
    // Narrow layers: two workgroups per tile, each exactly half of it (an
    // even unit count per tile keeps every tile at two contributors).
    if (2 * tiles > cus || QT % 2 != 0) return 0;
    nwg = 2 * tiles;
  } else if (tiles % nwg == 0) {
    return 0;  // whole tiles already load compute units evenly
  }
  const int64_t q1 = tiles * QT / nwg + 1;
  if ((q1 + QT - 1) / QT + 1 > SNTL) return 0;
  const int nslots = stream_slots(tiles, static_cast<int>(QT), static_cast<int>(nwg));
  if (gemv_stream_lds_bytes(MR, KS, nslots, true) > 160 * 1024 - 64) return 0;
  if (static_cast<size_t>(nwg) * MR * 16 * sizeof(unsigned long long) > cell_bytes) return 0;
  return static_cast<int>(nwg);
}

template <int DT, int SDT, int MR, int SX, int PF, bool AL, int WB = 4>
static void launch_stream_t(const GemmParams &p, int nwg, hipStream_t s) {
  auto kern = gemv_stream_kernel<DT, SDT, MR, SX, PF, AL, WB>;
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  (void)hipGetDevice(&dev);
  const uint64_t bit = dev < 64 ? (uint64_t{1} << dev) : 0;
  if (!bit || !(attr_set.load(std::memory_order_relaxed) & bit)) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024 - 64);
    attr_set.fetch_or(bit, std::memory_order_relaxed);
  }
  GemmParams q = p;
  q.stream_slots = stream_slots((p.N + TILE_N - 1) / TILE_N, (p.KS + 3) / 4, nwg);
  hipLaunchKernelGGL(kern, dim3(nwg), dim3(SNT), gemv_stream_lds_bytes(MR, p.KS, q.stream_slots, SX == SX_GLOBAL), s,
                     q);
}

template <int DT, int SDT, int MR, int SX>
static void launch_stream_pf(const GemmParams &p, int nwg, hipStream_t s) {
  constexpr int PF = 2;  // units in flight per wave (measured: 2 beats 1, 3, 4, 6 and 8, and a deeper head start through LDS)
  if (p.KS % 4 == 0) launch_stream_t<DT, SDT, MR, SX, PF, true>(p, nwg, s);
  else launch_stream_t<DT, SDT, MR, SX, PF, false>(p, nwg, s);
}

template <int DT, int SDT, int MR>
static void launch_stream_x(const GemmParams &p, int nwg, bool global_rows, hipStream_t s) {
  if constexpr (MR > 2) {
    if (global_rows) return launch_stream_pf<DT, SDT, MR, SX_GLOBAL>(p, nwg, s);
  }
  if (p.kinv) launch_stream_pf<DT, SDT, MR, SX_SCATTER>(p, nwg, s);
  else if (p.kmap) launch_stream_pf<DT, SDT, MR, SX_GATHER>(p, nwg, s);
  else launch_stream_pf<DT, SDT, MR, SX_CONTIG>(p, nwg, s);
}

template <int DT, int SDT>
static void launch_stream_m(const GemmParams &p, int nwg, bool g, hipStream_t s) {
  switch (stream_rows(p.M)) {
    case 1: launch_stream_x<DT, SDT, 1>(p, nwg, g, s); break;
    case 2: launch_stream_x<DT, SDT, 2>(p, nwg, g, s); break;
    case 4: launch_stream_x<DT, SDT, 4>(p, nwg, g, s); break;
    case 8: launch_stream_x<DT, SDT, 8>(p, nwg, g, s); break;
    default: launch_stream_x<DT, SDT, 16>(p, nwg, g, s); break;
  }
}

// 8-bit layers (tile16x8) at M <= 16: the global form on the same ranges,
// rows staged as 4, 8 or 16 (M <= 2 multiply rows past M that read nowhere).
int gemv_stream_global8_wgs(int M, int N, int KS, int cus, size_t cell_bytes) {
  if (M < 1 || M > 16) return 0;
  const int MR = std::max(4, stream_rows(M));
  const int64_t tiles = (N + TILE_N - 1) / TILE_N, QT = (KS + 3) / 4;
  int64_t nwg = cus;
  if (tiles < cus) {
    // Narrow layers: two workgroups per tile, each exactly half of it.
    if (2 * tiles > cus || QT % 2 != 0) return 0;
    nwg = 2 * tiles;
  }
  const int64_t q1 = tiles * QT / nwg + 1;
  if ((q1 + QT - 1) / QT + 1 > SNTL) return 0;
  const int nslots = stream_slots(tiles, static_cast<int>(QT), static_cast<int>(nwg));
  if (gemv_stream_lds_bytes(MR, KS, nslots, true) > 160 * 1024 - 64) return 0;
  if (static_cast<size_t>(nwg) * MR * 16 * sizeof(unsigned long long) > cell_bytes) return 0;
  return static_cast<int>(nwg);
}

template <int DT, int SDT, int MR>
static void launch_stream8_al(const GemmParams &p, int nwg, hipStream_t s) {
  if (p.KS % 4 == 0) launch_stream_t<DT, SDT, MR, SX_GLOBAL, 2, true, 8>(p, nwg, s);
  else launch_stream_t<DT, SDT, MR, SX_GLOBAL, 2, false, 8>(p, nwg, s);
}

template <int DT, int SDT>
static void launch_stream8_m(const GemmParams &p, int nwg, hipStream_t s) {
  const int MR = std::max(4, stream_rows(p.M));
  if (MR == 4) launch_stream8_al<DT, SDT, 4>(p, nwg, s);
  else if (MR == 8) launch_stream8_al<DT, SDT, 8>(p, nwg, s);
  else launch_stream8_al<DT, SDT, 16>(p, nwg, s);
}

void launch_gptq8_gemv_stream(const GemmParams &p, int a_dtype, int scale_dtype, int nwg, hipStream_t s) {
  const bool bf = a_dtype == OC_DTYPE_BF16, sbf = scale_dtype == OC_DTYPE_BF16;
  if (bf && sbf) launch_stream8_m<OC_DTYPE_BF16, OC_DTYPE_BF16>(p, nwg, s);
  else if (bf) launch_stream8_m<OC_DTYPE_BF16, OC_DTYPE_F16>(p, nwg, s);
  else if (sbf) launch_stream8_m<OC_DTYPE_F16, OC_DTYPE_BF16>(p, nwg, s);
  else launch_stream8_m<OC_DTYPE_F16, OC_DTYPE_F16>(p, nwg, s);
}

void launch_gptq_gemv_stream(const GemmParams &p, int a_dtype, int scale_dtype, int nwg, bool global_rows,
                             hipStream_t s) {
  const bool bf = a_dtype == OC_DTYPE_BF16, sbf = scale_dtype == OC_DTYPE_BF16;
  if (bf && sbf) launch_stream_m<OC_DTYPE_BF16, OC_DTYPE_BF16>(p, nwg, global_rows, s);
  else if (bf) launch_stream_m<OC_DTYPE_BF16, OC_DTYPE_F16>(p, nwg, global_rows, s);
  else if (sbf) launch_stream_m<OC_DTYPE_F16, OC_DTYPE_BF16>(p, nwg, global_rows, s);
  else launch_stream_m<OC_DTYPE_F16, OC_DTYPE_F16>(p, nwg, global_rows, s);
}

}  // namespace oc
