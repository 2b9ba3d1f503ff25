// Decode GEMV (M <= 2) as one balanced weight stream per workgroup, for gfx950.
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
// mantissa of B (bf16 128.0, fp16 1024.0), the first sum on
// v_dot2_f32_{bf16,f16} against activation pairs in LDS and the second from
// per-step activation sums staged beside them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>

#include "oc_gemm_common.h"

namespace oc {

namespace {

constexpr int SW = 16;        // waves per workgroup
constexpr int SNT = 64 * SW;  // threads per workgroup
constexpr int SNTL = 8;       // tiles one workgroup's range may touch
constexpr int SB = 3;         // staged octets per thread per batch

enum { SX_CONTIG = 0, SX_SCATTER = 1, SX_GATHER = 2 };

// Balanced ranges: U = nwg q + r units; workgroups b < r own q + 1 units,
// the others q (q >= QT: the host launches at most one workgroup per tile).
__device__ __forceinline__ int range_start(int b, int q, int r) { return b * q + min(b, r); }

}  // namespace

// AL: K steps per tile a multiple of 4, so unit u starts at byte 1024 u of
// the tile16 words and at group (4 u) >> gshift of the scales and zeros.
template <int DT, int SDT, int MR, int SX, int PF, bool AL>
__global__ __launch_bounds__(SNT) void gemv_stream_kernel(GemmParams p) {
  constexpr uint32_t MAGIC = DT == OC_DTYPE_BF16 ? 0x43004300u : 0x64006400u;
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
  uint4 *xpairs = sx_lds;                                            // [MR][KS4 * 4]
  float2 *xsum = reinterpret_cast<float2 *>(sx_lds + MR * KS4 * 4);  // [MR][KS4]: (sum, B * sum)
  float *red = reinterpret_cast<float *>(xsum + MR * KS4);           // [SNTL][SW][MR][16]
  // 16-bit slot that takes the scatter's writes for rows without a place.
  const int trash16 = static_cast<int>(reinterpret_cast<uint16_t *>(red + SNTL * SW * MR * 16) -
                                       reinterpret_cast<uint16_t *>(xpairs));

  // ---- activation staging, batch by batch; the weight stream starts after
  // the first batch's loads so both are in flight together ----
  const uint16_t *a = static_cast<const uint16_t *>(p.a);
  const int n_items = SX == SX_SCATTER ? (p.K_logical >> 3) : KS * 4;  // octets to stage
  const uint4 *kinv4 = reinterpret_cast<const uint4 *>(p.kinv);
  uint4 xr[MR][SB];
  uint4 rr[SB];
  auto stage_load = [&](int base) {
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int ic = min(base + SNT * u + tid, n_items - 1);  // clamped: every thread loads
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
            x16[r0 < K_phys ? xpair_slot(m, 32 * KS4, r0) : trash16] = static_cast<uint16_t>(xw[j]);
            x16[r1 < K_phys ? xpair_slot(m, 32 * KS4, r1) : trash16] = static_cast<uint16_t>(xw[j] >> 16);
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
            xpairs[m * KS4 * 4 + i] = pr;
            if ((i & 3) == 0) xsum[m * KS4 + (i >> 2)] = make_float2(sum, dot_base<DT>() * sum);
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
            x16[xpair_slot(m, 32 * KS4, r)] = a[static_cast<int64_t>(min(m, M - 1)) * p.lda + k];
        }
      }
    }
  };
  // One batch covers the rows (the common case): its loads go out first and
  // the weight prefetch follows, so both are in flight together. Longer or
  // ragged rows are staged before the weight stream starts.
  const bool one_batch = n_items <= SNT * SB && (SX != SX_SCATTER || (p.K_logical & 7) == 0);
  if (one_batch && n_items > 0) stage_load(0);

  // Zeros (while the activations load): the parked tile sums, and the
  // padding steps [KS, KS4) of every row (a unit's lanes past the last K
  // step multiply zeros).
  for (int i = tid; i < SNTL * SW * MR * 16; i += SNT) red[i] = 0.f;
  const int pad = 4 * (KS4 - KS);
  for (int i = tid; i < MR * pad; i += SNT) {
    const int m = i / pad, j = i - m * pad;
    xpairs[(m * KS4 + KS) * 4 + j] = make_uint4(0, 0, 0, 0);
    if (j < KS4 - KS) xsum[m * KS4 + KS + j] = make_float2(0.f, 0.f);
  }
  if constexpr (SX == SX_SCATTER) {
    if (p.K_logical != p.K_phys) {  // physical rows without a source stay zero
      for (int i = tid; i < MR * KS4 * 4; i += SNT) xpairs[i] = make_uint4(0, 0, 0, 0);
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
  struct Stage {
    uint4 q;
    uint32_t s;
    uint32_t z;
  };
  // Buffer loads: a wave-uniform unit offset plus a fixed per-lane offset.
  // Lanes past a tile's last K step read the next tile (or past the end:
  // zero), which meets the zero padding of the staged activations; units
  // past the wave's range get an offset beyond every buffer (zero, no
  // memory access).
  const int G = p.G, gshift = p.gshift, gs2 = min(gshift, 2);
  const __amdgpu_buffer_rsrc_t q_rs = buffer_rsrc(p.qw, static_cast<int64_t>(tiles) * KS * 256);
  const __amdgpu_buffer_rsrc_t s_rs = buffer_rsrc(p.scales, static_cast<int64_t>(tiles) * G * 32);
  const __amdgpu_buffer_rsrc_t z_rs = buffer_rsrc(p.zeros, static_cast<int64_t>(tiles) * G * 8);
  const uint32_t q_lane = lane * 16u;                                  // column c, K step 4 q + h
  const uint32_t s_lane = static_cast<uint32_t>((h >> gs2) * 16 + c) * 2u;  // group of K step 4 q + h
  const uint32_t z_lane = static_cast<uint32_t>((h >> gs2) * 2 + (c >> 3)) * 4u;
  constexpr uint32_t NOWHERE = 0xFFFFF000u;
  const int w_u0 = u0 + wave;  // this wave's first unit; it takes every SW-th from there
  int pu = w_u0;               // producer: next unit to load
  auto load = [&](Stage &S) {
    uint32_t qb, gb;
    if constexpr (AL) {
      qb = static_cast<uint32_t>(pu) * 1024u;
      gb = static_cast<uint32_t>(4 * pu) >> gshift;
    } else {
      const int tt = pu / QT, qq = pu - tt * QT;
      qb = static_cast<uint32_t>(tt * KS + 4 * qq) * 256u;
      gb = static_cast<uint32_t>(tt * G + ((4 * qq) >> gshift));
    }
    const bool in = pu < u1;
    const auto q = __builtin_amdgcn_raw_buffer_load_b128(q_rs, q_lane + (in ? qb : NOWHERE), 0, 0);
    S.q = make_uint4(q[0], q[1], q[2], q[3]);
    S.s = __builtin_amdgcn_raw_buffer_load_b16(s_rs, s_lane + (in ? gb * 32u : NOWHERE), 0, 0);
    S.z = __builtin_amdgcn_raw_buffer_load_b32(z_rs, z_lane + (in ? gb * 8u : NOWHERE), 0, 0);
    pu += SW;
  };
  // The prologue issues each stage's loads in the loop's order (no
  // regrouping by the scheduler): the loop's wait counts assume it.
  Stage st[PF];
#pragma unroll
  for (int f = 0; f < PF; ++f) {
    load(st[f]);
    __builtin_amdgcn_sched_barrier(0);
  }

  if (one_batch && n_items > 0) stage_store(0);
  if constexpr (SX == SX_SCATTER) {
    // Step sums from the staged pairs.
    barrier_no_fence();
    const uint32_t ones = DT == OC_DTYPE_BF16 ? 0x3F803F80u : 0x3C003C00u;
    for (int i = tid; i < MR * KS; i += SNT) {
      const int m = i / KS, ks = i - m * KS;
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint4 pr = xpairs[(m * KS4 + ks) * 4 + w];
        sum = dot2acc<DT>(pr.x, ones, sum);
        sum = dot2acc<DT>(pr.y, ones, sum);
        sum = dot2acc<DT>(pr.z, ones, sum);
        sum = dot2acc<DT>(pr.w, ones, sum);
      }
      xsum[m * KS4 + ks] = make_float2(sum, dot_base<DT>() * sum);
    }
  }
  barrier_no_fence();  // LDS only: the weight loads stay in flight

  // ---- consume: one tile at a time per wave, finished tiles parked in LDS ----
  const int nu = w_u0 < u1 ? (u1 - w_u0 + SW - 1) / SW : 0;
  int cu = w_u0, ct = w_u0 / QT;  // consumer: unit and its tile
  int t_end = (ct + 1) * QT;      // first unit of the next tile
  int cur_t = ct;                 // tile being accumulated
  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.f;
  auto flush = [&]() {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float v = acc[m];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (h == 0) red[(((cur_t - t_first) * SW + wave) * MR + m) * 16 + c] = v;
      acc[m] = 0.f;
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
      const int ks = 4 * min(cu - ct * QT, QT - 1) + h;  // < KS4 (padded rows)
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
          const uint4 xp = xpairs[(m * KS4 + ks) * 4 + w];
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
      load(cur);
      cu += SW;
    }
  }
  if (nu > 0) flush();
  __syncthreads();

  // ---- tiles of the range: waves added in order; cut tiles through the workspace ----
  const int ntl = t_last - t_first + 1;
  const int slot = tid / (16 * MR), m = (tid >> 4) % MR, cc = tid & 15;
  const int t = t_first + slot;
  const int n = TILE_N * t + cc;
  if (slot >= ntl) return;
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < SW; ++w) v += red[((slot * SW + w) * MR + m) * 16 + cc];
  const bool out_ok = m < M && n < p.N;
  if (t * QT >= u0 && (t + 1) * QT <= u1) {  // wholly inside the range
    if (out_ok) store_c<DT>(p.c, static_cast<int64_t>(m) * p.ldc + n, v + bias_at(p, n));
    return;
  }
  // A cut tile: the range's first (this workgroup is its upper contributor)
  // or its last (the lower one). Its cell: [lower workgroup][m][column].
  const bool upper = slot == 0;
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

size_t gemv_stream_lds_bytes(int MR, int KS) {
  const size_t KS4 = static_cast<size_t>(KS + 3) / 4 * 4;
  return static_cast<size_t>(MR) * KS4 * (4 * sizeof(uint4) + sizeof(float2)) +
         static_cast<size_t>(SNTL) * SW * MR * 16 * sizeof(float) + 16;  // + the scatter's trash slot
}

int gemv_stream_wgs(int M, int N, int KS, int cus, size_t cell_bytes) {
  static const int wpc = std::max(1, env_int("ONECOMP_HIP_STREAM_WPC", 1));  // tuning only
  if (M < 1 || M > 2) return 0;
  if (gemv_stream_lds_bytes(M, KS) > 160 * 1024 - 64) return 0;
  const int64_t tiles = (N + TILE_N - 1) / TILE_N, QT = (KS + 3) / 4;
  const int64_t nwg = static_cast<int64_t>(cus) * wpc;
  // At least a tile per workgroup (a cut tile then has two contributors), at
  // most SNTL tiles touched by a range, and a swap cell per cut value.
  if (tiles < nwg) return 0;
  const int64_t q1 = tiles * QT / nwg + 1;  // longest range, in units
  if ((q1 + QT - 1) / QT + 1 > SNTL) return 0;
  if (static_cast<size_t>(nwg) * M * 16 * sizeof(unsigned long long) > cell_bytes) return 0;
  return static_cast<int>(nwg);
}

template <int DT, int SDT, int MR, int SX, int PF, bool AL>
static void launch_stream_t(const GemmParams &p, int nwg, hipStream_t s) {
  auto kern = gemv_stream_kernel<DT, SDT, MR, SX, PF, AL>;
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  (void)hipGetDevice(&dev);
  const uint64_t bit = dev < 64 ? (uint64_t{1} << dev) : 0;
  if (!bit || !(attr_set.load(std::memory_order_relaxed) & bit)) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024 - 64);
    attr_set.fetch_or(bit, std::memory_order_relaxed);
  }
  hipLaunchKernelGGL(kern, dim3(nwg), dim3(SNT), gemv_stream_lds_bytes(MR, p.KS), s, p);
}

template <int DT, int SDT, int MR, int SX>
static void launch_stream_pf(const GemmParams &p, int nwg, hipStream_t s) {
  constexpr int PF = 2;  // units in flight per wave (measured: 2 beats 1, 3, 4, 6 and 8, and a deeper head start through LDS)
  if (p.KS % 4 == 0) launch_stream_t<DT, SDT, MR, SX, PF, true>(p, nwg, s);
  else launch_stream_t<DT, SDT, MR, SX, PF, false>(p, nwg, s);
}

template <int DT, int SDT, int MR>
static void launch_stream_x(const GemmParams &p, int nwg, hipStream_t s) {
  if (p.kinv) launch_stream_pf<DT, SDT, MR, SX_SCATTER>(p, nwg, s);
  else if (p.kmap) launch_stream_pf<DT, SDT, MR, SX_GATHER>(p, nwg, s);
  else launch_stream_pf<DT, SDT, MR, SX_CONTIG>(p, nwg, s);
}

template <int DT, int SDT>
static void launch_stream_m(const GemmParams &p, int nwg, hipStream_t s) {
  if (p.M == 1) launch_stream_x<DT, SDT, 1>(p, nwg, s);
  else launch_stream_x<DT, SDT, 2>(p, nwg, s);
}

void launch_gptq_gemv_stream(const GemmParams &p, int a_dtype, int scale_dtype, int nwg, hipStream_t s) {
  const bool bf = a_dtype == OC_DTYPE_BF16, sbf = scale_dtype == OC_DTYPE_BF16;
  if (bf && sbf) launch_stream_m<OC_DTYPE_BF16, OC_DTYPE_BF16>(p, nwg, s);
  else if (bf) launch_stream_m<OC_DTYPE_BF16, OC_DTYPE_F16>(p, nwg, s);
  else if (sbf) launch_stream_m<OC_DTYPE_F16, OC_DTYPE_BF16>(p, nwg, s);
  else launch_stream_m<OC_DTYPE_F16, OC_DTYPE_F16>(p, nwg, s);
}

}  // namespace oc
