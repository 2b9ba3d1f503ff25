// Decode GEMV (M <= 2) over balanced work items, for gfx950.
//
// A layer's work is cut into items of T 16-column tiles x S K steps (32
// physical rows each), sized by the host so that the items spread evenly over
// the compute units: whole tiles alone leave CUs idle or doubly loaded when
// the tile count is not a multiple of the CU count (320 tiles on 256 CUs), and
// re-stage the whole activation row for every 16 columns. Each item stages only
// the activations of its own K range (gathered through kmap for act-order and
// padded layers), streams its weights 1 KB per wave instruction, and, when K
// is split, writes fp32 partial sums; the last item of a tile group to finish
// (a device-scope counter per group) adds the partials in split order, so the
// result does not depend on which item finishes last. The counter returns to
// zero, so the counters stay valid across calls and HIP graph replays without
// any fill.
//
// Inner product (as in the whole-tile decode kernel): the scale and zero are
// factored out of each 32-row group,
//   sum_k x_k * s * (w_k - z) = s * (sum_k x_k * (B + w_k) - (B + z) * sum_k x_k),
// with B + w_k the exact 16-bit number made by OR-ing the code into the
// mantissa of B (bf16 128.0, fp16 1024.0), the first sum on
// v_dot2_f32_{bf16,f16} against activation pairs staged in LDS and the second
// from per-step activation sums staged beside them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "oc_gemm_common.h"

namespace oc {

template <int DT, int SDT, int MR, int T, int NQ>
__global__ __launch_bounds__(256) void gemv_split_kernel(GemmParams p) {
  // Item = T tiles x S K steps, S = 16 NQ / T: each of the 4 waves owns one
  // tile and NQ quads of K steps (lane (c, h): column c, step 4q + h), so a
  // wave instruction streams 1 KB of one tile. All of a wave's weight loads
  // are issued before the item's activations are staged and consumed in
  // order: straight-line code whose waits the compiler counts exactly
  // (other resident workgroups overlap the next item's loads).
  static_assert(T == 1 || T == 2 || T == 4, "tiles per item");
  constexpr int WPT = 4 / T;  // waves per tile
  constexpr int S = 16 * NQ / T;
  static_assert(S <= 64, "staging covers 64 K steps (4 octets per thread)");
  constexpr uint32_t MAGIC = DT == OC_DTYPE_BF16 ? 0x43004300u : 0x64006400u;
  extern __shared__ __attribute__((aligned(16))) uint4 gemv_lds[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane & 15, h = lane >> 4;
  const int item = blockIdx.x;
  const int grp = item / p.ksplit, sp = item - grp * p.ksplit;
  const int ks0 = sp * S, ks1 = min(ks0 + S, p.KS);
  const int nks = ks1 - ks0;  // K steps of this item (>= 1)
  const int tiles = (p.N + TILE_N - 1) / TILE_N;
  const int KS = p.KS;

  // LDS: x-pairs [MR][S][4] uint4, step sums [MR][S] float2, reduction [4][MR][16] float.
  uint4 *xpairs = gemv_lds;
  float2 *xsum = reinterpret_cast<float2 *>(gemv_lds + MR * S * 4);
  float *red = reinterpret_cast<float *>(xsum + MR * S);

  // ---- 1. activation loads for rows [32 ks0, 32 ks1) ----
  // Thread o < 4 nks owns octet o (8 physical rows) of local step o / 4.
  const uint16_t *a = static_cast<const uint16_t *>(p.a);
  const int o = tid;
  const bool own = o < 4 * nks;
  const int r0 = 32 * ks0 + 8 * min(o, 4 * nks - 1);  // clamped: every thread loads
  uint32_t xv[MR][8];
  if (p.kmap) {
    const int4 k0 = *reinterpret_cast<const int4 *>(p.kmap + r0);
    const int4 k1 = *reinterpret_cast<const int4 *>(p.kmap + r0 + 4);
    const int kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const uint16_t *arow = a + static_cast<int64_t>(min(m, p.M - 1)) * p.lda;
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[m][i] = arow[max(kk[i], 0)];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (kk[i] < 0) xv[m][i] = 0u;
    }
  } else {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const uint4 raw = *reinterpret_cast<const uint4 *>(a + static_cast<int64_t>(min(m, p.M - 1)) * p.lda + r0);
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xv[m][2 * i] = w[i] & 0xFFFFu;
        xv[m][2 * i + 1] = w[i] >> 16;
      }
    }
  }

  // ---- 2. all weight loads of this wave ----
  const int j = wave % T;
  const int t = min(grp * T + j, tiles - 1);  // tail groups re-read the last tile (never stored)
  const int q0 = wave / T;                    // quad slot of this wave
  const uint4 *qt4 = static_cast<const uint4 *>(p.qw) + static_cast<int64_t>(t) * KS * TILE_N + c;
  const uint16_t *stp = static_cast<const uint16_t *>(p.scales) + static_cast<int64_t>(t) * p.G * TILE_N + c;
  const uint32_t *ztp = static_cast<const uint32_t *>(p.zeros) + static_cast<int64_t>(t) * p.G * 2 + (c >> 3);
  uint4 wq[NQ];
  uint32_t ws[NQ], wz[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int ks = ks0 + min(4 * (q0 + WPT * i) + h, nks - 1);  // clamped into the item (unused if past it)
    wq[i] = qt4[static_cast<int64_t>(ks) * TILE_N];
    const int g = ks >> p.gshift;
    ws[i] = stp[g * TILE_N];
    wz[i] = ztp[g * 2];
  }

  // ---- 3. stage the activations (pairs and step sums) ----
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const uint4 raw = make_uint4(xv[m][0] | xv[m][1] << 16, xv[m][2] | xv[m][3] << 16, xv[m][4] | xv[m][5] << 16,
                                 xv[m][6] | xv[m][7] << 16);
    float sum;
    const uint4 pr = octet_pairs<DT>(raw, sum);
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    if (own && m < p.M) {
      xpairs[m * S * 4 + o] = pr;
      if ((o & 3) == 0) xsum[m * S + (o >> 2)] = make_float2(sum, dot_base<DT>() * sum);
    }
  }
  barrier_no_fence();  // LDS only: the weight loads stay in flight

  // ---- 4. consume the weights in issue order ----
  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int lk_raw = 4 * (q0 + WPT * i) + h;  // local K step
    const bool valid = lk_raw < nks;
    const int lk = min(lk_raw, nks - 1);
    float d[MR][2];
#pragma unroll
    for (int m = 0; m < MR; ++m) d[m][0] = d[m][1] = 0.f;
    const uint32_t qs[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t qw = qs[w];
      const uint32_t b0 = and_or(qw, 0x000F000Fu, MAGIC);
      const uint32_t b1 = and_or(qw >> 4, 0x000F000Fu, MAGIC);
      const uint32_t b2 = and_or(qw >> 8, 0x000F000Fu, MAGIC);
      const uint32_t b3 = and_or(qw >> 12, 0x000F000Fu, MAGIC);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const uint4 xp = xpairs[(m * S + lk) * 4 + w];
        float &dd = d[m][w >> 1];
        dd = dot2acc<DT>(b0, xp.x, dd);
        dd = dot2acc<DT>(b1, xp.y, dd);
        dd = dot2acc<DT>(b2, xp.z, dd);
        dd = dot2acc<DT>(b3, xp.w, dd);
      }
    }
    const float zf = static_cast<float>(tile_zero(wz[i], c));
    const float sc = valid ? scale_f32<SDT>(ws[i]) : 0.f;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float2 xs = xsum[m * S + lk];
      acc[m] = __builtin_fmaf(sc, __builtin_fmaf(-zf, xs.x, (d[m][0] + d[m][1]) - xs.y), acc[m]);
    }
  }

  // ---- reduction: phases h (xor 16, 32), then the waves of a tile in order ----
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    acc[m] += __shfl_xor(acc[m], 16);
    acc[m] += __shfl_xor(acc[m], 32);
  }
  if (h == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) red[(wave * MR + m) * 16 + c] = acc[m];
  }
  __syncthreads();
  // Thread (m, col) of the item's 16 T columns: its value.
  const int col = tid % (16 * T), mo = tid / (16 * T);
  const bool has_out = mo < MR && mo < p.M;
  const int n = 16 * (grp * T) + col;
  float v = 0.f;
  if (has_out) {
    const int jj = col >> 4;
#pragma unroll
    for (int w = 0; w < WPT; ++w) v += red[((jj + T * w) * MR + mo) * 16 + (col & 15)];
  }
  if (p.ksplit == 1) {
    if (has_out && n < p.N) store_c<DT>(p.c, static_cast<int64_t>(mo) * p.ldc + n, v + bias_at(p, n));
    return;
  }

  // ---- split K: partials, then the last item of the group sums them ----
  // Partials and counters use device-coherent (agent-scope) accesses, which
  // need no cache maintenance; ordering comes from waiting for this
  // workgroup's partial stores to complete before the count goes up. (An
  // acquire/release fence at agent scope would write back and invalidate
  // the whole L2 for every item.)
  float *part = p.partials;
  const int64_t prow = static_cast<int64_t>(MR) * p.N;  // floats per split
  if (has_out && n < p.N)
    __hip_atomic_store(part + sp * prow + static_cast<int64_t>(mo) * p.N + n, v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  __shared__ int last;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores are complete
  __syncthreads();                // ... and every wave's
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(p.counters + grp, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == p.ksplit - 1;
    if (last) __hip_atomic_store(p.counters + grp, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last || !has_out || n >= p.N) return;
  float sum = 0.f;
  for (int s = 0; s < p.ksplit; ++s)
    sum += __hip_atomic_load(part + s * prow + static_cast<int64_t>(mo) * p.N + n, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  store_c<DT>(p.c, static_cast<int64_t>(mo) * p.ldc + n, sum + bias_at(p, n));
}

size_t gemv_lds_bytes(int MR, int S) {
  return static_cast<size_t>(MR) * S * (4 * sizeof(uint4) + sizeof(float2)) + 4 * MR * 16 * sizeof(float);
}

template <int DT, int SDT, int MR, int T, int NQ>
static void launch_gemv_t(const GemmParams &p, int items, hipStream_t s) {
  hipLaunchKernelGGL((gemv_split_kernel<DT, SDT, MR, T, NQ>), dim3(items), dim3(256), gemv_lds_bytes(MR, 16 * NQ / T),
                     s, p);
}

// Shapes with S = 16 NQ / T in {8, 16, 32, 64} (T = 1: S >= 16).
template <int DT, int SDT, int MR, int T>
static void launch_gemv_s(const GemmParams &p, int items, hipStream_t s) {
  const int nq = p.ksteps_per_split * T / 16;
  if constexpr (T == 4) {
    if (nq == 16) launch_gemv_t<DT, SDT, MR, 4, 16>(p, items, s);
    else if (nq == 8) launch_gemv_t<DT, SDT, MR, 4, 8>(p, items, s);
    else if (nq == 4) launch_gemv_t<DT, SDT, MR, 4, 4>(p, items, s);
    else launch_gemv_t<DT, SDT, MR, 4, 2>(p, items, s);
  } else if constexpr (T == 2) {
    if (nq == 8) launch_gemv_t<DT, SDT, MR, 2, 8>(p, items, s);
    else if (nq == 4) launch_gemv_t<DT, SDT, MR, 2, 4>(p, items, s);
    else if (nq == 2) launch_gemv_t<DT, SDT, MR, 2, 2>(p, items, s);
    else launch_gemv_t<DT, SDT, MR, 2, 1>(p, items, s);
  } else {
    if (nq == 4) launch_gemv_t<DT, SDT, MR, 1, 4>(p, items, s);
    else if (nq == 2) launch_gemv_t<DT, SDT, MR, 1, 2>(p, items, s);
    else launch_gemv_t<DT, SDT, MR, 1, 1>(p, items, s);
  }
}

template <int DT, int SDT, int MR>
static void launch_gemv_m(const GemmParams &p, int T, int items, hipStream_t s) {
  if (T == 4) launch_gemv_s<DT, SDT, MR, 4>(p, items, s);
  else if (T == 2) launch_gemv_s<DT, SDT, MR, 2>(p, items, s);
  else launch_gemv_s<DT, SDT, MR, 1>(p, items, s);
}

template <int DT, int SDT>
static void launch_gemv_d(const GemmParams &p, int T, int items, hipStream_t s) {
  if (p.M == 1) launch_gemv_m<DT, SDT, 1>(p, T, items, s);
  else launch_gemv_m<DT, SDT, 2>(p, T, items, s);
}

void launch_gptq_gemv(const GemmParams &p, int a_dtype, int scale_dtype, int T, hipStream_t s) {
  const int tiles = (p.N + TILE_N - 1) / TILE_N;
  const int items = (tiles + T - 1) / T * p.ksplit;
  const bool bf = a_dtype == OC_DTYPE_BF16, sbf = scale_dtype == OC_DTYPE_BF16;
  if (bf && sbf) launch_gemv_d<OC_DTYPE_BF16, OC_DTYPE_BF16>(p, T, items, s);
  else if (bf) launch_gemv_d<OC_DTYPE_BF16, OC_DTYPE_F16>(p, T, items, s);
  else if (sbf) launch_gemv_d<OC_DTYPE_F16, OC_DTYPE_BF16>(p, T, items, s);
  else launch_gemv_d<OC_DTYPE_F16, OC_DTYPE_F16>(p, T, items, s);
}

GemvPlan plan_gemv(int M, int N, int KS, bool gather, int cus) {
  // Cost of an item in weight-byte equivalents: its weights (256 code bytes,
  // 32 scale bytes and 8 zero bytes per tile and K step), the activation
  // staging of its K range (a gathered row costs like 24 streamed bytes), a
  // fixed start cost, and the partial-sum round trip when K is split. Items
  // of one launch are resident together, so the busiest CU carries
  // ceil(items / CUs) of them.
  // ONECOMP_HIP_GEMV_T / ONECOMP_HIP_GEMV_S force a shape (tuning only).
  static const int force_t = env_int("ONECOMP_HIP_GEMV_T", 0);
  static const int force_s = env_int("ONECOMP_HIP_GEMV_S", 0);
  const int tiles = (N + TILE_N - 1) / TILE_N;
  GemvPlan best{4, 64, (KS + 63) / 64};
  double best_cost = 1e300;
  for (int T : {4, 2, 1}) {
    if ((T > 1 && tiles < T) || (force_t && T != force_t)) continue;
    const int groups = (tiles + T - 1) / T;
    for (int S : {8, 16, 32, 64}) {
      if ((T == 1 && S < 16) || (force_s && S != force_s)) continue;
      const int ksplit = (KS + S - 1) / S;
      const int ks_eff = std::min(S, KS);
      const double wbytes = static_cast<double>(T) * ks_eff * 296.0;
      const double stage = static_cast<double>(ks_eff) * 32.0 * M * (gather ? 24.0 : 2.0);
      const double fixed = 6144.0 + (ksplit > 1 ? 8192.0 : 0.0);
      const double item = wbytes + stage + fixed;
      const double items = static_cast<double>(groups) * ksplit;
      const double cost = std::ceil(items / cus) * item;
      if (cost < best_cost - 1e-9) {
        best_cost = cost;
        best = GemvPlan{T, S, ksplit};
      }
    }
  }
  return best;
}

}  // namespace oc
