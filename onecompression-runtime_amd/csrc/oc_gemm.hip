// Fused int4 dequant + GEMM kernels for gfx950 and their host dispatch.
//
// Two regimes:
//  * split-K streaming kernel (M <= 64): every lane streams 16-byte chunks of
//    packed weights (4 adjacent columns x 8 K rows), dequantizes them in
//    registers and feeds v_mfma_f32_16x16x32 with the activation rows as the
//    A operand. Waves of a workgroup split K and reduce through LDS; the
//    workgroups of one column tile split K further and the last one to finish
//    reduces their fp32 partials in a fixed order (deterministic).
//  * LDS-tiled kernel (large M): a workgroup owns a BM x BN output tile; the
//    activation tile for each 32-row K step is staged in LDS (double
//    buffered) and shared by the 4 waves, which split BN; each wave
//    dequantizes only its own columns, once per K step, straight into MFMA
//    B operands (no weight re-dequant across waves).
// Both use dequant8() (exact fp32 product, one RNE to the activation type),
// the same routine the standalone dequant kernel is tested with.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "oc_device.h"
#include "oc_internal.h"

namespace oc {

enum { FMT_GPTQ = 0, FMT_RTN = 1 };

struct GemmParams {
  const void *a;
  int64_t lda;
  int M;
  int K_logical;
  const void *qw;      // GPTQ: int32 [K_phys/8, N]; RTN: uint8 [N, row_bytes]
  const void *scales;  // GPTQ: [G, N] 16-bit; RTN: [N, G] of scale_dtype
  const void *zeros;   // GPTQ: int32 [G, N/8]; RTN: [N, G] of zero_dtype
  int zero_mode;       // GPTQ
  int scale_dtype;     // RTN (runtime)
  int zero_dtype;      // RTN (runtime)
  int rtn_gs;          // RTN: columns per group
  int rtn_G;           // RTN: groups per row
  int row_bytes;       // RTN
  int N;
  int K_phys;
  int group_rows;
  const int32_t *kmap;
  const void *bias;
  int bias_dtype;
  void *c;
  int64_t ldc;
  float *partials;    // [ksplit, M, N] fp32 (split-K only)
  int32_t *counters;  // one per output tile (split-K only), zero on entry and exit
  int ksplit;
  int ksteps_per_split;
  // grouped (MoE) launch
  const int32_t *expert_offsets;
  const int32_t *sorted_pairs;
  int topk;
  int64_t qw_expert_stride;  // elements of qw per expert
  int64_t s_expert_stride;
  int64_t z_expert_stride;
};

// ---------------------------------------------------------------------------
// Weight access, per format.

// Packed word (8 codes, code i at bits 4i) of column n, K rows 8*wrow .. 8*wrow+7.
template <int FMT>
__device__ __forceinline__ uint32_t load_word(const GemmParams &p, const void *qw, int wrow, int n) {
  if constexpr (FMT == FMT_GPTQ) {
    return static_cast<const uint32_t *>(qw)[static_cast<int64_t>(wrow) * p.N + n];
  } else {
    return *reinterpret_cast<const uint32_t *>(static_cast<const uint8_t *>(qw) +
                                               static_cast<int64_t>(n) * p.row_bytes + 4 * wrow);
  }
}

template <int SDT>
__device__ __forceinline__ GroupParam gptq_param(const GemmParams &p, const void *scales,
                                                 const void *zeros, int g, int n) {
  const uint16_t sb = static_cast<const uint16_t *>(scales)[static_cast<int64_t>(g) * p.N + n];
  const float s = SDT == OC_DTYPE_BF16 ? bf16_to_f32(sb) : f16_to_f32(sb);
  const uint32_t zw =
      static_cast<const uint32_t *>(zeros)[static_cast<int64_t>(g) * (p.N >> 3) + (n >> 3)];
  return make_group_param(s, unpack_zero(zw, n, p.zero_mode));
}

template <int DT>
__device__ __forceinline__ RtnParam rtn_param(const GemmParams &p, int g, int n) {
  const int64_t i = static_cast<int64_t>(n) * p.rtn_G + g;
  RtnParam r;
  r.zq = round_to<DT>(load_any_f32(p.zeros, i, p.zero_dtype));
  r.sq = round_to<DT>(load_any_f32(p.scales, i, p.scale_dtype));
  return r;
}

// Dequantized B operand (8 K rows of column n starting at row 8*wrow).
template <int DT, int SDT, int FMT>
__device__ __forceinline__ uint4 load_b(const GemmParams &p, const void *qw, const void *scales,
                                        const void *zeros, int wrow, int n) {
  const uint32_t q = load_word<FMT>(p, qw, wrow, n);
  if constexpr (FMT == FMT_GPTQ) {
    const int g = (8 * wrow) / p.group_rows;
    return dequant8<DT>(q, gptq_param<SDT>(p, scales, zeros, g, n));
  } else {
    const int g = (8 * wrow) / p.rtn_gs;
    return rtn_dequant8<DT>(q, rtn_param<DT>(p, g, n));
  }
}

// 8 activation values of row `row`, physical K rows k0 .. k0+7.
template <bool KMAP>
__device__ __forceinline__ uint4 load_a8(const GemmParams &p, const uint16_t *arow, int k0) {
  if constexpr (!KMAP) {
    return *reinterpret_cast<const uint4 *>(arow + k0);
  } else {
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int src = p.kmap[k0 + e];
      h[e] = src >= 0 ? arow[src] : 0u;
    }
    return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                      h[6] | (h[7] << 16));
  }
}

template <int DT>
__device__ __forceinline__ void store_c(void *c, int64_t i, float v) {
  static_cast<uint16_t *>(c)[i] = static_cast<uint16_t>(pack2<DT>(v, 0.f));
}

__device__ __forceinline__ float bias_at(const GemmParams &p, int n) {
  return p.bias ? load_any_f32(p.bias, n, p.bias_dtype) : 0.f;
}

// Split-K completion: returns true in every thread of the workgroup that
// finished last for counter `tile` (after all partial stores are visible).
__device__ __forceinline__ bool splitk_arrive(const GemmParams &p, int tile, int *s_flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(p.counters + tile, 1);
    *s_flag = prev == p.ksplit - 1;
  }
  __syncthreads();
  const bool last = *s_flag != 0;
  if (last) __threadfence();
  return last;
}

__device__ __forceinline__ void splitk_reset(const GemmParams &p, int tile) {
  if (threadIdx.x == 0) __hip_atomic_store(p.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Split-K streaming kernel. grid = (ceil(N/64), ksplit); 256 threads.
// Lane (quad = l/16, c16 = l%16) of a wave owns columns n0 + 4*c16 + j
// (j = 0..3, one 16-byte load per K step) and K rows 32*ks + 8*quad + 0..7.
// MFMA j therefore computes the columns {n0 + 4*i + j : i = 0..15}.
template <int DT, int SDT, int MT, bool KMAP, int FMT>
__global__ __launch_bounds__(256) void gemv_splitk_kernel(GemmParams p) {
  constexpr int WAVES = 4;
  __shared__ float red[WAVES][MT * 16][65];
  __shared__ int s_last;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int quad = lane >> 4, c16 = lane & 15;
  const int n0 = blockIdx.x * 64;
  const int ncol = n0 + 4 * c16;
  const bool col_ok = ncol < p.N;
  const int ksteps = p.K_phys / 32;
  const int ks_begin = blockIdx.y * p.ksteps_per_split;
  const int ks_end = min(ks_begin + p.ksteps_per_split, ksteps);
  const uint16_t *a = static_cast<const uint16_t *>(p.a);

  v4f32 acc[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[t][j] = v4f32{0.f, 0.f, 0.f, 0.f};

  for (int ks = ks_begin + wave; ks < ks_end; ks += WAVES) {
    const int wrow = 4 * ks + quad;
    uint4 b[4];
    if (col_ok) {
      if constexpr (FMT == FMT_GPTQ) {
        const uint4 q = *reinterpret_cast<const uint4 *>(static_cast<const uint32_t *>(p.qw) +
                                                         static_cast<int64_t>(wrow) * p.N + ncol);
        const int g = (32 * ks) / p.group_rows;
        const uint2 sr = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(p.scales) +
                                                          static_cast<int64_t>(g) * p.N + ncol);
        const uint32_t zw = static_cast<const uint32_t *>(p.zeros)[static_cast<int64_t>(g) * (p.N >> 3) + (ncol >> 3)];
        const uint16_t sb[4] = {static_cast<uint16_t>(sr.x), static_cast<uint16_t>(sr.x >> 16),
                                static_cast<uint16_t>(sr.y), static_cast<uint16_t>(sr.y >> 16)};
        const uint32_t qs[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float s = SDT == OC_DTYPE_BF16 ? bf16_to_f32(sb[j]) : f16_to_f32(sb[j]);
          b[j] = dequant8<DT>(qs[j], make_group_param(s, unpack_zero(zw, ncol + j, p.zero_mode)));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = load_b<DT, SDT, FMT>(p, p.qw, p.scales, p.zeros, wrow, ncol + j);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int row = 16 * t + c16;
      uint4 av = make_uint4(0, 0, 0, 0);
      if (row < p.M) av = load_a8<KMAP>(p, a + static_cast<int64_t>(row) * p.lda, 32 * ks + 8 * quad);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][j] = mfma16x16x32<DT>(av, b[j], acc[t][j]);
    }
  }

  // Cross-wave reduction. Lane value acc[t][j][i] is row 16t + 4*quad + i,
  // local column 4*c16 + j.
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * t + 4 * quad + i;
        if (row < p.M) red[wave][row][4 * c16 + j] = acc[t][j][i];
      }
  __syncthreads();

  const int M = p.M;
  if (p.ksplit == 1) {
    for (int e = tid; e < M * 64; e += 256) {
      const int row = e >> 6, col = e & 63, n = n0 + col;
      if (n >= p.N) continue;
      const float v = red[0][row][col] + red[1][row][col] + red[2][row][col] + red[3][row][col];
      store_c<DT>(p.c, static_cast<int64_t>(row) * p.ldc + n, v + bias_at(p, n));
    }
    return;
  }
  float *part = p.partials + static_cast<int64_t>(blockIdx.y) * M * p.N;
  for (int e = tid; e < M * 64; e += 256) {
    const int row = e >> 6, col = e & 63, n = n0 + col;
    if (n >= p.N) continue;
    part[static_cast<int64_t>(row) * p.N + n] =
        red[0][row][col] + red[1][row][col] + red[2][row][col] + red[3][row][col];
  }
  if (!splitk_arrive(p, blockIdx.x, &s_last)) return;
  for (int e = tid; e < M * 64; e += 256) {
    const int row = e >> 6, col = e & 63, n = n0 + col;
    if (n >= p.N) continue;
    float v = 0.f;
    for (int s = 0; s < p.ksplit; ++s)
      v += load_coherent(p.partials + (static_cast<int64_t>(s) * M + row) * p.N + n);
    store_c<DT>(p.c, static_cast<int64_t>(row) * p.ldc + n, v + bias_at(p, n));
  }
  splitk_reset(p, blockIdx.x);
}

// ---------------------------------------------------------------------------
// LDS-tiled kernel. BM = 16*WM rows, BN = 64*WN columns (4 waves x 16*WN).
// grid = (ceil(N/BN), ceil(M/BM), ksplit) or, grouped, (ceil(N/BN), 1, E).
constexpr int A_LDS_STRIDE = 40;  // halves per LDS row: 32 data + 8 pad (80 B)

template <int DT, int SDT, int WM, int WN, bool KMAP, int FMT, bool MOE>
__global__ __launch_bounds__(256) void gemm_tiled_kernel(GemmParams p) {
  constexpr int BM = 16 * WM;
  constexpr int BN = 64 * WN;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * A_LDS_STRIDE];
  __shared__ int s_last;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int quad = lane >> 4, c16 = lane & 15;
  const int n0 = blockIdx.x * BN;
  const int nw = n0 + wave * 16 * WN;  // first column of this wave
  const uint16_t *a = static_cast<const uint16_t *>(p.a);

  const void *qw = p.qw;
  const void *scales = p.scales;
  const void *zeros = p.zeros;
  int row_begin = 0, row_end = p.M, m_first;
  if constexpr (MOE) {
    const int e = blockIdx.z;
    row_begin = p.expert_offsets[e];
    row_end = p.expert_offsets[e + 1];
    qw = static_cast<const uint32_t *>(p.qw) + e * p.qw_expert_stride;
    scales = static_cast<const uint16_t *>(p.scales) + e * p.s_expert_stride;
    zeros = static_cast<const uint32_t *>(p.zeros) + e * p.z_expert_stride;
    m_first = row_begin;
  } else {
    m_first = blockIdx.y * BM;
  }
  const int ksteps = p.K_phys / 32;
  int ks_begin = 0, ks_end = ksteps;
  if constexpr (!MOE) {
    ks_begin = blockIdx.z * p.ksteps_per_split;
    ks_end = min(ks_begin + p.ksteps_per_split, ksteps);
  }

  // Activation staging: chunk c = (row, 16-byte piece) of the BM x 32 tile.
  constexpr int A_CHUNKS = BM * 4;
  constexpr int A_PER_THREAD = (A_CHUNKS + 255) / 256;

  for (int m0 = m_first; m0 < (MOE ? row_end : m_first + 1); m0 += BM) {
    // Source row pointer of each staged chunk (null = zero row).
    const uint16_t *src_row[A_PER_THREAD];
#pragma unroll
    for (int i = 0; i < A_PER_THREAD; ++i) {
      const int ch = tid + 256 * i;
      const int r = m0 + (ch >> 2);
      src_row[i] = nullptr;
      if (ch < A_CHUNKS && r < row_end) {
        int64_t arow = r;
        if constexpr (MOE) arow = p.sorted_pairs[r] / p.topk;
        src_row[i] = a + arow * p.lda;
      }
    }
    auto load_a_tile = [&](int ks, uint4 (&areg)[A_PER_THREAD]) {
#pragma unroll
      for (int i = 0; i < A_PER_THREAD; ++i) {
        const int ch = tid + 256 * i;
        areg[i] = src_row[i] ? load_a8<KMAP>(p, src_row[i], 32 * ks + 8 * (ch & 3)) : make_uint4(0, 0, 0, 0);
      }
    };
    auto store_a_tile = [&](int buf, const uint4 (&areg)[A_PER_THREAD]) {
#pragma unroll
      for (int i = 0; i < A_PER_THREAD; ++i) {
        const int ch = tid + 256 * i;
        if (ch < A_CHUNKS)
          *reinterpret_cast<uint4 *>(&As[buf][(ch >> 2) * A_LDS_STRIDE + 8 * (ch & 3)]) = areg[i];
      }
    };
    // Weight words and group parameters of the next K step, per column subtile.
    uint32_t qreg[WN];
    auto load_w = [&](int ks) {
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int n = nw + 16 * j + c16;
        qreg[j] = n < p.N ? load_word<FMT>(p, qw, 4 * ks + quad, n) : 0u;
      }
    };
    auto dequant_w = [&](int ks, uint4 (&b)[WN]) {
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int n = min(nw + 16 * j + c16, p.N - 1);
        if constexpr (FMT == FMT_GPTQ) {
          b[j] = dequant8<DT>(qreg[j], gptq_param<SDT>(p, scales, zeros, (32 * ks) / p.group_rows, n));
        } else {
          b[j] = rtn_dequant8<DT>(qreg[j], rtn_param<DT>(p, (32 * ks + 8 * quad) / p.rtn_gs, n));
        }
      }
    };

    v4f32 acc[WM][WN];
#pragma unroll
    for (int t = 0; t < WM; ++t)
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[t][j] = v4f32{0.f, 0.f, 0.f, 0.f};

    uint4 areg[A_PER_THREAD];
    if (ks_begin < ks_end) {
      load_a_tile(ks_begin, areg);
      load_w(ks_begin);
      store_a_tile(0, areg);
    }
    __syncthreads();
    for (int ks = ks_begin; ks < ks_end; ++ks) {
      const int buf = (ks - ks_begin) & 1;
      uint4 b[WN];
      dequant_w(ks, b);
      const bool has_next = ks + 1 < ks_end;
      if (has_next) {
        load_a_tile(ks + 1, areg);
        load_w(ks + 1);
      }
#pragma unroll
      for (int t = 0; t < WM; ++t) {
        const uint4 av = *reinterpret_cast<const uint4 *>(&As[buf][(16 * t + c16) * A_LDS_STRIDE + 8 * quad]);
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[t][j] = mfma16x16x32<DT>(av, b[j], acc[t][j]);
      }
      if (has_next) store_a_tile(buf ^ 1, areg);
      __syncthreads();
    }

    // Epilogue. acc[t][j][i] = tile row 16t + 4*quad + i, column nw + 16j + c16.
    if constexpr (MOE) {
#pragma unroll
      for (int t = 0; t < WM; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = m0 + 16 * t + 4 * quad + i;
          if (r >= row_end) continue;
          const int64_t orow = p.sorted_pairs[r];
#pragma unroll
          for (int j = 0; j < WN; ++j) {
            const int n = nw + 16 * j + c16;
            if (n < p.N) store_c<DT>(p.c, orow * p.ldc + n, acc[t][j][i]);
          }
        }
    } else if (p.ksplit == 1) {
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int n = nw + 16 * j + c16;
        if (n >= p.N) continue;
        const float bv = bias_at(p, n);
#pragma unroll
        for (int t = 0; t < WM; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = m0 + 16 * t + 4 * quad + i;
            if (r < p.M) store_c<DT>(p.c, static_cast<int64_t>(r) * p.ldc + n, acc[t][j][i] + bv);
          }
      }
    } else {
      float *part = p.partials + static_cast<int64_t>(blockIdx.z) * p.M * p.N;
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int n = nw + 16 * j + c16;
        if (n >= p.N) continue;
#pragma unroll
        for (int t = 0; t < WM; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = m0 + 16 * t + 4 * quad + i;
            if (r < p.M) part[static_cast<int64_t>(r) * p.N + n] = acc[t][j][i];
          }
      }
      const int tile = blockIdx.y * gridDim.x + blockIdx.x;
      if (!splitk_arrive(p, tile, &s_last)) return;
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int n = nw + 16 * j + c16;
        if (n >= p.N) continue;
        const float bv = bias_at(p, n);
#pragma unroll
        for (int t = 0; t < WM; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = m0 + 16 * t + 4 * quad + i;
            if (r >= p.M) continue;
            float v = 0.f;
            for (int s = 0; s < p.ksplit; ++s)
              v += load_coherent(p.partials + (static_cast<int64_t>(s) * p.M + r) * p.N + n);
            store_c<DT>(p.c, static_cast<int64_t>(r) * p.ldc + n, v + bv);
          }
      }
      splitk_reset(p, tile);
    }
  }
}

// ---------------------------------------------------------------------------
// MoE routing: stable counting sort of (token, slot) pairs by expert.
// One workgroup of 256 threads; thread t owns the contiguous pair range
// [t*per, (t+1)*per), so ranks computed from per-thread prefix counts keep
// the original pair order inside every expert.
constexpr int ROUTE_THREADS = 256;

__global__ __launch_bounds__(ROUTE_THREADS) void moe_route_kernel(const int64_t *__restrict__ ids, int P,
                                                                  int E, int32_t *__restrict__ offsets,
                                                                  int32_t *__restrict__ sorted) {
  extern __shared__ int32_t cnt[];  // [ROUTE_THREADS + 1][E]: per-thread counts, then totals
  const int tid = threadIdx.x;
  const int per = (P + ROUTE_THREADS - 1) / ROUTE_THREADS;
  const int p_begin = min(tid * per, P), p_end = min(p_begin + per, P);
  for (int e = tid; e < (ROUTE_THREADS + 1) * E; e += ROUTE_THREADS) cnt[e] = 0;
  __syncthreads();
  for (int q = p_begin; q < p_end; ++q) {
    const int64_t e = ids[q];
    if (e >= 0 && e < E) ++cnt[tid * E + e];
  }
  __syncthreads();
  // Exclusive prefix over threads for each expert (expert e handled by thread e % 256).
  for (int e = tid; e < E; e += ROUTE_THREADS) {
    int run = 0;
    for (int t = 0; t < ROUTE_THREADS; ++t) {
      const int c = cnt[t * E + e];
      cnt[t * E + e] = run;
      run += c;
    }
    cnt[ROUTE_THREADS * E + e] = run;
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int e = 0; e < E; ++e) {
      offsets[e] = run;
      const int c = cnt[ROUTE_THREADS * E + e];
      cnt[ROUTE_THREADS * E + e] = run;
      run += c;
    }
    offsets[E] = run;
  }
  __syncthreads();
  for (int q = p_begin; q < p_end; ++q) {
    const int64_t e = ids[q];
    if (e >= 0 && e < E) {
      const int pos = cnt[ROUTE_THREADS * E + e] + cnt[tid * E + e]++;
      sorted[pos] = q;
    }
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.

struct TileCfg {
  int wm, wn;
};

int env_int(const char *name, int dflt) {
  const char *v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

struct SplitPlan {
  int regime;
  int mt;         // split-K: row tiles of 16
  TileCfg tile;   // tiled
  int ksplit;
  int ksteps_per_split;
  int tiles;      // counters needed
};

SplitPlan plan_gemm(int M, int N, int K_phys, int regime) {
  SplitPlan sp{};
  const int ksteps = K_phys / 32;
  if (regime == OC_REGIME_AUTO) regime = M <= 64 ? OC_REGIME_SPLITK : OC_REGIME_TILED;
  sp.regime = regime;
  if (regime == OC_REGIME_SPLITK) {
    sp.mt = std::max(1, (M + 15) / 16);
    const int col_tiles = (N + 63) / 64;
    const int target = env_int("ONECOMP_HIP_SPLITK_TARGET_WGS", 1024);
    const int min_ksteps = env_int("ONECOMP_HIP_SPLITK_MIN_KSTEPS", 8);
    int ksplit = (target + col_tiles - 1) / col_tiles;
    ksplit = std::max(1, std::min(ksplit, std::max(1, ksteps / std::max(1, min_ksteps))));
    sp.ksteps_per_split = (ksteps + ksplit - 1) / ksplit;
    sp.ksplit = (ksteps + sp.ksteps_per_split - 1) / sp.ksteps_per_split;
    sp.tiles = col_tiles;
    return sp;
  }
  static const TileCfg cfgs[] = {{16, 3}, {8, 2}, {4, 1}};
  const int want = env_int("ONECOMP_HIP_TILED_MIN_WGS", 256);
  TileCfg pick = cfgs[2];
  for (const TileCfg &c : cfgs) {
    const int64_t tiles = static_cast<int64_t>((M + 16 * c.wm - 1) / (16 * c.wm)) *
                          ((N + 64 * c.wn - 1) / (64 * c.wn));
    if (tiles >= want) {
      pick = c;
      break;
    }
  }
  sp.tile = pick;
  const int tiles = ((M + 16 * pick.wm - 1) / (16 * pick.wm)) * ((N + 64 * pick.wn - 1) / (64 * pick.wn));
  int ksplit = 1;
  if (tiles < want) ksplit = std::min((want + tiles - 1) / tiles, std::max(1, ksteps / 8));
  sp.ksteps_per_split = (ksteps + ksplit - 1) / ksplit;
  sp.ksplit = (ksteps + sp.ksteps_per_split - 1) / sp.ksteps_per_split;
  sp.tiles = tiles;
  return sp;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t workspace_bytes(const SplitPlan &sp, int M, int N) {
  if (sp.ksplit <= 1) return 0;
  return align_up(static_cast<size_t>(sp.tiles) * 4, 256) +
         static_cast<size_t>(sp.ksplit) * M * N * sizeof(float);
}

template <int DT, int SDT, int MT, bool KMAP, int FMT>
void launch_splitk_t(const GemmParams &p, int col_tiles, hipStream_t s) {
  hipLaunchKernelGGL((gemv_splitk_kernel<DT, SDT, MT, KMAP, FMT>), dim3(col_tiles, p.ksplit), dim3(256), 0,
                     s, p);
}

template <int DT, int SDT, bool KMAP, int FMT>
void launch_splitk_mt(const GemmParams &p, int mt, int col_tiles, hipStream_t s) {
  switch (mt) {
    case 1: launch_splitk_t<DT, SDT, 1, KMAP, FMT>(p, col_tiles, s); break;
    case 2: launch_splitk_t<DT, SDT, 2, KMAP, FMT>(p, col_tiles, s); break;
    case 3: launch_splitk_t<DT, SDT, 3, KMAP, FMT>(p, col_tiles, s); break;
    default: launch_splitk_t<DT, SDT, 4, KMAP, FMT>(p, col_tiles, s); break;
  }
}

template <int DT, int SDT, int WM, int WN, bool KMAP, int FMT>
void launch_tiled_t(const GemmParams &p, hipStream_t s) {
  const dim3 grid((p.N + 64 * WN - 1) / (64 * WN), (p.M + 16 * WM - 1) / (16 * WM), p.ksplit);
  hipLaunchKernelGGL((gemm_tiled_kernel<DT, SDT, WM, WN, KMAP, FMT, false>), grid, dim3(256), 0, s, p);
}

template <int DT, int SDT, bool KMAP, int FMT>
void launch_tiled_cfg(const GemmParams &p, TileCfg c, hipStream_t s) {
  if (c.wm == 16 && c.wn == 3) launch_tiled_t<DT, SDT, 16, 3, KMAP, FMT>(p, s);
  else if (c.wm == 8 && c.wn == 2) launch_tiled_t<DT, SDT, 8, 2, KMAP, FMT>(p, s);
  else launch_tiled_t<DT, SDT, 4, 1, KMAP, FMT>(p, s);
}

template <int DT, int SDT, bool KMAP, int FMT>
void launch_plan(const GemmParams &p, const SplitPlan &sp, hipStream_t s) {
  if (sp.regime == OC_REGIME_SPLITK) launch_splitk_mt<DT, SDT, KMAP, FMT>(p, sp.mt, sp.tiles, s);
  else launch_tiled_cfg<DT, SDT, KMAP, FMT>(p, sp.tile, s);
}

template <int FMT>
void launch_dispatch(const GemmParams &p, const SplitPlan &sp, int a_dtype, int scale_dtype, bool kmap,
                     hipStream_t s) {
  // RTN parameters are read with their runtime dtypes; only the activation
  // type is a template parameter there.
  const bool bf = a_dtype == OC_DTYPE_BF16;
  if constexpr (FMT == FMT_RTN) {
    bf ? launch_plan<OC_DTYPE_BF16, OC_DTYPE_F16, false, FMT>(p, sp, s)
       : launch_plan<OC_DTYPE_F16, OC_DTYPE_F16, false, FMT>(p, sp, s);
    return;
  }
  const bool sbf = scale_dtype == OC_DTYPE_BF16;
  if (bf) {
    if (sbf) {
      kmap ? launch_plan<OC_DTYPE_BF16, OC_DTYPE_BF16, true, FMT>(p, sp, s)
           : launch_plan<OC_DTYPE_BF16, OC_DTYPE_BF16, false, FMT>(p, sp, s);
    } else {
      kmap ? launch_plan<OC_DTYPE_BF16, OC_DTYPE_F16, true, FMT>(p, sp, s)
           : launch_plan<OC_DTYPE_BF16, OC_DTYPE_F16, false, FMT>(p, sp, s);
    }
  } else {
    if (sbf) {
      kmap ? launch_plan<OC_DTYPE_F16, OC_DTYPE_BF16, true, FMT>(p, sp, s)
           : launch_plan<OC_DTYPE_F16, OC_DTYPE_BF16, false, FMT>(p, sp, s);
    } else {
      kmap ? launch_plan<OC_DTYPE_F16, OC_DTYPE_F16, true, FMT>(p, sp, s)
           : launch_plan<OC_DTYPE_F16, OC_DTYPE_F16, false, FMT>(p, sp, s);
    }
  }
}

int attach_workspace(GemmParams &p, const SplitPlan &sp, void *workspace, size_t workspace_bytes_given) {
  p.ksplit = sp.ksplit;
  p.ksteps_per_split = sp.ksteps_per_split;
  p.partials = nullptr;
  p.counters = nullptr;
  if (sp.ksplit <= 1) return OC_OK;
  const size_t need = workspace_bytes(sp, p.M, p.N);
  if (!workspace || workspace_bytes_given < need)
    return fail(OC_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                workspace ? workspace_bytes_given : static_cast<size_t>(0));
  if (!aligned(workspace, 256)) return fail(OC_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  p.counters = static_cast<int32_t *>(workspace);
  p.partials = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                         align_up(static_cast<size_t>(sp.tiles) * 4, 256));
  return OC_OK;
}

}  // namespace oc

using namespace oc;

extern "C" {

size_t oc_int4_gemm_workspace_bytes(int32_t M, int32_t N, int32_t K_phys, int32_t regime) {
  if (M <= 0 || N <= 0 || K_phys <= 0) return 0;
  return workspace_bytes(plan_gemm(M, N, K_phys, regime), M, N);
}

int oc_int4_gemm(const void *a, int64_t lda, int32_t a_dtype, int32_t M, int32_t K_logical,
                 const int32_t *qweight, const void *scales, int32_t scale_dtype,
                 const int32_t *qzeros, int32_t zero_mode, int32_t N, int32_t K_phys,
                 int32_t group_rows, const int32_t *kmap, const void *bias, int32_t bias_dtype,
                 void *c, int64_t ldc, void *workspace, size_t workspace_bytes_given, int32_t regime,
                 void *stream) {
  clear_error();
  if (M < 0 || N <= 0 || K_phys <= 0 || K_logical <= 0)
    return fail(OC_ERR_SHAPE, "bad shape M=%d N=%d K_logical=%d K_phys=%d", M, N, K_logical, K_phys);
  if (M == 0) return OC_OK;
  if (!a || !qweight || !scales || !qzeros || !c) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(a_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "a_dtype must be F16 or BF16");
  if (!is_half_dtype(scale_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "scale_dtype must be F16 or BF16");
  if (zero_mode != OC_ZERO_V1 && zero_mode != OC_ZERO_V2)
    return fail(OC_ERR_INVALID_ARGUMENT, "zero_mode must be OC_ZERO_V1 or OC_ZERO_V2");
  if (bias && !is_float_dtype(bias_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "bad bias dtype");
  if (regime < OC_REGIME_AUTO || regime > OC_REGIME_TILED)
    return fail(OC_ERR_INVALID_ARGUMENT, "unknown regime %d", regime);
  if (N % 8 != 0) return fail(OC_ERR_SHAPE, "N must be a multiple of 8 (qzeros packing), got N=%d", N);
  if (K_phys % 32 != 0 || group_rows <= 0 || group_rows % 32 != 0 || K_phys % group_rows != 0)
    return fail(OC_ERR_SHAPE, "K_phys=%d / group_rows=%d must be multiples of 32 with K_phys %% group_rows == 0",
                K_phys, group_rows);
  if (!kmap && K_logical != K_phys)
    return fail(OC_ERR_SHAPE, "K_logical=%d != K_phys=%d requires a kmap", K_logical, K_phys);
  if (lda < K_logical || ldc < N) return fail(OC_ERR_SHAPE, "lda/ldc smaller than the row length");
  if (!kmap && (lda % 8 != 0 || !aligned(a, 16)))
    return fail(OC_ERR_SHAPE, "activations need 16-byte aligned rows (lda %% 8 == 0) without kmap");
  if (!aligned(qweight, 16) || !aligned(scales, 8) || !aligned(qzeros, 4))
    return fail(OC_ERR_SHAPE, "qweight must be 16-byte and scales 8-byte aligned");
  if (regime == OC_REGIME_SPLITK && M > 64)
    return fail(OC_ERR_UNSUPPORTED, "split-K regime supports M <= 64, got M=%d", M);

  const SplitPlan sp = plan_gemm(M, N, K_phys, regime);
  GemmParams p{};
  p.a = a;
  p.lda = lda;
  p.M = M;
  p.K_logical = K_logical;
  p.qw = qweight;
  p.scales = scales;
  p.zeros = qzeros;
  p.zero_mode = zero_mode;
  p.N = N;
  p.K_phys = K_phys;
  p.group_rows = group_rows;
  p.kmap = kmap;
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.c = c;
  p.ldc = ldc;
  const int ws = attach_workspace(p, sp, workspace, workspace_bytes_given);
  if (ws != OC_OK) return ws;
  launch_dispatch<FMT_GPTQ>(p, sp, a_dtype, scale_dtype, kmap != nullptr, static_cast<hipStream_t>(stream));
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_rtn_linear(const void *x, int64_t ldx, int32_t x_dtype, int32_t M, int32_t K,
                  const uint8_t *qweight_u8, int32_t row_bytes, const void *scales, int32_t scale_dtype,
                  const void *zeros, int32_t zero_dtype, int32_t G, int32_t N, const void *bias,
                  int32_t bias_dtype, void *c, int64_t ldc, void *stream) {
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
  // kernels add it in fp32, which is exact for a 16-bit value.
  SplitPlan sp = plan_gemm(M, N, K, OC_REGIME_AUTO);
  if (sp.ksplit > 1) {  // no workspace in this entry point
    sp.ksplit = 1;
    sp.ksteps_per_split = K / 32;
  }
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
  p.N = N;
  p.K_phys = K;
  p.group_rows = 32;
  p.bias = bias;
  p.bias_dtype = bias_dtype;
  p.c = c;
  p.ldc = ldc;
  p.ksplit = 1;
  p.ksteps_per_split = sp.ksteps_per_split;
  launch_dispatch<FMT_RTN>(p, sp, x_dtype, OC_DTYPE_F16, false, static_cast<hipStream_t>(stream));
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_moe_route(const int64_t *topk_ids, int32_t T, int32_t topk, int32_t E, int32_t *expert_offsets,
                 int32_t *sorted_pairs, void *stream) {
  clear_error();
  if (!topk_ids || !expert_offsets || !sorted_pairs) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (T < 0 || topk <= 0 || E <= 0 || E > 1024 || static_cast<int64_t>(T) * topk > 65536)
    return fail(OC_ERR_SHAPE, "unsupported routing shape T=%d topk=%d E=%d", T, topk, E);
  const size_t lds = sizeof(int32_t) * (ROUTE_THREADS + 1) * E;
  if (lds > 160 * 1024) return fail(OC_ERR_UNSUPPORTED, "too many experts for one workgroup (E=%d)", E);
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(ROUTE_THREADS), lds, static_cast<hipStream_t>(stream),
                     topk_ids, T * topk, E, expert_offsets, sorted_pairs);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_int4_moe_gemm(const void *x, int64_t ldx, int32_t x_dtype, int32_t T, int32_t topk, int32_t K,
                     const int32_t *qweight, const void *scales, int32_t scale_dtype, const int32_t *qzeros,
                     int32_t zero_mode, int32_t group_rows, int32_t E, int32_t N,
                     const int32_t *expert_offsets, const int32_t *sorted_pairs, void *y, int64_t ldy,
                     void *stream) {
  clear_error();
  if (T < 0 || topk <= 0 || K <= 0 || E <= 0 || N <= 0) return fail(OC_ERR_SHAPE, "bad shape");
  if (T == 0) return OC_OK;
  if (!x || !qweight || !scales || !qzeros || !expert_offsets || !sorted_pairs || !y)
    return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(x_dtype) || !is_half_dtype(scale_dtype))
    return fail(OC_ERR_INVALID_ARGUMENT, "x and scales must be F16 or BF16");
  if (zero_mode != OC_ZERO_V1 && zero_mode != OC_ZERO_V2)
    return fail(OC_ERR_INVALID_ARGUMENT, "zero_mode must be OC_ZERO_V1 or OC_ZERO_V2");
  if (K % 32 != 0 || group_rows <= 0 || group_rows % 32 != 0 || K % group_rows != 0 || N % 64 != 0)
    return fail(OC_ERR_SHAPE, "need K %% 32 == 0, group_rows | K (multiple of 32), N %% 64 == 0");
  if (ldx % 8 != 0 || !aligned(x, 16) || ldx < K || ldy < N)
    return fail(OC_ERR_SHAPE, "x needs 16-byte aligned rows");
  GemmParams p{};
  p.a = x;
  p.lda = ldx;
  p.M = T * topk;
  p.K_logical = K;
  p.qw = qweight;
  p.scales = scales;
  p.zeros = qzeros;
  p.zero_mode = zero_mode;
  p.N = N;
  p.K_phys = K;
  p.group_rows = group_rows;
  p.c = y;
  p.ldc = ldy;
  p.ksplit = 1;
  p.ksteps_per_split = K / 32;
  p.expert_offsets = expert_offsets;
  p.sorted_pairs = sorted_pairs;
  p.topk = topk;
  p.qw_expert_stride = static_cast<int64_t>(K / 8) * N;
  p.s_expert_stride = static_cast<int64_t>(K / group_rows) * N;
  p.z_expert_stride = static_cast<int64_t>(K / group_rows) * (N / 8);
  constexpr int WM = 6, WN = 4;
  const dim3 grid((N + 64 * WN - 1) / (64 * WN), 1, E);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf = x_dtype == OC_DTYPE_BF16, sbf = scale_dtype == OC_DTYPE_BF16;
  if (bf && sbf)
    hipLaunchKernelGGL((gemm_tiled_kernel<OC_DTYPE_BF16, OC_DTYPE_BF16, WM, WN, false, FMT_GPTQ, true>), grid, dim3(256), 0, s, p);
  else if (bf)
    hipLaunchKernelGGL((gemm_tiled_kernel<OC_DTYPE_BF16, OC_DTYPE_F16, WM, WN, false, FMT_GPTQ, true>), grid, dim3(256), 0, s, p);
  else if (sbf)
    hipLaunchKernelGGL((gemm_tiled_kernel<OC_DTYPE_F16, OC_DTYPE_BF16, WM, WN, false, FMT_GPTQ, true>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_tiled_kernel<OC_DTYPE_F16, OC_DTYPE_F16, WM, WN, false, FMT_GPTQ, true>), grid, dim3(256), 0, s, p);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

}  // extern "C"
