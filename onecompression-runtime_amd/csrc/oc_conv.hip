// Packed int4 Conv1d / ConvTranspose1d (reference layers/packed_conv.py:123-222)
// as GEMMs over the RTN nibble rows, for gfx950.
//
// Conv1d (groups = 1): out[b, o, t] = sum_{ci, kk} W[o, ci * k + kk] *
// x[b, ci, t * stride + kk * dilation - pad_left]. Output positions are taken
// in chunks of rows (b, t); each chunk's activation rows are written to the
// workspace in the weight's column order (im2col, zeros outside [0, L)), the
// LDS-tiled RTN kernel multiplies them into fp32 partials, and the epilogue
// adds the K splits in order and the bias and rounds once into [B, O, T].
//
// ConvTranspose1d (groups = 1): out[b, o, t] = sum_{ci, kk, j : j * stride +
// kk * dilation - padding = t} x[b, ci, j] W[ci, o * k + kk]. The stored rows
// are input channels with quant groups along the output columns, so at load
// time the codes are re-laid transposed (rows = output columns (o, kk), K =
// ci) with the scales and zeros as [groups][C_in] (FMT_RTN_T reads the 8 K
// rows' parameters of its lane). Per chunk of input positions j of one batch
// row the GEMM gives Z[j, (o, kk)] in fp32; the scatter adds each output's
// taps (kk ascending) into an fp32 accumulator, which the last pass rounds
// with the bias. Chunks are added in order, so results are deterministic.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "oc_gemm_common.h"

namespace oc {
namespace {

inline unsigned grid_1d(int64_t n, int block = 256) { return static_cast<unsigned>((n + block - 1) / block); }

// A[r, c] (r < rows, c < K) for output rows r0 + r = b * T + t.
__global__ __launch_bounds__(256) void im2col_kernel(const uint16_t *__restrict__ x, int C, int L, int k,
                                                     int stride, int dilation, int pad_left, int T, int64_t r0,
                                                     int rows, int K, uint16_t *__restrict__ a) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(rows) * K) return;
  const int c = static_cast<int>(idx % K);
  const int64_t r = r0 + idx / K;
  const int b = static_cast<int>(r / T), t = static_cast<int>(r % T);
  const int ci = c / k, kk = c % k;
  const int pos = t * stride + kk * dilation - pad_left;
  a[idx] = (pos >= 0 && pos < L) ? x[(static_cast<int64_t>(b) * C + ci) * L + pos] : static_cast<uint16_t>(0);
}

// The same rows by tiles of I2C_TR output rows x I2C_CB input channels: the
// tile's input window (channels ci0.., positions t0 * stride - pad_left ..,
// W of them, zeros outside [0, L)) is read once into LDS (a wave reads 64
// consecutive positions of each of its 8 channels per pass, the 8 loads in
// flight together), then every output row's I2C_CB * k columns are written as
// 16-byte chunks. A tile whose rows span two batch rows reads its values from
// global memory instead. 128 rows per tile: the window rows (W positions of
// a channel) span fewer partial cache lines than at 64.
constexpr int I2C_TR = 128, I2C_CB = 32;
inline int i2c_window(int k, int stride, int dilation) { return (I2C_TR - 1) * stride + (k - 1) * dilation + 1; }

__global__ __launch_bounds__(256) void im2col_tile_kernel(const uint16_t *__restrict__ x, int C, int L, int k,
                                                          int stride, int dilation, int pad_left, int T, int64_t r0,
                                                          int rows, int K, int W, uint16_t *__restrict__ a) {
  extern __shared__ uint16_t win[];  // [I2C_CB][W]
  const int64_t ra = r0 + static_cast<int64_t>(blockIdx.x) * I2C_TR;  // first row of the tile
  const int nrow = static_cast<int>(min<int64_t>(I2C_TR, r0 + rows - ra));
  const int b0 = static_cast<int>(ra / T), t0 = static_cast<int>(ra % T);
  const bool one_batch = (ra + nrow - 1) / T == b0;
  const int ci0 = blockIdx.y * I2C_CB;
  if (one_batch) {
    const int p0 = t0 * stride - pad_left;
    const uint16_t *xb = x + (static_cast<int64_t>(b0) * C + ci0) * L;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int CPW = I2C_CB / 4;  // channels per wave
    for (int q0 = 0; q0 < W; q0 += 64) {
      const int q = q0 + lane, pos = p0 + q;
      const bool in = q < W && pos >= 0 && pos < L;
      uint16_t v[CPW];
#pragma unroll
      for (int u = 0; u < CPW; ++u)
        v[u] = in ? xb[static_cast<int64_t>(wave + 4 * u) * L + pos] : static_cast<uint16_t>(0);
      if (q < W) {
#pragma unroll
        for (int u = 0; u < CPW; ++u) win[(wave + 4 * u) * W + q] = v[u];
      }
    }
    __syncthreads();
  }
  const int CH = I2C_CB * k / 8;  // 16-byte chunks of one row in this channel block
  if (one_batch && CH <= 256) {
    // A thread keeps one chunk column j (its 8 window offsets computed once)
    // and walks the rows 256 / CH apart.
    const int RS = 256 / CH, j = threadIdx.x % CH;
    if (threadIdx.x >= RS * CH) return;
    int off[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int cc = 8 * j + e, ci = cc / k;
      off[e] = ci * W + (cc - ci * k) * dilation;
    }
    uint16_t *dst = a + (ra - r0) * K + static_cast<int64_t>(ci0) * k + 8 * j;
    for (int rr = threadIdx.x / CH; rr < nrow; rr += RS) {
      uint32_t v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = win[off[e] + rr * stride];
      *reinterpret_cast<uint4 *>(dst + static_cast<int64_t>(rr) * K) =
          make_uint4(v[0] | v[1] << 16, v[2] | v[3] << 16, v[4] | v[5] << 16, v[6] | v[7] << 16);
    }
    return;
  }
  for (int i = threadIdx.x; i < nrow * CH; i += blockDim.x) {
    const int rr = i / CH, j = i - rr * CH;
    const int64_t r = ra + rr;
    uint32_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int cc = 8 * j + e, ci = cc / k, kk = cc - ci * k;
      if (one_batch) {
        v[e] = win[ci * W + rr * stride + kk * dilation];
      } else {
        const int64_t b = r / T;
        const int pos = static_cast<int>(r % T) * stride + kk * dilation - pad_left;
        v[e] = pos >= 0 && pos < L ? x[(b * C + ci0 + ci) * L + pos] : 0u;
      }
    }
    *reinterpret_cast<uint4 *>(a + (r - r0) * K + static_cast<int64_t>(ci0) * k + 8 * j) =
        make_uint4(v[0] | v[1] << 16, v[2] | v[3] << 16, v[4] | v[5] << 16, v[6] | v[7] << 16);
  }
}

// out[b, o, t] for the chunk's rows: the K splits of the fp32 partials in
// order, plus bias, rounded once. Tiles of EP_R rows x EP_N columns pass
// through LDS: the partials are read along their rows (columns fastest) and
// the outputs written along t, both coalesced.
constexpr int EP_R = 64, EP_N = 64;
template <int DT>
__global__ __launch_bounds__(256) void conv1d_epilogue_tile_kernel(const float *__restrict__ part, int ksplit,
                                                                   int rows, int N, int T, int64_t r0,
                                                                   const void *bias, int bias_dtype,
                                                                   void *__restrict__ y) {
  __shared__ float tile[EP_R][EP_N + 1];
  __shared__ float bs[EP_N];  // the tile's biases (no global loads among the stores)
  const int rb = static_cast<int>(blockIdx.x) * EP_R, nb = static_cast<int>(blockIdx.y) * EP_N;
  if (threadIdx.x < EP_N)
    bs[threadIdx.x] = bias && nb + static_cast<int>(threadIdx.x) < N ? load_any_f32(bias, nb + threadIdx.x, bias_dtype)
                                                                      : 0.f;
  const int64_t mn = static_cast<int64_t>(rows) * N;
  constexpr int U = EP_R * EP_N / 256;
  if ((N & 3) == 0) {
    // 16-byte loads of 4 columns (N % 4 == 0: a run never leaves its row).
    constexpr int U4 = U / 4, C4 = EP_N / 4;
    int64_t e[U4];
    float4 v[U4];
#pragma unroll
    for (int u = 0; u < U4; ++u) {
      const int i = threadIdx.x + 256 * u, rr = i / C4, c = 4 * (i % C4);
      e[u] = rb + rr < rows && nb + c < N ? static_cast<int64_t>(rb + rr) * N + nb + c : -1;
      v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int sp = 0; sp < ksplit; ++sp) {
#pragma unroll
      for (int u = 0; u < U4; ++u)
        if (e[u] >= 0) {
          const float4 t = *reinterpret_cast<const float4 *>(part + sp * mn + e[u]);
          v[u].x += t.x;
          v[u].y += t.y;
          v[u].z += t.z;
          v[u].w += t.w;
        }
    }
#pragma unroll
    for (int u = 0; u < U4; ++u) {
      const int i = threadIdx.x + 256 * u, rr = i / C4, c = 4 * (i % C4);
      tile[rr][c] = v[u].x;
      tile[rr][c + 1] = v[u].y;
      tile[rr][c + 2] = v[u].z;
      tile[rr][c + 3] = v[u].w;
    }
  } else {
    int64_t e[U];
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = threadIdx.x + 256 * u, rr = i / EP_N, nn = i % EP_N;
      e[u] = rb + rr < rows && nb + nn < N ? static_cast<int64_t>(rb + rr) * N + nb + nn : -1;
      v[u] = 0.f;
    }
    for (int sp = 0; sp < ksplit; ++sp) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (e[u] >= 0) v[u] += part[sp * mn + e[u]];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = threadIdx.x + 256 * u;
      tile[i / EP_N][i % EP_N] = v[u];
    }
  }
  __syncthreads();
  const int64_t ra = r0 + rb;
  const int64_t b0 = ra / T;
  const int t0 = static_cast<int>(ra - b0 * T);
  if ((T & 1) == 0) {
    // Pairs of positions as 4-byte stores: T even keeps t0 (ra is even) and
    // every pair's first position even, so a pair never leaves its batch row.
    uint32_t *y32 = static_cast<uint32_t *>(y);
#pragma unroll
    for (int u = 0; u < U / 2; ++u) {
      const int i = threadIdx.x + 256 * u, nn = i / (EP_R / 2), rr = 2 * (i % (EP_R / 2)), n = nb + nn;
      if (rb + rr >= rows || n >= N) continue;
      float v0 = tile[rr][nn], v1 = tile[rr + 1][nn];
      if (bias) {
        v0 += bs[nn];
        v1 += bs[nn];
      }
      int t = t0 + rr;
      int64_t b = b0;
      while (t >= T) {
        t -= T;
        ++b;
      }
      const int64_t o = (b * N + n) * T + t;
      if (rb + rr + 1 < rows) y32[o >> 1] = pack2<DT>(v0, v1);
      else store_c<DT>(y, o, v0);
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = threadIdx.x + 256 * u, nn = i / EP_R, rr = i % EP_R, n = nb + nn;
    if (rb + rr >= rows || n >= N) continue;
    float val = tile[rr][nn];
    if (bias) val += bs[nn];
    int t = t0 + rr;
    int64_t b = b0;
    while (t >= T) {  // rows of the tile past the end of a batch row
      t -= T;
      ++b;
    }
    store_c<DT>(y, (b * N + n) * T + t, val);
  }
}

// Transposed-weight re-layout: codes [C_in rows, cols] (RTN nibbles) ->
// [cols rows, C_in / 2 bytes]; one thread per output byte (n, ci pair).
__global__ __launch_bounds__(256) void rtn_transpose_kernel(const uint8_t *__restrict__ q, int rows, int row_bytes,
                                                            int cols, uint8_t *__restrict__ qt) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int half = rows / 2;
  if (idx >= static_cast<int64_t>(cols) * half) return;
  const int n = static_cast<int>(idx / half), i = static_cast<int>(idx % half);
  uint32_t v = 0;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int ci = 2 * i + e;
    const uint8_t byte = q[static_cast<int64_t>(ci) * row_bytes + n / 2];
    v |= ((n & 1) ? (byte >> 4) : (byte & 0xF)) << (4 * e);
  }
  qt[idx] = static_cast<uint8_t>(v);
}

// [rows, G] 16-bit -> [G, rows].
__global__ __launch_bounds__(256) void transpose16_kernel(const uint16_t *__restrict__ in, int rows, int G,
                                                          uint16_t *__restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(rows) * G) return;
  const int g = static_cast<int>(idx / rows), r = static_cast<int>(idx % rows);
  out[idx] = in[static_cast<int64_t>(r) * G + g];
}

// A[j, ci] = x[b, ci, j0 + j] for the chunk's input positions, by 64 x 64
// tiles through LDS: read along the positions, written as channel pairs
// along the rows (C even), both coalesced.
constexpr int PT = 64;
__global__ __launch_bounds__(256) void positions_to_rows_tile_kernel(const uint16_t *__restrict__ x, int C, int L,
                                                                     int b, int j0, int rows,
                                                                     uint16_t *__restrict__ a) {
  __shared__ uint16_t tile[PT][PT + 2];
  const int jb = static_cast<int>(blockIdx.x) * PT, cb = static_cast<int>(blockIdx.y) * PT;
  constexpr int NL = PT * PT / 256;  // loads per thread, all in flight
  uint16_t v[NL];
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int i = threadIdx.x + 256 * u, cc = i / PT, jj = i % PT, ci = cb + cc, j = jb + jj;
    v[u] = ci < C && j < rows ? x[(static_cast<int64_t>(b) * C + ci) * L + j0 + j] : static_cast<uint16_t>(0);
  }
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int i = threadIdx.x + 256 * u;
    tile[i / PT][i % PT] = v[u];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < PT * PT / 2; i += 256) {
    const int jj = i / (PT / 2), cp = 2 * (i % (PT / 2)), j = jb + jj, ci = cb + cp;
    if (j < rows && ci < C)
      *reinterpret_cast<uint32_t *>(a + static_cast<int64_t>(j) * C + ci) =
          tile[cp][jj] | static_cast<uint32_t>(tile[cp + 1][jj]) << 16;
  }
}

// acc[o, t] += taps of input positions j0 .. j0 + rows - 1, kk ascending, for
// t in [t_lo, t_hi). Z = the chunk's partials [ksplit][rows][O * k].
__global__ __launch_bounds__(256) void col2im_add_kernel(const float *__restrict__ part, int ksplit, int rows, int O,
                                                         int k, int stride, int dilation, int padding, int j0,
                                                         int t_lo, int t_hi, int Lout, float *__restrict__ acc) {
  const int span = t_hi - t_lo;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(span) * O) return;
  const int t = t_lo + static_cast<int>(idx % span);
  const int o = static_cast<int>(idx / span);
  const int N = O * k;
  const int64_t mn = static_cast<int64_t>(rows) * N;
  float v = 0.f;
  for (int kk = 0; kk < k; ++kk) {
    const int num = t + padding - kk * dilation;
    if (num < 0 || num % stride != 0) continue;
    const int j = num / stride - j0;
    if (j < 0 || j >= rows) continue;
    for (int s = 0; s < ksplit; ++s) v += part[s * mn + static_cast<int64_t>(j) * N + o * k + kk];
  }
  acc[static_cast<int64_t>(o) * Lout + t] += v;
}

// The same sums by tiles of CT_T output positions x CT_O output channels: the
// input rows that reach the tile (JR of them, the K splits already added) are
// read into LDS along the GEMM's columns, then each output adds its taps (kk
// ascending, as above). FINAL (one chunk covers the whole input): the output
// is written directly with the bias, rounded once (no accumulator pass).
constexpr int CT_T = 128, CT_O = 16;
__host__ __device__ inline int floor_div(int a, int b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }
inline int col2im_rows(int k, int stride, int dilation) { return (CT_T - 1 + (k - 1) * dilation) / stride + 2; }

template <int DT, bool FINAL>
__global__ __launch_bounds__(256) void col2im_tile_kernel(const float *__restrict__ part, int ksplit, int rows, int O,
                                                          int k, int stride, int dilation, int padding, int j0,
                                                          int t_lo, int t_hi, int Lout, int JR,
                                                          float *__restrict__ acc, const void *bias, int bias_dtype,
                                                          void *__restrict__ y) {
  extern __shared__ __attribute__((aligned(16))) float zs[];  // [JR][CT_O * k + 8] (rows 8 floats apart
                                                              // in bank: conflict-free tap reads)
  __shared__ float bs[CT_O];                                  // the tile's biases
  const int t0 = t_lo + static_cast<int>(blockIdx.x) * CT_T, o0 = static_cast<int>(blockIdx.y) * CT_O;
  const int N = O * k, W = CT_O * k;
  const int wlim = min(W, (O - o0) * k);  // columns of the tile's channels that exist
  const int64_t mn = static_cast<int64_t>(rows) * N;
  const int jlo = floor_div(t0 + padding - (k - 1) * dilation, stride);  // first input position reaching the tile
  const int total = JR * W, WS = W + 8;
  if (FINAL && threadIdx.x < CT_O)
    bs[threadIdx.x] = bias && o0 + static_cast<int>(threadIdx.x) < O ? load_any_f32(bias, o0 + threadIdx.x, bias_dtype)
                                                                      : 0.f;
  // U independent loads per thread in flight (one chain per element); with
  // N % 4 == 0 (then the tile's columns are whole 16-byte runs: o0 k and the
  // existing width N - o0 k are multiples of 4) as 16-byte loads.
  constexpr int U = 8;
  if ((N & 3) == 0) {
    const int W4 = W >> 2, tot4 = total >> 2;
    // (row, column) of element i = threadIdx.x + 256 n, advanced by 256
    // elements per step (one division per thread, none per element)
    const int dq = 256 / W4, dr = 256 - dq * W4;
    int jj = static_cast<int>(threadIdx.x) / W4, c4 = static_cast<int>(threadIdx.x) - jj * W4;
    for (int i0 = threadIdx.x; i0 < tot4; i0 += U * 256) {
      int64_t e[U];
      int li[U];
      float4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * 256;
        const int c = 4 * c4;
        const int j = jlo + jj - j0;
        li[u] = (jj * WS + c) >> 2;
        e[u] = i < tot4 && j >= 0 && j < rows && c < wlim
                   ? static_cast<int64_t>(j) * N + static_cast<int64_t>(o0) * k + c
                   : -1;
        v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        jj += dq;
        c4 += dr;
        if (c4 >= W4) {
          c4 -= W4;
          ++jj;
        }
      }
      for (int sp = 0; sp < ksplit; ++sp) {
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (e[u] >= 0) {
            const float4 t = *reinterpret_cast<const float4 *>(part + sp * mn + e[u]);
            v[u].x += t.x;
            v[u].y += t.y;
            v[u].z += t.z;
            v[u].w += t.w;
          }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (i0 + u * 256 < tot4) reinterpret_cast<float4 *>(zs)[li[u]] = v[u];
    }
  } else
  for (int i0 = threadIdx.x; i0 < total; i0 += U * 256) {
    int64_t e[U];
    int li[U];
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * 256;
      const int jj = i / W, c = i - jj * W;
      const int j = jlo + jj - j0;  // row of the chunk
      li[u] = jj * WS + c;
      e[u] = i < total && j >= 0 && j < rows && c < wlim ? static_cast<int64_t>(j) * N + static_cast<int64_t>(o0) * k + c
                                                          : -1;
      v[u] = 0.f;
    }
    for (int sp = 0; sp < ksplit; ++sp) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (e[u] >= 0) v[u] += part[sp * mn + e[u]];
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u * 256 < total) zs[li[u]] = v[u];
  }
  __syncthreads();
  const int dmax = (k - 1) * dilation;
  // A thread keeps one position t of the tile and takes NO of its channels
  // (ol = olb, olb + 2, ...): the taps depend on t only, so they are walked
  // once for all NO sums. Taps kk ascending = input positions j descending
  // (j * stride = t + padding - kk * dilation); only the positions that are
  // whole multiples are visited.
  static_assert(CT_T * 2 == 256, "two channel rows per pass of 256 threads");
  constexpr int NO = CT_O / 2;
  const int tl = static_cast<int>(threadIdx.x) % CT_T, olb = static_cast<int>(threadIdx.x) / CT_T;
  const int t = t0 + tl;
  if (t >= t_hi) return;
  float v[NO];
#pragma unroll
  for (int u = 0; u < NO; ++u) v[u] = 0.f;
  const int base = t + padding;
  for (int j = floor_div(base, stride); j >= jlo; --j) {
    const int d = base - j * stride;  // kk * dilation
    if (d > dmax || j < j0) break;
    if (j >= j0 + rows) continue;
    int kk = d;
    if (dilation != 1) {
      if (d % dilation != 0) continue;
      kk = d / dilation;
    }
    const float *zr = zs + (j - jlo) * WS + olb * k + kk;
#pragma unroll
    for (int u = 0; u < NO; ++u) v[u] += zr[2 * u * k];
  }
#pragma unroll
  for (int u = 0; u < NO; ++u) {
    const int ol = olb + 2 * u, o = o0 + ol;
    if (o >= O) break;
    if constexpr (FINAL) {
      store_c<DT>(y, static_cast<int64_t>(o) * Lout + t, bias ? v[u] + bs[ol] : v[u]);
    } else {
      acc[static_cast<int64_t>(o) * Lout + t] += v[u];
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void finish_kernel(const float *__restrict__ acc, int O, int Lout, const void *bias,
                                                     int bias_dtype, void *__restrict__ y) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(O) * Lout) return;
  const int o = static_cast<int>(idx / Lout);
  float v = acc[idx];
  if (bias) v += load_any_f32(bias, o, bias_dtype);
  store_c<DT>(y, idx, v);
}

__global__ __launch_bounds__(256) void zero_f32_kernel(float *__restrict__ p, int64_t n) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx < n) p[idx] = 0.f;
}

// RTN rows -> the large-M kernel's tiles (tile16 words): word (t, ks, c, w)
// = codes of K rows 32 ks + 8 w .. + 7 of output column 16 t + c, which in
// an RTN row are 4 consecutive bytes (code i at bits 4 i either way).
__global__ __launch_bounds__(256) void rtn_tile_words_kernel(const uint8_t *__restrict__ q, int N, int row_bytes,
                                                             int KS, int tiles, uint32_t *__restrict__ qt) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(tiles) * KS * 64) return;
  const int w = static_cast<int>(idx & 3), c = static_cast<int>((idx >> 2) & 15);
  const int64_t tk = idx >> 6;
  const int ks = static_cast<int>(tk % KS), n = static_cast<int>(tk / KS) * 16 + c;
  qt[idx] = n < N ? *reinterpret_cast<const uint32_t *>(q + static_cast<int64_t>(n) * row_bytes + 16 * ks + 4 * w)
                  : 0u;
}

__global__ void rtn_tile_flags_kernel(int *fast) {
  if (threadIdx.x < 2) fast[threadIdx.x] = 1;
}

// Per (tile, group, column): scale | zero << 16 (16-bit values as stored;
// columns past N zero). fast[0] / fast[1] are cleared when a column's group
// parameter does not allow the exact single-rounding dequant for bf16 /
// fp16 activations (rtn_fast_ok on the values rounded to that dtype).
__global__ __launch_bounds__(256) void rtn_tile_params_kernel(const uint16_t *__restrict__ sc,
                                                              const uint16_t *__restrict__ zr, int N, int G,
                                                              int tiles, int sdt, uint32_t *__restrict__ sz,
                                                              int *fast) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(tiles) * G * 16) return;
  const int c = static_cast<int>(idx & 15);
  const int64_t tg = idx >> 4;
  const int g = static_cast<int>(tg % G), n = static_cast<int>(tg / G) * 16 + c;
  if (n >= N) {
    sz[idx] = 0u;
    return;
  }
  const uint32_t sv = sc[static_cast<int64_t>(n) * G + g], zv = zr[static_cast<int64_t>(n) * G + g];
  sz[idx] = sv | zv << 16;
  const float s = sdt == OC_DTYPE_BF16 ? half_to_f32<OC_DTYPE_BF16>(sv) : half_to_f32<OC_DTYPE_F16>(sv);
  const float z = sdt == OC_DTYPE_BF16 ? half_to_f32<OC_DTYPE_BF16>(zv) : half_to_f32<OC_DTYPE_F16>(zv);
  RtnParam pb, ph;
  pb.sq = round_to<OC_DTYPE_BF16>(s);
  pb.zq = round_to<OC_DTYPE_BF16>(z);
  ph.sq = round_to<OC_DTYPE_F16>(s);
  ph.zq = round_to<OC_DTYPE_F16>(z);
  if (!rtn_fast_ok<OC_DTYPE_BF16>(pb)) atomicAnd(&fast[0], 0);
  if (!rtn_fast_ok<OC_DTYPE_F16>(ph)) atomicAnd(&fast[1], 0);
}

// A weight whose quant groups run along its columns ([K rows, N cols], the
// ConvTranspose1d layout) -> the same tiles: word (t, ks, c, w) gathers the
// codes of rows 32 ks + 8 w + i (i < 8, at bits 4 i) of column 16 t + c.
__global__ __launch_bounds__(256) void rtnt_tile_words_kernel(const uint8_t *__restrict__ q, int row_bytes, int N,
                                                              int KS, int tiles, uint32_t *__restrict__ qt) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(tiles) * KS * 64) return;
  const int w = static_cast<int>(idx & 3), c = static_cast<int>((idx >> 2) & 15);
  const int64_t tk = idx >> 6;
  const int ks = static_cast<int>(tk % KS), n = static_cast<int>(tk / KS) * 16 + c;
  uint32_t v = 0;
  if (n < N) {
    const uint8_t *col = q + (n >> 1) + static_cast<int64_t>(32 * ks + 8 * w) * row_bytes;
#pragma unroll
    for (int i = 0; i < 8; ++i) v |= ((col[static_cast<int64_t>(i) * row_bytes] >> (4 * (n & 1))) & 0xFu) << (4 * i);
  }
  qt[idx] = v;
}

// Per (tile, K row): sq | zq << 16, the row's scale and zero for the tile's
// column group (host: groups of a multiple of 16 columns) rounded to DT and
// stored as DT bits; zero past N. fast[0] is cleared where rtn_fast_ok<DT>
// fails.
template <int DT>
__global__ __launch_bounds__(256) void rtnt_tile_rows_kernel(const uint16_t *__restrict__ sc,
                                                             const uint16_t *__restrict__ zr, int K, int N, int G,
                                                             int tiles, int sdt, uint32_t *__restrict__ szt,
                                                             int *fast) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(tiles) * K) return;
  const int row = static_cast<int>(idx % K), n0 = static_cast<int>(idx / K) * 16;
  if (n0 >= N) {
    szt[idx] = 0u;
    return;
  }
  const int64_t e = static_cast<int64_t>(row) * G + n0 / (N / G);
  const float s = sdt == OC_DTYPE_BF16 ? half_to_f32<OC_DTYPE_BF16>(sc[e]) : half_to_f32<OC_DTYPE_F16>(sc[e]);
  const float z = sdt == OC_DTYPE_BF16 ? half_to_f32<OC_DTYPE_BF16>(zr[e]) : half_to_f32<OC_DTYPE_F16>(zr[e]);
  RtnParam rp;
  rp.sq = round_to<DT>(s);
  rp.zq = round_to<DT>(z);
  szt[idx] = pack2<DT>(rp.sq, rp.zq);
  if (!rtn_fast_ok<DT>(rp)) atomicAnd(fast, 0);
}

// Large-M conv GEMM (the tiled RTN kernel below this many rows per chunk).
constexpr int WIDE_CONV_MIN_ROWS = 1024;

// Large-M plan of a rows x N x K chunk: K slices (each 16 K steps or more)
// enough to fill the compute units with 256-row workgroups, for column
// blocks of 64 wn; *wn (when given) gets the block width, 192 or 128, whose
// grid keeps the most CUs busy on useful columns (ties: 192); without wn,
// 192 only.
int wide_conv_ksplit(int rows, int N, int K, int *kps, int *wn = nullptr) {
  const int KS = K / 32, cus = device_cus();
  double best = -1.0;
  int best_ks = 1, best_wn = 3;
  for (int w : {3, 2}) {
    if (w == 2 && !wn) continue;
    const int nbn = (N + 64 * w - 1) / (64 * w), base = nbn * ((rows + 255) / 256);
    const int ks = std::max(1, std::min(cus / std::max(1, base), KS / 16));
    const int kp = (KS + ks - 1) / ks, ksr = (KS + kp - 1) / kp;
    const int64_t wgs = static_cast<int64_t>(base) * ksr;
    const double fill = static_cast<double>(wgs) / (static_cast<double>((wgs + cus - 1) / cus) * cus);
    const double useful = static_cast<double>(N) / (static_cast<double>(nbn) * 64 * w);
    if (fill * useful > best + 0.02) {
      best = fill * useful;
      best_ks = ksr;
      best_wn = w;
      *kps = kp;
    }
  }
  if (wn) *wn = best_wn;
  return best_ks;
}

// Rows per chunk: a bounded workspace (activation rows plus fp32 partials),
// the rows spread evenly over the chunks (multiples of 256), so that no
// chunk is a small remainder whose GEMM fills a fraction of the chip.
constexpr size_t CONV_CHUNK_BYTES = size_t{128} << 20;

int chunk_rows(int64_t total, int K, int N) {
  const int64_t per_row = 2 * static_cast<int64_t>(K) + 4 * static_cast<int64_t>(N);
  const int64_t rmax = std::max<int64_t>(256, static_cast<int64_t>(CONV_CHUNK_BYTES) / per_row) / 256 * 256;
  if (total <= rmax) return static_cast<int>(total);
  const int64_t chunks = (total + rmax - 1) / rmax;
  const int64_t r = ((total + chunks - 1) / chunks + 255) / 256 * 256;
  return static_cast<int>(std::min(r, rmax));
}

// Workspace of one chunk of `rows` rows: activations, then fp32 partials
// (as many K splits as the tiled or the large-M plan of the chunk takes).
size_t chunk_bytes(int rows, int K, int N) {
  int wm, wn, kg, ksplit, kps;
  plan_tiled(rows, N, K, &wm, &wn, &kg, &ksplit, &kps);
  if (rows >= WIDE_CONV_MIN_ROWS) {
    int wn;
    ksplit = std::max(ksplit, wide_conv_ksplit(rows, N, K, &kps, &wn));
  }
  const size_t a = (static_cast<size_t>(rows) * K * 2 + 255) / 256 * 256;
  return a + static_cast<size_t>(ksplit) * rows * N * sizeof(float);
}

size_t conv_chunks_bytes(int64_t total, int K, int N) {
  if (total <= 0) return 0;
  const int r = chunk_rows(total, K, N);
  const int rem = static_cast<int>(total % r);
  return std::max(chunk_bytes(r, K, N), rem ? chunk_bytes(rem, K, N) : size_t{0});
}

// One chunk's GEMM: A [rows, K] (in the workspace) times the packed rows into
// fp32 partials right after A. Returns the K splits.
int chunk_gemm(const void *a, int x_dtype, int rows, int K, const uint8_t *q, int row_bytes, const void *scales,
               int scale_dtype, const void *zeros, int zero_dtype, int gs, int64_t stride_n, int64_t stride_g,
               int N, bool transposed, float *part, hipStream_t s) {
  int wm, wn, kg, ksplit, kps;
  plan_tiled(rows, N, K, &wm, &wn, &kg, &ksplit, &kps);
  GemmParams p{};
  p.a = a;
  p.lda = K;
  p.M = rows;
  p.K_logical = K;
  p.qw = q;
  p.scales = scales;
  p.zeros = zeros;
  p.scale_dtype = scale_dtype;
  p.zero_dtype = zero_dtype;
  p.rtn_gs = gs;
  p.rtn_G = K / gs;
  p.row_bytes = row_bytes;
  p.sz_stride_n = stride_n;
  p.sz_stride_g = stride_g;
  p.N = N;
  p.K_phys = K;
  p.KS = K / 32;
  p.group_rows = 32;
  p.gshift = 0;
  p.partials = part;
  p.out_f32 = 1;
  p.ksplit = ksplit;
  p.ksteps_per_split = kps;
  launch_rtn_tiled(p, x_dtype, transposed, wm, wn, kg, s);
  return ksplit;
}

}  // namespace
}  // namespace oc

using namespace oc;

extern "C" {

size_t oc_rtn_conv1d_workspace_bytes(int32_t B, int32_t C_in, int32_t C_out, int32_t kernel_size, int32_t T_out) {
  const int64_t K = static_cast<int64_t>(C_in) * kernel_size;
  if (B <= 0 || T_out <= 0 || K <= 0 || K > (1 << 30)) return 0;
  return conv_chunks_bytes(static_cast<int64_t>(B) * T_out, static_cast<int>(K), C_out);
}

int oc_rtn_tile_prepare(const uint8_t *qweight, int32_t N, int32_t row_bytes, int32_t K, const void *scales,
                        const void *zeros, int32_t dtype, int32_t G, int32_t *qt, uint32_t *sz, int32_t *fast,
                        void *stream) {
  clear_error();
  if (!qweight || !scales || !zeros || !qt || !sz || !fast) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (N <= 0 || K <= 0 || K % 32 != 0 || G <= 0 || K % G != 0 || (K / G) % 32 != 0 || row_bytes < K / 2 ||
      row_bytes % 4 != 0)
    return fail(OC_ERR_SHAPE, "tile layout needs K %% 32 == 0, groups of a multiple of 32 columns and 4-byte rows "
                "(N=%d K=%d G=%d row_bytes=%d)", N, K, G, row_bytes);
  if (dtype != OC_DTYPE_F16 && dtype != OC_DTYPE_BF16)
    return fail(OC_ERR_INVALID_ARGUMENT, "scales and zeros must share a 16-bit dtype");
  if (!aligned(qweight, 4)) return fail(OC_ERR_SHAPE, "misaligned weight");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int tiles = (N + 15) / 16, KS = K / 32;
  hipLaunchKernelGGL(rtn_tile_words_kernel, dim3(grid_1d(static_cast<int64_t>(tiles) * KS * 64)), dim3(256), 0, s,
                     qweight, N, row_bytes, KS, tiles, reinterpret_cast<uint32_t *>(qt));
  hipLaunchKernelGGL(rtn_tile_flags_kernel, dim3(1), dim3(64), 0, s, fast);
  hipLaunchKernelGGL(rtn_tile_params_kernel, dim3(grid_1d(static_cast<int64_t>(tiles) * G * 16)), dim3(256), 0, s,
                     static_cast<const uint16_t *>(scales), static_cast<const uint16_t *>(zeros), N, G, tiles, dtype,
                     sz, fast);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_rtn_tile_prepare_t(const uint8_t *qweight, int32_t K, int32_t row_bytes, int32_t N, const void *scales,
                          const void *zeros, int32_t scale_dtype, int32_t G, int32_t x_dtype, int32_t *qt,
                          uint32_t *szt, int32_t *fast, void *stream) {
  clear_error();
  if (!qweight || !scales || !zeros || !qt || !szt || !fast) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (K <= 0 || K % 32 != 0 || N <= 0 || G <= 0 || N % G != 0 || (N / G) % 16 != 0 || row_bytes < (N + 1) / 2)
    return fail(OC_ERR_SHAPE, "transposed tile layout needs K %% 32 == 0 and groups of a multiple of 16 columns "
                "(K=%d N=%d G=%d row_bytes=%d)", K, N, G, row_bytes);
  if (!is_half_dtype(scale_dtype) || !is_half_dtype(x_dtype))
    return fail(OC_ERR_INVALID_ARGUMENT, "scales/zeros and activations must be F16 or BF16");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int tiles = (N + 15) / 16, KS = K / 32;
  hipLaunchKernelGGL(rtnt_tile_words_kernel, dim3(grid_1d(static_cast<int64_t>(tiles) * KS * 64)), dim3(256), 0, s,
                     qweight, row_bytes, N, KS, tiles, reinterpret_cast<uint32_t *>(qt));
  hipLaunchKernelGGL(rtn_tile_flags_kernel, dim3(1), dim3(64), 0, s, fast);
  const dim3 g(grid_1d(static_cast<int64_t>(tiles) * K));
  if (x_dtype == OC_DTYPE_BF16)
    hipLaunchKernelGGL(rtnt_tile_rows_kernel<OC_DTYPE_BF16>, g, dim3(256), 0, s, static_cast<const uint16_t *>(scales),
                       static_cast<const uint16_t *>(zeros), K, N, G, tiles, scale_dtype, szt, fast);
  else
    hipLaunchKernelGGL(rtnt_tile_rows_kernel<OC_DTYPE_F16>, g, dim3(256), 0, s, static_cast<const uint16_t *>(scales),
                       static_cast<const uint16_t *>(zeros), K, N, G, tiles, scale_dtype, szt, fast);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_rtn_conv1d(const void *x, int32_t x_dtype, int32_t B, int32_t C_in, int32_t L, const uint8_t *qweight,
                  int32_t row_bytes, const void *scales, int32_t scale_dtype, const void *zeros, int32_t zero_dtype,
                  int32_t G, int32_t C_out, int32_t kernel_size, int32_t stride, int32_t dilation, int32_t pad_left,
                  int32_t T_out, const void *bias, int32_t bias_dtype, void *y, void *workspace,
                  size_t workspace_bytes, void *stream) {
  return oc_rtn_conv1d_prepared(x, x_dtype, B, C_in, L, qweight, row_bytes, scales, scale_dtype, zeros, zero_dtype,
                                G, nullptr, nullptr, 0, C_out, kernel_size, stride, dilation, pad_left, T_out, bias,
                                bias_dtype, y, workspace, workspace_bytes, stream);
}

int oc_rtn_conv1d_prepared(const void *x, int32_t x_dtype, int32_t B, int32_t C_in, int32_t L,
                           const uint8_t *qweight, int32_t row_bytes, const void *scales, int32_t scale_dtype,
                           const void *zeros, int32_t zero_dtype, int32_t G, const int32_t *qt, const uint32_t *sz,
                           int32_t tiles_fast, int32_t C_out, int32_t kernel_size, int32_t stride, int32_t dilation,
                           int32_t pad_left, int32_t T_out, const void *bias, int32_t bias_dtype, void *y,
                           void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  if (B < 0 || C_in <= 0 || L < 0 || C_out <= 0 || kernel_size <= 0 || stride <= 0 || dilation <= 0 || T_out < 0 ||
      G <= 0)
    return fail(OC_ERR_SHAPE, "bad conv shape");
  if (B == 0 || T_out == 0) return OC_OK;
  if (!x || !qweight || !scales || !zeros || !y) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(x_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "x_dtype must be F16 or BF16");
  if (!is_float_dtype(scale_dtype) || dtype_bytes(zero_dtype) == 0)
    return fail(OC_ERR_INVALID_ARGUMENT, "unsupported scale/zero dtype");
  if (bias && !is_float_dtype(bias_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "bad bias dtype");
  const int64_t K64 = static_cast<int64_t>(C_in) * kernel_size;
  if (K64 % 32 != 0 || K64 % G != 0 || (K64 / G) % 8 != 0 || row_bytes < K64 / 2 || row_bytes % 4 != 0)
    return fail(OC_ERR_UNSUPPORTED,
                "fused conv1d needs C_in * kernel_size %% 32 == 0, groups of a multiple of 8 columns and "
                "4-byte weight rows (K=%lld G=%d row_bytes=%d)", static_cast<long long>(K64), G, row_bytes);
  const int K = static_cast<int>(K64);
  const int64_t total = static_cast<int64_t>(B) * T_out;
  const size_t need = conv_chunks_bytes(total, K, C_out);
  if (!workspace || workspace_bytes < need)
    return fail(OC_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                workspace ? workspace_bytes : static_cast<size_t>(0));
  if (!aligned(workspace, 256) || !aligned(qweight, 4)) return fail(OC_ERR_SHAPE, "misaligned workspace or weight");
  if ((qt && !aligned(qt, 16)) || (sz && !aligned(sz, 4))) return fail(OC_ERR_SHAPE, "misaligned tile layout");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The large-M kernel on the tile layout: 16-bit scales and zeros of one
  // dtype, power-of-two group steps, every group fast-dequant eligible for
  // x_dtype (tiles_fast, as oc_rtn_tile_prepare reported it); ONECOMP_HIP_CONV_WIDE=0
  // (read per call; tests) keeps the tiled kernel.
  const int gs = K / G;
  const bool wide = qt && sz && tiles_fast && scale_dtype == zero_dtype && is_half_dtype(scale_dtype) &&
                    gs % 32 == 0 && ilog2_exact(gs / 32) >= 0 && C_out % 8 == 0 &&
                    env_int("ONECOMP_HIP_CONV_WIDE", 1) != 0;
  const int R = chunk_rows(total, K, C_out);
  for (int64_t r0 = 0; r0 < total; r0 += R) {
    const int rows = static_cast<int>(std::min<int64_t>(R, total - r0));
    uint16_t *a = static_cast<uint16_t *>(workspace);
    float *part = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                            (static_cast<size_t>(rows) * K * 2 + 255) / 256 * 256);
    const int W = i2c_window(kernel_size, stride, dilation);
    if (C_in % I2C_CB == 0 && static_cast<size_t>(I2C_CB) * W * 2 <= 48 * 1024)
      hipLaunchKernelGGL(im2col_tile_kernel, dim3((rows + I2C_TR - 1) / I2C_TR, C_in / I2C_CB), dim3(256),
                         static_cast<size_t>(I2C_CB) * W * 2, s, static_cast<const uint16_t *>(x), C_in, L,
                         kernel_size, stride, dilation, pad_left, T_out, r0, rows, K, W, a);
    else
      hipLaunchKernelGGL(im2col_kernel, dim3(grid_1d(static_cast<int64_t>(rows) * K)), dim3(256), 0, s,
                         static_cast<const uint16_t *>(x), C_in, L, kernel_size, stride, dilation, pad_left, T_out,
                         r0, rows, K, a);
    int ksplit;
    if (wide && rows >= WIDE_CONV_MIN_ROWS && static_cast<int64_t>(rows) * K * 2 < (int64_t{1} << 31)) {
      GemmParams p{};
      p.a = a;
      p.lda = K;
      p.a_bytes = static_cast<int64_t>(rows) * K * 2;
      p.M = rows;
      p.K_logical = K;
      p.qw = qt;
      p.scales = sz;
      p.N = C_out;
      p.K_phys = K;
      p.KS = K / 32;
      p.G = G;
      p.group_rows = gs;
      p.gshift = ilog2_exact(gs / 32);
      p.partials = part;
      p.out_f32 = 1;
      int wn;
      p.ksplit = wide_conv_ksplit(rows, C_out, K, &p.ksteps_per_split, &wn);
      launch_rtn_wide(p, x_dtype, scale_dtype, wn, s);
      ksplit = p.ksplit;
    } else {
      ksplit = chunk_gemm(a, x_dtype, rows, K, qweight, row_bytes, scales, scale_dtype, zeros, zero_dtype, K / G, G,
                          1, C_out, false, part, s);
    }
    const dim3 grid((rows + EP_R - 1) / EP_R, (C_out + EP_N - 1) / EP_N);
    if (x_dtype == OC_DTYPE_BF16)
      hipLaunchKernelGGL(conv1d_epilogue_tile_kernel<OC_DTYPE_BF16>, grid, dim3(256), 0, s, part, ksplit, rows, C_out,
                         T_out, r0, bias, bias_dtype, y);
    else
      hipLaunchKernelGGL(conv1d_epilogue_tile_kernel<OC_DTYPE_F16>, grid, dim3(256), 0, s, part, ksplit, rows, C_out,
                         T_out, r0, bias, bias_dtype, y);
  }
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_rtn_transpose_prepare(const uint8_t *qweight, int32_t rows, int32_t row_bytes, int32_t cols,
                             const void *scales, const void *zeros, int32_t G, uint8_t *qweight_t, void *scales_t,
                             void *zeros_t, void *stream) {
  clear_error();
  if (!qweight || !scales || !zeros || !qweight_t || !scales_t || !zeros_t)
    return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (rows <= 0 || rows % 2 != 0 || cols <= 0 || row_bytes < (cols + 1) / 2 || G <= 0)
    return fail(OC_ERR_SHAPE, "bad shape rows=%d cols=%d row_bytes=%d G=%d", rows, cols, row_bytes, G);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(rtn_transpose_kernel, dim3(grid_1d(static_cast<int64_t>(cols) * (rows / 2))), dim3(256), 0, s,
                     qweight, rows, row_bytes, cols, qweight_t);
  const dim3 g(grid_1d(static_cast<int64_t>(rows) * G));
  hipLaunchKernelGGL(transpose16_kernel, g, dim3(256), 0, s, static_cast<const uint16_t *>(scales), rows, G,
                     static_cast<uint16_t *>(scales_t));
  hipLaunchKernelGGL(transpose16_kernel, g, dim3(256), 0, s, static_cast<const uint16_t *>(zeros), rows, G,
                     static_cast<uint16_t *>(zeros_t));
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

size_t oc_rtn_conv_transpose1d_workspace_bytes(int32_t B, int32_t C_in, int32_t L_in, int32_t C_out,
                                               int32_t kernel_size, int32_t L_out) {
  if (B <= 0 || L_in <= 0 || C_in <= 0 || C_out <= 0 || kernel_size <= 0 || L_out <= 0) return 0;
  const int N = C_out * kernel_size;
  const size_t acc = (static_cast<size_t>(C_out) * L_out * sizeof(float) + 255) / 256 * 256;
  return acc + conv_chunks_bytes(L_in, C_in, N);
}

int oc_rtn_conv_transpose1d(const void *x, int32_t x_dtype, int32_t B, int32_t C_in, int32_t L_in,
                            const uint8_t *qweight_t, const void *scales_t, const void *zeros_t, int32_t scale_dtype,
                            int32_t G, int32_t C_out, int32_t kernel_size, int32_t stride, int32_t dilation,
                            int32_t padding, int32_t L_out, const void *bias, int32_t bias_dtype, void *y,
                            void *workspace, size_t workspace_bytes, void *stream) {
  return oc_rtn_conv_transpose1d_prepared(x, x_dtype, B, C_in, L_in, qweight_t, scales_t, zeros_t, scale_dtype, G,
                                          nullptr, nullptr, 0, C_out, kernel_size, stride, dilation, padding, L_out,
                                          bias, bias_dtype, y, workspace, workspace_bytes, stream);
}

int oc_rtn_conv_transpose1d_prepared(const void *x, int32_t x_dtype, int32_t B, int32_t C_in, int32_t L_in,
                                     const uint8_t *qweight_t, const void *scales_t, const void *zeros_t,
                                     int32_t scale_dtype, int32_t G, const int32_t *qt, const uint32_t *szt,
                                     int32_t tiles_fast, int32_t C_out, int32_t kernel_size, int32_t stride,
                                     int32_t dilation, int32_t padding, int32_t L_out, const void *bias,
                                     int32_t bias_dtype, void *y, void *workspace, size_t workspace_bytes,
                                     void *stream) {
  clear_error();
  if (B < 0 || C_in <= 0 || L_in < 0 || C_out <= 0 || kernel_size <= 0 || stride <= 0 || dilation <= 0 ||
      L_out < 0 || G <= 0 || padding < 0)
    return fail(OC_ERR_SHAPE, "bad conv-transpose shape");
  if (B == 0 || L_in == 0 || L_out == 0) return OC_OK;
  if (!x || !qweight_t || !scales_t || !zeros_t || !y) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(x_dtype) || !is_half_dtype(scale_dtype))
    return fail(OC_ERR_INVALID_ARGUMENT, "x and scales/zeros must be F16 or BF16");
  if (bias && !is_float_dtype(bias_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "bad bias dtype");
  const int N = C_out * kernel_size;
  if (C_in % 32 != 0 || N % G != 0)
    return fail(OC_ERR_UNSUPPORTED, "fused conv-transpose needs C_in %% 32 == 0 and groups dividing the columns");
  const size_t need = oc_rtn_conv_transpose1d_workspace_bytes(B, C_in, L_in, C_out, kernel_size, L_out);
  if (!workspace || workspace_bytes < need)
    return fail(OC_ERR_WORKSPACE, "workspace of %zu bytes required, %zu given", need,
                workspace ? workspace_bytes : static_cast<size_t>(0));
  if (!aligned(workspace, 256) || !aligned(qweight_t, 4) || !aligned(scales_t, 16) || !aligned(zeros_t, 16))
    return fail(OC_ERR_SHAPE, "misaligned workspace or weights");
  if ((qt && !aligned(qt, 16)) || (szt && !aligned(szt, 16))) return fail(OC_ERR_SHAPE, "misaligned tile layout");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The large-M kernel on the transposed tile layout (prepared for x_dtype,
  // tiles_fast as oc_rtn_tile_prepare_t reported it) for chunks of
  // WIDE_CONV_MIN_ROWS or more positions; ONECOMP_HIP_CONV_WIDE=0 (read per
  // call; tests) keeps the tiled kernel.
  const bool wide = qt && szt && tiles_fast && (N / G) % 16 == 0 && N % 8 == 0 &&
                    env_int("ONECOMP_HIP_CONV_WIDE", 1) != 0;
  float *acc = static_cast<float *>(workspace);
  char *chunk_ws = static_cast<char *>(workspace) + (static_cast<size_t>(C_out) * L_out * 4 + 255) / 256 * 256;
  const int R = chunk_rows(L_in, C_in, N);
  const int64_t outs = static_cast<int64_t>(C_out) * L_out;
  const int span_max = (R - 1) * stride + (kernel_size - 1) * dilation + 1;
  const int JR = col2im_rows(kernel_size, stride, dilation);
  const size_t tile_lds = static_cast<size_t>(JR) * (CT_O * kernel_size + 8) * 4;
  const bool tiled = tile_lds <= 48 * 1024;
  const bool direct = tiled && R >= L_in;  // one chunk: outputs written by the col2im pass itself
  const bool bf = x_dtype == OC_DTYPE_BF16;
  for (int b = 0; b < B; ++b) {
    void *yb = static_cast<char *>(y) + static_cast<size_t>(b) * outs * 2;
    if (!direct) hipLaunchKernelGGL(zero_f32_kernel, dim3(grid_1d(outs)), dim3(256), 0, s, acc, outs);
    for (int j0 = 0; j0 < L_in; j0 += R) {
      const int rows = std::min(R, L_in - j0);
      uint16_t *a = reinterpret_cast<uint16_t *>(chunk_ws);
      float *part = reinterpret_cast<float *>(chunk_ws + (static_cast<size_t>(rows) * C_in * 2 + 255) / 256 * 256);
      hipLaunchKernelGGL(positions_to_rows_tile_kernel, dim3((rows + PT - 1) / PT, (C_in + PT - 1) / PT), dim3(256), 0,
                         s, static_cast<const uint16_t *>(x), C_in, L_in, b, j0, rows, a);
      int ksplit;
      if (wide && rows >= WIDE_CONV_MIN_ROWS) {
        GemmParams p{};
        p.a = a;
        p.lda = C_in;
        p.a_bytes = static_cast<int64_t>(rows) * C_in * 2;
        p.M = rows;
        p.K_logical = C_in;
        p.qw = qt;
        p.scales = szt;
        p.N = N;
        p.K_phys = C_in;
        p.KS = C_in / 32;
        p.G = 1;
        p.group_rows = C_in;
        p.gshift = 0;
        p.partials = part;
        p.out_f32 = 1;
        int wn;
        p.ksplit = wide_conv_ksplit(rows, N, C_in, &p.ksteps_per_split, &wn);
        launch_rtnt_wide(p, x_dtype, wn, s);
        ksplit = p.ksplit;
      } else {
        ksplit = chunk_gemm(a, x_dtype, rows, C_in, qweight_t, C_in / 2, scales_t, scale_dtype, zeros_t, scale_dtype,
                            N / G, 0, 0, N, true, part, s);
      }
      int t_lo = std::max(0, j0 * stride - padding);
      int t_hi = std::min(L_out, (j0 + rows - 1) * stride + (kernel_size - 1) * dilation - padding + 1);
      if (direct) {
        t_lo = 0;  // every output, tapped or not (bias only)
        t_hi = L_out;
      }
      if (t_hi <= t_lo) continue;
      (void)span_max;
      if (tiled) {
        const dim3 g((t_hi - t_lo + CT_T - 1) / CT_T, (C_out + CT_O - 1) / CT_O);
        if (direct && bf)
          hipLaunchKernelGGL((col2im_tile_kernel<OC_DTYPE_BF16, true>), g, dim3(256), tile_lds, s, part, ksplit, rows,
                             C_out, kernel_size, stride, dilation, padding, j0, t_lo, t_hi, L_out, JR, acc, bias,
                             bias_dtype, yb);
        else if (direct)
          hipLaunchKernelGGL((col2im_tile_kernel<OC_DTYPE_F16, true>), g, dim3(256), tile_lds, s, part, ksplit, rows,
                             C_out, kernel_size, stride, dilation, padding, j0, t_lo, t_hi, L_out, JR, acc, bias,
                             bias_dtype, yb);
        else
          hipLaunchKernelGGL((col2im_tile_kernel<OC_DTYPE_F16, false>), g, dim3(256), tile_lds, s, part, ksplit, rows,
                             C_out, kernel_size, stride, dilation, padding, j0, t_lo, t_hi, L_out, JR, acc, bias,
                             bias_dtype, yb);
      } else {
        hipLaunchKernelGGL(col2im_add_kernel, dim3(grid_1d(static_cast<int64_t>(t_hi - t_lo) * C_out)), dim3(256),
                           0, s, part, ksplit, rows, C_out, kernel_size, stride, dilation, padding, j0, t_lo, t_hi,
                           L_out, acc);
      }
    }
    if (direct) continue;
    if (x_dtype == OC_DTYPE_BF16)
      hipLaunchKernelGGL(finish_kernel<OC_DTYPE_BF16>, dim3(grid_1d(outs)), dim3(256), 0, s, acc, C_out, L_out, bias,
                         bias_dtype, yb);
    else
      hipLaunchKernelGGL(finish_kernel<OC_DTYPE_F16>, dim3(grid_1d(outs)), dim3(256), 0, s, acc, C_out, L_out, bias,
                         bias_dtype, yb);
  }
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

}  // extern "C"
