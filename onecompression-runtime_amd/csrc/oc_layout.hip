// Load-time construction of the tiled GPTQ layout (tile16, see oc_device.h)
// and its inverse dequant, plus the activation column gather used by the
// MFMA kernels for act-order / padded-group layers.
#include <hip/hip_runtime.h>

#include "oc_device.h"
#include "oc_internal.h"

namespace oc {

namespace {

inline unsigned grid_of(int64_t n, int block = 256) {
  return static_cast<unsigned>((n + block - 1) / block);
}

// One thread per tiled word (t, ks, c, w): the physical word row r = 4ks + w
// of column n = 16t + c, whose 8 codes come from input rows kmap[8r + i].
__global__ __launch_bounds__(256) void prepare_words_kernel(const int32_t *__restrict__ qin, int K, int N,
                                                            const int32_t *__restrict__ kmap, int KS,
                                                            int tiles, uint32_t *__restrict__ qt) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(tiles) * KS * 64) return;
  const int w = static_cast<int>(idx & 3);
  const int c = static_cast<int>((idx >> 2) & 15);
  const int64_t rest = idx >> 6;
  const int ks = static_cast<int>(rest % KS);
  const int t = static_cast<int>(rest / KS);
  const int n = TILE_N * t + c;
  uint32_t word = 0;
  if (n < N) {
    const int r = 4 * ks + w;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kp = 8 * r + i;
      const int src = kmap ? kmap[kp] : (kp < K ? kp : -1);
      if (src >= 0 && src < K) {
        const uint32_t v = static_cast<uint32_t>(qin[static_cast<int64_t>(src >> 3) * N + n]);
        word |= ((v >> (4 * (src & 7))) & 0xFu) << (4 * i);
      }
    }
  }
  qt[idx] = word;
}

// One thread per (t, g, c): scale copy; threads c = 0 and c = 8 also write the
// zero word of columns c..c+7, restored to the zero itself (v1 adds 1).
__global__ __launch_bounds__(256) void prepare_meta_kernel(const uint16_t *__restrict__ scales,
                                                           const int32_t *__restrict__ qzeros, int zero_mode,
                                                           int N, int G, int tiles, uint16_t *__restrict__ st,
                                                           uint32_t *__restrict__ zt) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(tiles) * G * TILE_N) return;
  const int c = static_cast<int>(idx & 15);
  const int64_t tg = idx >> 4;  // t * G + g
  const int g = static_cast<int>(tg % G);
  const int t = static_cast<int>(tg / G);
  const int n = TILE_N * t + c;
  st[idx] = n < N ? scales[static_cast<int64_t>(g) * N + n] : static_cast<uint16_t>(0);
  if ((c & 7) == 0) {
    uint32_t out = 0;
    if (n < N) {
      const uint32_t zw = static_cast<uint32_t>(qzeros[static_cast<int64_t>(g) * (N >> 3) + (n >> 3)]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t z = (zw >> (4 * j)) & 0xFu;
        if (zero_mode == OC_ZERO_V1) z = (z + 1) & 0xFu;
        if (n + j < N) out |= z << (4 * j);
      }
    }
    zt[tg * 2 + (c >> 3)] = out;
  }
}

// Dense [N, K_logical] weight from the tiled layout (columns of the original
// K order; physical zero rows are skipped). One thread per (n, physical k).
template <int ODT>
__global__ __launch_bounds__(256) void dequant_tiled_kernel(const uint32_t *__restrict__ qt,
                                                            const uint16_t *__restrict__ st, int scale_dtype,
                                                            const uint32_t *__restrict__ zt,
                                                            const int32_t *__restrict__ kmap, int N, int K_phys,
                                                            int group_rows, int K_logical, void *__restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(N) * K_phys) return;
  const int kp = static_cast<int>(idx % K_phys);
  const int n = static_cast<int>(idx / K_phys);
  const int k = kmap ? kmap[kp] : (kp < K_logical ? kp : -1);
  if (k < 0 || k >= K_logical) return;
  const int KS = K_phys / 32, G = K_phys / group_rows;
  const int t = n / TILE_N, c = n % TILE_N;
  const int ks = kp / 32, w = (kp / 8) & 3, i = kp & 7;
  const int g = kp / group_rows;
  const uint32_t word = qt[((static_cast<int64_t>(t) * KS + ks) * TILE_N + c) * 4 + w];
  const int code = static_cast<int>((word >> (4 * i)) & 0xFu);
  const int64_t tg = static_cast<int64_t>(t) * G + g;
  const uint16_t sb = st[tg * TILE_N + c];
  const float s = scale_dtype == OC_DTYPE_BF16 ? bf16_to_f32(sb) : f16_to_f32(sb);
  const int z = tile_zero(zt[tg * 2 + (c >> 3)], c);
  const float v = s * static_cast<float>(code - z);
  const int64_t o = static_cast<int64_t>(n) * K_logical + k;
  if constexpr (ODT == OC_DTYPE_F32) static_cast<float *>(out)[o] = v;
  else static_cast<uint16_t *>(out)[o] = static_cast<uint16_t>(pack2<ODT>(v, 0.f));
}

// ---- 8-bit GPTQ (4 codes per int32, mask 0xFF) ----
// One thread per tiled word (t, ks, c, w), w = 0..7: the codes of physical
// rows 32 ks + 4 w + i (byte i) of column n = 16 t + c, from input rows kmap[.].
__global__ __launch_bounds__(256) void prepare8_words_kernel(const int32_t *__restrict__ qin, int K, int N,
                                                             const int32_t *__restrict__ kmap, int KS, int tiles,
                                                             uint32_t *__restrict__ qt) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(tiles) * KS * 128) return;
  const int w = static_cast<int>(idx & 7);
  const int c = static_cast<int>((idx >> 3) & 15);
  const int64_t rest = idx >> 7;
  const int ks = static_cast<int>(rest % KS);
  const int t = static_cast<int>(rest / KS);
  const int n = TILE_N * t + c;
  uint32_t word = 0;
  if (n < N) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kp = 32 * ks + 4 * w + i;
      const int src = kmap ? kmap[kp] : (kp < K ? kp : -1);
      if (src >= 0 && src < K) {
        const uint32_t v = static_cast<uint32_t>(qin[static_cast<int64_t>(src >> 2) * N + n]);
        word |= ((v >> (8 * (src & 3))) & 0xFFu) << (8 * i);
      }
    }
  }
  qt[idx] = word;
}

// One thread per (t, g, c): scale copy; threads with c % 4 == 0 also write the
// zero word of columns c..c+3, restored to the zero itself (v1 adds 1 mod 256).
__global__ __launch_bounds__(256) void prepare8_meta_kernel(const uint16_t *__restrict__ scales,
                                                            const int32_t *__restrict__ qzeros, int zero_mode,
                                                            int N, int G, int tiles, uint16_t *__restrict__ st,
                                                            uint32_t *__restrict__ zt) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(tiles) * G * TILE_N) return;
  const int c = static_cast<int>(idx & 15);
  const int64_t tg = idx >> 4;
  const int g = static_cast<int>(tg % G);
  const int t = static_cast<int>(tg / G);
  const int n = TILE_N * t + c;
  st[idx] = n < N ? scales[static_cast<int64_t>(g) * N + n] : static_cast<uint16_t>(0);
  if ((c & 3) == 0) {
    uint32_t out = 0;
    if (n < N) {
      const uint32_t zw = static_cast<uint32_t>(qzeros[static_cast<int64_t>(g) * (N >> 2) + (n >> 2)]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t z = (zw >> (8 * j)) & 0xFFu;
        if (zero_mode == OC_ZERO_V1) z = (z + 1) & 0xFFu;
        if (n + j < N) out |= z << (8 * j);
      }
    }
    zt[tg * 4 + (c >> 2)] = out;
  }
}

// Dense [N, K_logical] weight of an 8-bit tiled layer (as dequant_tiled_kernel).
template <int ODT>
__global__ __launch_bounds__(256) void dequant8_tiled_kernel(const uint32_t *__restrict__ qt,
                                                             const uint16_t *__restrict__ st, int scale_dtype,
                                                             const uint32_t *__restrict__ zt,
                                                             const int32_t *__restrict__ kmap, int N, int K_phys,
                                                             int group_rows, int K_logical, void *__restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(N) * K_phys) return;
  const int kp = static_cast<int>(idx % K_phys);
  const int n = static_cast<int>(idx / K_phys);
  const int k = kmap ? kmap[kp] : (kp < K_logical ? kp : -1);
  if (k < 0 || k >= K_logical) return;
  const int KS = K_phys / 32, G = K_phys / group_rows;
  const int t = n / TILE_N, c = n % TILE_N;
  const uint32_t word = qt[((static_cast<int64_t>(t) * KS + kp / 32) * TILE_N + c) * 8 + ((kp >> 2) & 7)];
  const int code = static_cast<int>((word >> (8 * (kp & 3))) & 0xFFu);
  const int64_t tg = static_cast<int64_t>(t) * G + kp / group_rows;
  const uint16_t sb = st[tg * TILE_N + c];
  const float sv = scale_dtype == OC_DTYPE_BF16 ? bf16_to_f32(sb) : f16_to_f32(sb);
  const int z = static_cast<int>((zt[tg * 4 + (c >> 2)] >> (8 * (c & 3))) & 0xFFu);
  const float v = sv * static_cast<float>(code - z);
  const int64_t o = static_cast<int64_t>(n) * K_logical + k;
  if constexpr (ODT == OC_DTYPE_F32) static_cast<float *>(out)[o] = v;
  else static_cast<uint16_t *>(out)[o] = static_cast<uint16_t>(pack2<ODT>(v, 0.f));
}

// Checkpoint-format 8-bit words: qweight [ceil(out_rows / 4), N], code row
// k = physical row row_src[k] (or k); zeros / past-K rows give zero codes.
__global__ __launch_bounds__(256) void export8_words_kernel(const uint32_t *__restrict__ qt, int KS,
                                                            const int32_t *__restrict__ row_src, int out_rows, int N,
                                                            uint32_t *__restrict__ qweight) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int rows4 = (out_rows + 3) / 4;
  if (idx >= static_cast<int64_t>(rows4) * N) return;
  const int n = static_cast<int>(idx % N);
  const int r = static_cast<int>(idx / N);
  const int t = n / TILE_N, c = n % TILE_N;
  const int K_phys = 32 * KS;
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = 4 * r + i;
    if (k >= out_rows) break;
    const int kp = row_src ? row_src[k] : k;
    if (kp < 0 || kp >= K_phys) continue;
    const uint32_t w = qt[((static_cast<int64_t>(t) * KS + kp / 32) * TILE_N + c) * 8 + ((kp >> 2) & 7)];
    word |= ((w >> (8 * (kp & 3))) & 0xFFu) << (8 * i);
  }
  qweight[idx] = word;
}

// One thread per 8-bit qzeros word (g, n / 4) and its 4 scales.
__global__ __launch_bounds__(256) void export8_meta_kernel(const uint16_t *__restrict__ st,
                                                           const uint32_t *__restrict__ zt, int G, int out_groups,
                                                           int N, int zero_mode, uint16_t *__restrict__ scales,
                                                           uint32_t *__restrict__ qzeros) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int words = N / 4;
  if (idx >= static_cast<int64_t>(out_groups) * words) return;
  const int g = static_cast<int>(idx / words);
  const int n0 = 4 * static_cast<int>(idx % words);
  const int t = n0 / TILE_N, c0 = n0 % TILE_N;
  uint32_t zout = 0;
  uint16_t sv[4] = {0, 0, 0, 0};
  if (g < G) {
    const int64_t tg = static_cast<int64_t>(t) * G + g;
    const uint32_t zw = zt[tg * 4 + (c0 >> 2)];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t z = (zw >> (8 * j)) & 0xFFu;
      if (zero_mode == OC_ZERO_V1) z = (z + 255u) & 0xFFu;
      zout |= z << (8 * j);
      sv[j] = st[tg * TILE_N + c0 + j];
    }
  }
  qzeros[idx] = zout;
  uint16_t *srow = scales + static_cast<int64_t>(g) * N + n0;
#pragma unroll
  for (int j = 0; j < 4; ++j) srow[j] = sv[j];
}

// Checkpoint-format words from the tiled layout (the inverse of
// prepare_words_kernel). One thread per output word (r, n) of
// qweight [ceil(out_rows / 8), N]: code row k = 8r + i is physical row
// row_src[k] (or k without a map); rows past out_rows, rows whose source is
// -1 and sources past K_phys give zero codes.
__global__ __launch_bounds__(256) void export_words_kernel(const uint32_t *__restrict__ qt, int KS,
                                                           const int32_t *__restrict__ row_src, int out_rows, int N,
                                                           uint32_t *__restrict__ qweight) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int rows8 = (out_rows + 7) / 8;
  if (idx >= static_cast<int64_t>(rows8) * N) return;
  const int n = static_cast<int>(idx % N);
  const int r = static_cast<int>(idx / N);
  const int t = n / TILE_N, c = n % TILE_N;
  const int K_phys = 32 * KS;
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int k = 8 * r + i;
    if (k >= out_rows) break;
    const int kp = row_src ? row_src[k] : k;
    if (kp < 0 || kp >= K_phys) continue;
    const uint32_t w = qt[((static_cast<int64_t>(t) * KS + kp / 32) * TILE_N + c) * 4 + ((kp >> 3) & 3)];
    word |= ((w >> (4 * (kp & 7))) & 0xFu) << (4 * i);
  }
  qweight[idx] = word;
}

// One thread per qzeros word (g, n / 8) and the 8 scales beside it. Groups
// past the layer's G are written as zero scales and zero stored zeros (the
// reference's K padding); a v1 checkpoint stores zero - 1 (mod 16).
__global__ __launch_bounds__(256) void export_meta_kernel(const uint16_t *__restrict__ st,
                                                          const uint32_t *__restrict__ zt, int G, int out_groups,
                                                          int N, int zero_mode, uint16_t *__restrict__ scales,
                                                          uint32_t *__restrict__ qzeros) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int words = N / 8;
  if (idx >= static_cast<int64_t>(out_groups) * words) return;
  const int g = static_cast<int>(idx / words);
  const int n0 = 8 * static_cast<int>(idx % words);
  const int t = n0 / TILE_N, c0 = n0 % TILE_N;
  uint32_t zout = 0;
  uint16_t sv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (g < G) {
    const int64_t tg = static_cast<int64_t>(t) * G + g;
    const uint32_t zw = zt[tg * 2 + (c0 >> 3)];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t z = (zw >> (4 * j)) & 0xFu;
      if (zero_mode == OC_ZERO_V1) z = (z + 15u) & 0xFu;
      zout |= z << (4 * j);
      sv[j] = st[tg * TILE_N + c0 + j];
    }
  }
  qzeros[idx] = zout;
  uint16_t *srow = scales + static_cast<int64_t>(g) * N + n0;
#pragma unroll
  for (int j = 0; j < 8; ++j) srow[j] = sv[j];
}

}  // namespace

namespace {
// Activations in physical row order: out[m, k'] = a[m, kmap[k']], or 0 where
// kmap[k'] is outside [0, K_logical) (the -1 of a padding row).
__global__ __launch_bounds__(256) void gather_cols_kernel(const uint16_t *__restrict__ a, int64_t lda, int M,
                                                          int K_logical, const int32_t *__restrict__ kmap,
                                                          int K_phys, uint16_t *__restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(M) * K_phys) return;
  const int kp = static_cast<int>(idx % K_phys);
  const int64_t m = idx / K_phys;
  const int src = kmap[kp];
  out[idx] = static_cast<unsigned>(src) < static_cast<unsigned>(K_logical) ? a[m * lda + src]
                                                                          : static_cast<uint16_t>(0);
}
}  // namespace

namespace {
// The same permutation by rows through the inverse map: one workgroup per
// activation row reads the row and kinv contiguously, scatters into LDS
// (physical order; rows without a source stay zero) and writes the physical
// row out contiguously. Every global access is coalesced, unlike the gather's
// one cache line per lane.
constexpr int SCATTER_ROW_MAX = 32768;  // physical rows per LDS row buffer (64 KB)

__global__ __launch_bounds__(1024) void scatter_rows_kernel(const uint16_t *__restrict__ a, int64_t lda,
                                                            int K_logical, const uint16_t *__restrict__ kinv,
                                                            int K_phys, uint16_t *__restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint16_t row[SCATTER_ROW_MAX];
  const int m = blockIdx.x, tid = threadIdx.x;
  uint4 *row4 = reinterpret_cast<uint4 *>(row);
  if (K_phys != K_logical)
    for (int i = tid; i < K_phys / 8; i += blockDim.x) row4[i] = make_uint4(0, 0, 0, 0);
  __syncthreads();
  const uint16_t *src = a + static_cast<int64_t>(m) * lda;
  // Octets of 8 logical rows (16-byte loads of the row and of kinv), then the K % 8 tail.
  const int octets = K_logical >> 3;
  for (int o = tid; o < octets; o += blockDim.x) {
    const uint4 xv = reinterpret_cast<const uint4 *>(src)[o];
    const uint4 rv = reinterpret_cast<const uint4 *>(kinv)[o];
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, rw[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r0 = static_cast<int>(rw[j] & 0xFFFFu), r1 = static_cast<int>(rw[j] >> 16);
      if (r0 < K_phys) row[r0] = static_cast<uint16_t>(xw[j]);
      if (r1 < K_phys) row[r1] = static_cast<uint16_t>(xw[j] >> 16);
    }
  }
  for (int k = 8 * octets + tid; k < K_logical; k += blockDim.x) {
    const int r = kinv[k];
    if (r < K_phys) row[r] = src[k];
  }
  __syncthreads();
  uint4 *dst = reinterpret_cast<uint4 *>(out + static_cast<int64_t>(m) * K_phys);
  for (int i = tid; i < K_phys / 8; i += blockDim.x) dst[i] = row4[i];
}
}  // namespace

constexpr int SCATTER_MIN_ROWS = 32;  // rows from which one workgroup per row pays

void launch_gather_cols(const void *a, int64_t lda, int M, int K_logical, const int32_t *kmap,
                        const uint16_t *kinv, int K_phys, void *out, void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  // One workgroup per row pays for many rows; a few rows (M = 8: 8 workgroups)
  // spread better as one thread per physical element.
  if (kinv && K_phys <= SCATTER_ROW_MAX && M >= SCATTER_MIN_ROWS) {
    hipLaunchKernelGGL(scatter_rows_kernel, dim3(M), dim3(1024), 0, s, static_cast<const uint16_t *>(a), lda,
                       K_logical, kinv, K_phys, static_cast<uint16_t *>(out));
    return;
  }
  const int64_t total = static_cast<int64_t>(M) * K_phys;
  hipLaunchKernelGGL(gather_cols_kernel, dim3(grid_of(total)), dim3(256), 0, s, static_cast<const uint16_t *>(a),
                     lda, M, K_logical, kmap, K_phys, static_cast<uint16_t *>(out));
}

}  // namespace oc

using namespace oc;

extern "C" {

int oc_int4_prepare(const int32_t *qweight, int32_t K, int32_t N, const int32_t *kmap, int32_t K_phys,
                    int32_t group_rows, const void *scales, int32_t scale_dtype, const int32_t *qzeros,
                    int32_t zero_mode, int32_t *qt, void *st, int32_t *zt, void *stream) {
  clear_error();
  if (!qweight || !scales || !qzeros || !qt || !st || !zt) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(scale_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "scale_dtype must be F16 or BF16");
  if (zero_mode != OC_ZERO_V1 && zero_mode != OC_ZERO_V2)
    return fail(OC_ERR_INVALID_ARGUMENT, "zero_mode must be OC_ZERO_V1 or OC_ZERO_V2");
  if (K <= 0 || N <= 0 || N % 8 != 0 || K_phys <= 0 || K_phys % 32 != 0 || group_rows <= 0 ||
      group_rows % 32 != 0 || K_phys % group_rows != 0)
    return fail(OC_ERR_SHAPE, "bad shape K=%d N=%d K_phys=%d group_rows=%d", K, N, K_phys, group_rows);
  const int tiles = (N + TILE_N - 1) / TILE_N;
  const int KS = K_phys / 32, G = K_phys / group_rows;
  if (static_cast<int64_t>(tiles) * KS * 256 >= (1LL << 31))  // kernels address the words with 32-bit byte offsets
    return fail(OC_ERR_UNSUPPORTED, "layer too large: packed words of 2 GiB or more (K_phys=%d N=%d)", K_phys, N);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t words = static_cast<int64_t>(tiles) * KS * 64;
  hipLaunchKernelGGL(prepare_words_kernel, dim3(grid_of(words)), dim3(256), 0, s, qweight, K, N, kmap, KS, tiles,
                     reinterpret_cast<uint32_t *>(qt));
  const int64_t metas = static_cast<int64_t>(tiles) * G * TILE_N;
  hipLaunchKernelGGL(prepare_meta_kernel, dim3(grid_of(metas)), dim3(256), 0, s,
                     static_cast<const uint16_t *>(scales), qzeros, zero_mode, N, G, tiles,
                     static_cast<uint16_t *>(st), reinterpret_cast<uint32_t *>(zt));
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_int4_export(const int32_t *qt, const void *st, const int32_t *zt, int32_t N, int32_t K_phys,
                   int32_t group_rows, const int32_t *row_src, int32_t out_rows, int32_t out_groups,
                   int32_t zero_mode, int32_t *qweight, void *scales, int32_t *qzeros, void *stream) {
  clear_error();
  if (!qt || !st || !zt || !qweight || !scales || !qzeros) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (zero_mode != OC_ZERO_V1 && zero_mode != OC_ZERO_V2)
    return fail(OC_ERR_INVALID_ARGUMENT, "zero_mode must be OC_ZERO_V1 or OC_ZERO_V2");
  if (N <= 0 || N % 8 != 0 || K_phys <= 0 || K_phys % 32 != 0 || group_rows <= 0 || group_rows % 32 != 0 ||
      K_phys % group_rows != 0 || out_rows <= 0 || out_groups <= 0)
    return fail(OC_ERR_SHAPE, "bad shape N=%d K_phys=%d group_rows=%d out_rows=%d out_groups=%d", N, K_phys,
                group_rows, out_rows, out_groups);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t words = static_cast<int64_t>((out_rows + 7) / 8) * N;
  hipLaunchKernelGGL(export_words_kernel, dim3(grid_of(words)), dim3(256), 0, s,
                     reinterpret_cast<const uint32_t *>(qt), K_phys / 32, row_src, out_rows, N,
                     reinterpret_cast<uint32_t *>(qweight));
  const int64_t metas = static_cast<int64_t>(out_groups) * (N / 8);
  hipLaunchKernelGGL(export_meta_kernel, dim3(grid_of(metas)), dim3(256), 0, s, static_cast<const uint16_t *>(st),
                     reinterpret_cast<const uint32_t *>(zt), K_phys / group_rows, out_groups, N, zero_mode,
                     static_cast<uint16_t *>(scales), reinterpret_cast<uint32_t *>(qzeros));
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_int8_prepare(const int32_t *qweight, int32_t K, int32_t N, const int32_t *kmap, int32_t K_phys,
                    int32_t group_rows, const void *scales, int32_t scale_dtype, const int32_t *qzeros,
                    int32_t zero_mode, int32_t *qt, void *st, int32_t *zt, void *stream) {
  clear_error();
  if (!qweight || !scales || !qzeros || !qt || !st || !zt) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(scale_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "scale_dtype must be F16 or BF16");
  if (zero_mode != OC_ZERO_V1 && zero_mode != OC_ZERO_V2)
    return fail(OC_ERR_INVALID_ARGUMENT, "zero_mode must be OC_ZERO_V1 or OC_ZERO_V2");
  if (K <= 0 || N <= 0 || N % 4 != 0 || K_phys <= 0 || K_phys % 32 != 0 || group_rows <= 0 ||
      group_rows % 32 != 0 || K_phys % group_rows != 0)
    return fail(OC_ERR_SHAPE, "bad shape K=%d N=%d K_phys=%d group_rows=%d", K, N, K_phys, group_rows);
  const int tiles = (N + TILE_N - 1) / TILE_N;
  const int KS = K_phys / 32, G = K_phys / group_rows;
  if (static_cast<int64_t>(tiles) * KS * 512 >= (1LL << 31))
    return fail(OC_ERR_UNSUPPORTED, "layer too large: packed words of 2 GiB or more (K_phys=%d N=%d)", K_phys, N);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t words = static_cast<int64_t>(tiles) * KS * 128;
  hipLaunchKernelGGL(prepare8_words_kernel, dim3(grid_of(words)), dim3(256), 0, s, qweight, K, N, kmap, KS, tiles,
                     reinterpret_cast<uint32_t *>(qt));
  const int64_t metas = static_cast<int64_t>(tiles) * G * TILE_N;
  hipLaunchKernelGGL(prepare8_meta_kernel, dim3(grid_of(metas)), dim3(256), 0, s,
                     static_cast<const uint16_t *>(scales), qzeros, zero_mode, N, G, tiles,
                     static_cast<uint16_t *>(st), reinterpret_cast<uint32_t *>(zt));
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_int8_export(const int32_t *qt, const void *st, const int32_t *zt, int32_t N, int32_t K_phys,
                   int32_t group_rows, const int32_t *row_src, int32_t out_rows, int32_t out_groups,
                   int32_t zero_mode, int32_t *qweight, void *scales, int32_t *qzeros, void *stream) {
  clear_error();
  if (!qt || !st || !zt || !qweight || !scales || !qzeros) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (zero_mode != OC_ZERO_V1 && zero_mode != OC_ZERO_V2)
    return fail(OC_ERR_INVALID_ARGUMENT, "zero_mode must be OC_ZERO_V1 or OC_ZERO_V2");
  if (N <= 0 || N % 4 != 0 || K_phys <= 0 || K_phys % 32 != 0 || group_rows <= 0 || group_rows % 32 != 0 ||
      K_phys % group_rows != 0 || out_rows <= 0 || out_groups <= 0)
    return fail(OC_ERR_SHAPE, "bad shape N=%d K_phys=%d group_rows=%d out_rows=%d out_groups=%d", N, K_phys,
                group_rows, out_rows, out_groups);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t words = static_cast<int64_t>((out_rows + 3) / 4) * N;
  hipLaunchKernelGGL(export8_words_kernel, dim3(grid_of(words)), dim3(256), 0, s,
                     reinterpret_cast<const uint32_t *>(qt), K_phys / 32, row_src, out_rows, N,
                     reinterpret_cast<uint32_t *>(qweight));
  const int64_t metas = static_cast<int64_t>(out_groups) * (N / 4);
  hipLaunchKernelGGL(export8_meta_kernel, dim3(grid_of(metas)), dim3(256), 0, s, static_cast<const uint16_t *>(st),
                     reinterpret_cast<const uint32_t *>(zt), K_phys / group_rows, out_groups, N, zero_mode,
                     static_cast<uint16_t *>(scales), reinterpret_cast<uint32_t *>(qzeros));
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_int8_dequant_tiled(const int32_t *qt, const void *st, int32_t scale_dtype, const int32_t *zt,
                          const int32_t *kmap, int32_t N, int32_t K_phys, int32_t group_rows, int32_t K_logical,
                          void *out, int32_t out_dtype, void *stream) {
  clear_error();
  if (!qt || !st || !zt || !out) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(scale_dtype) || !is_float_dtype(out_dtype))
    return fail(OC_ERR_INVALID_ARGUMENT, "bad scale/out dtype");
  if (N <= 0 || K_phys <= 0 || K_phys % 32 != 0 || group_rows <= 0 || group_rows % 32 != 0 ||
      K_phys % group_rows != 0 || K_logical <= 0 || (!kmap && K_logical > K_phys))
    return fail(OC_ERR_SHAPE, "bad shape N=%d K_phys=%d group_rows=%d K_logical=%d", N, K_phys, group_rows,
                K_logical);
  const int64_t total = static_cast<int64_t>(N) * K_phys;
  auto kern = out_dtype == OC_DTYPE_BF16   ? dequant8_tiled_kernel<OC_DTYPE_BF16>
              : out_dtype == OC_DTYPE_F16 ? dequant8_tiled_kernel<OC_DTYPE_F16>
                                          : dequant8_tiled_kernel<OC_DTYPE_F32>;
  hipLaunchKernelGGL(kern, dim3(grid_of(total)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint32_t *>(qt), static_cast<const uint16_t *>(st), scale_dtype,
                     reinterpret_cast<const uint32_t *>(zt), kmap, N, K_phys, group_rows, K_logical, out);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_int4_dequant_tiled(const int32_t *qt, const void *st, int32_t scale_dtype, const int32_t *zt,
                          const int32_t *kmap, int32_t N, int32_t K_phys, int32_t group_rows, int32_t K_logical,
                          void *out, int32_t out_dtype, void *stream) {
  clear_error();
  if (!qt || !st || !zt || !out) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_half_dtype(scale_dtype) || !is_float_dtype(out_dtype))
    return fail(OC_ERR_INVALID_ARGUMENT, "bad scale/out dtype");
  if (N <= 0 || K_phys <= 0 || K_phys % 32 != 0 || group_rows <= 0 || group_rows % 32 != 0 ||
      K_phys % group_rows != 0 || K_logical <= 0 || (!kmap && K_logical > K_phys))
    return fail(OC_ERR_SHAPE, "bad shape N=%d K_phys=%d group_rows=%d K_logical=%d", N, K_phys, group_rows,
                K_logical);
  const int64_t total = static_cast<int64_t>(N) * K_phys;
  auto kern = out_dtype == OC_DTYPE_BF16   ? dequant_tiled_kernel<OC_DTYPE_BF16>
              : out_dtype == OC_DTYPE_F16 ? dequant_tiled_kernel<OC_DTYPE_F16>
                                          : dequant_tiled_kernel<OC_DTYPE_F32>;
  hipLaunchKernelGGL(kern, dim3(grid_of(total)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint32_t *>(qt), static_cast<const uint16_t *>(st), scale_dtype,
                     reinterpret_cast<const uint32_t *>(zt), kmap, N, K_phys, group_rows, K_logical, out);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

}  // extern "C"
