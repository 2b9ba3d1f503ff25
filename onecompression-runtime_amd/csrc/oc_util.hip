// Status/error API, the host-side group-layout planner, and the
// memory-bound kernels on checkpoint-format tensors: integer unpack, GPTQ and
// RTN dequant to a dense weight, and the packed RTN embedding gather.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <vector>

#include "oc_device.h"
#include "oc_internal.h"

namespace oc {

namespace {
thread_local char g_last_error[512] = {0};
}

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_last_error[0] = 0; }

// ---------------------------------------------------------------------------
// Integer unpack along dim 0 (see oc_unpack_rows).
__global__ __launch_bounds__(256) void unpack_rows_kernel(const int32_t *__restrict__ packed, int cols,
                                                          int wbits, int num_rows,
                                                          int32_t *__restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(num_rows) * cols) return;
  const int c = static_cast<int>(idx % cols);
  const int r = static_cast<int>(idx / cols);
  const int per_word = 32 / wbits;
  const uint32_t w = static_cast<uint32_t>(packed[static_cast<int64_t>(r / per_word) * cols + c]);
  out[idx] = static_cast<int32_t>((w >> (wbits * (r % per_word))) & ((1u << wbits) - 1u));
}

// ---------------------------------------------------------------------------
// GPTQ dequant to out[N, K] (see oc_int4_dequant). One thread per packed word
// of one column: consecutive threads walk along K so the stores coalesce.
template <int ODT>
__device__ __forceinline__ void store_out(void *out, int64_t i, float v) {
  if constexpr (ODT == OC_DTYPE_F32) {
    static_cast<float *>(out)[i] = v;
  } else {
    static_cast<uint16_t *>(out)[i] = static_cast<uint16_t>(pack2<ODT>(v, 0.f));
  }
}

// Fast path: 4-bit codes, contiguous groups (groupsize % 8 == 0), 16-bit
// scales and output, K % 8 == 0. Uses the same dequant8() the GEMM kernels use.
template <int ODT>
__global__ __launch_bounds__(256) void gptq_dequant4_kernel(
    const int32_t *__restrict__ qweight, const uint16_t *__restrict__ scales, int scale_dtype,
    const int32_t *__restrict__ qzeros, int zero_mode, int groupsize, int K, int N,
    uint4 *__restrict__ out) {
  const int KW = K / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(KW) * N) return;
  const int kw = static_cast<int>(idx % KW);
  const int n = static_cast<int>(idx / KW);
  const int g = (8 * kw) / groupsize;
  const uint16_t sb = scales[static_cast<int64_t>(g) * N + n];
  const float s = scale_dtype == OC_DTYPE_BF16 ? bf16_to_f32(sb) : f16_to_f32(sb);
  const int z = unpack_zero(static_cast<uint32_t>(qzeros[static_cast<int64_t>(g) * (N / 8) + n / 8]),
                            n, zero_mode);
  const uint32_t q = static_cast<uint32_t>(qweight[static_cast<int64_t>(kw) * N + n]);
  out[static_cast<int64_t>(n) * KW + kw] = dequant8<ODT>(q, make_group_param(s, z));
}

// Generic path: any g_idx, wbits in {4, 8}, any float scale type. Follows
// quant_utils.py:62-69 literally: p = f32(s) * f32(w - z), then one rounding.
template <int ODT>
__global__ __launch_bounds__(256) void gptq_dequant_generic_kernel(
    const int32_t *__restrict__ qweight, const void *__restrict__ scales, int scale_dtype,
    const int32_t *__restrict__ qzeros, int zero_mode, const int32_t *__restrict__ g_idx,
    int groupsize, int wbits, int K, int N, void *__restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(K) * N) return;
  const int k = static_cast<int>(idx % K);
  const int n = static_cast<int>(idx / K);
  const int per_word = 32 / wbits;
  const uint32_t mask = (1u << wbits) - 1u;
  const uint32_t w = static_cast<uint32_t>(qweight[static_cast<int64_t>(k / per_word) * N + n]);
  const int code = static_cast<int>((w >> (wbits * (k % per_word))) & mask);
  const int g = g_idx ? g_idx[k] : k / groupsize;
  const uint32_t zw = static_cast<uint32_t>(
      qzeros[static_cast<int64_t>(g) * (N / per_word) + n / per_word]);
  int z = static_cast<int>((zw >> (wbits * (n % per_word))) & mask);
  if (zero_mode == OC_ZERO_V1) z = (z + 1) & static_cast<int>(mask);
  const float s = load_any_f32(scales, static_cast<int64_t>(g) * N + n, scale_dtype);
  // rounded to fp32 before the output conversion (fp32 scales: the product may round)
  const float p = opaque(s * static_cast<float>(code - z));
  store_out<ODT>(out, idx, p);
}

// ---------------------------------------------------------------------------
// RTN dequant to out[rows, K] (see oc_rtn_dequant). One thread per byte.
template <int ODT>
__global__ __launch_bounds__(256) void rtn_dequant_kernel(
    const uint8_t *__restrict__ q, int rows, int row_bytes, const void *__restrict__ scales,
    int scale_dtype, const void *__restrict__ zeros, int zero_dtype, int G, int K,
    void *__restrict__ out) {
  const int KB = (K + 1) / 2;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(KB) * rows) return;
  const int j = static_cast<int>(idx % KB);
  const int r = static_cast<int>(idx / KB);
  const int gs = K / G;
  const uint32_t byte = q[static_cast<int64_t>(r) * row_bytes + j];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int col = 2 * j + h;
    if (col >= K) break;
    const int g = col / gs;
    RtnParam p;
    p.zq = round_to<ODT>(load_any_f32(zeros, static_cast<int64_t>(r) * G + g, zero_dtype));
    p.sq = round_to<ODT>(load_any_f32(scales, static_cast<int64_t>(r) * G + g, scale_dtype));
    const float v = rtn_value<ODT>(static_cast<int>((byte >> (4 * h)) & 0xFu), p);
    store_out<ODT>(out, static_cast<int64_t>(r) * K + col, v);
  }
}

// ---------------------------------------------------------------------------
// Packed RTN embedding. Vector path: each thread turns 8 packed bytes (16
// codes of one group) into 16 outputs with two 16-byte stores.
__device__ __forceinline__ int64_t resolve_id(const int64_t *ids, int64_t t, int64_t V,
                                              int32_t *bad_flag) {
  int64_t id = ids[t];
  if (id < 0) id += V;  // torch indexing accepts negative ids
  if (id < 0 || id >= V) {
    if (bad_flag) *bad_flag = 1;
    return -1;
  }
  return id;
}

template <int ODT>
__global__ __launch_bounds__(256) void rtn_embedding_vec_kernel(
    const int64_t *__restrict__ ids, int64_t T, const uint8_t *__restrict__ q, int64_t V,
    int row_bytes, const void *__restrict__ scales, int scale_dtype, const void *__restrict__ zeros,
    int zero_dtype, int G, int D, uint4 *__restrict__ out, int32_t *bad_flag) {
  const int chunks = D / 16;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= T * chunks) return;
  const int ch = static_cast<int>(idx % chunks);
  const int64_t t = idx / chunks;
  uint4 lo = make_uint4(0, 0, 0, 0), hi = make_uint4(0, 0, 0, 0);
  const int64_t id = resolve_id(ids, t, V, bad_flag);
  if (id >= 0) {
    // Table bytes and output rows are touched once per call: non-temporal
    // (4096 tokens of D=1024 from V=32768: 5.3 -> 5.0 us with the stores so
    // marked).
    using u32x2 = __attribute__((ext_vector_type(2))) uint32_t;
    const u32x2 bv = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(q + id * row_bytes + 8 * ch));
    const uint2 bytes = make_uint2(bv[0], bv[1]);
    const int g = (16 * ch) / (D / G);
    RtnParam p;
    p.zq = round_to<ODT>(load_any_f32(zeros, id * G + g, zero_dtype));
    p.sq = round_to<ODT>(load_any_f32(scales, id * G + g, scale_dtype));
    lo = rtn_dequant8<ODT>(bytes.x, p);
    hi = rtn_dequant8<ODT>(bytes.y, p);
  }
  using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;
  __builtin_nontemporal_store(u32x4{lo.x, lo.y, lo.z, lo.w}, reinterpret_cast<u32x4 *>(out + 2 * idx));
  __builtin_nontemporal_store(u32x4{hi.x, hi.y, hi.z, hi.w}, reinterpret_cast<u32x4 *>(out + 2 * idx + 1));
}

template <int ODT>
__global__ __launch_bounds__(256) void rtn_embedding_scalar_kernel(
    const int64_t *__restrict__ ids, int64_t T, const uint8_t *__restrict__ q, int64_t V,
    int row_bytes, const void *__restrict__ scales, int scale_dtype, const void *__restrict__ zeros,
    int zero_dtype, int G, int D, void *__restrict__ out, int32_t *bad_flag) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= T * D) return;
  const int col = static_cast<int>(idx % D);
  const int64_t t = idx / D;
  const int64_t id = resolve_id(ids, t, V, bad_flag);
  float v = 0.f;
  if (id >= 0) {
    const int g = col / (D / G);
    RtnParam p;
    p.zq = round_to<ODT>(load_any_f32(zeros, id * G + g, zero_dtype));
    p.sq = round_to<ODT>(load_any_f32(scales, id * G + g, scale_dtype));
    const uint32_t byte = q[id * row_bytes + col / 2];
    v = rtn_value<ODT>(static_cast<int>((byte >> (4 * (col & 1))) & 0xFu), p);
  }
  store_out<ODT>(out, idx, v);
}

// DSV4 dequant (layers/dsv4_packed_linear.py:22-56): one thread per output
// element, out[n, k] = RNE_out(fp32(fp32(code - z) * s)).
template <int ODT>
__global__ __launch_bounds__(256) void dsv4_dequant_kernel(const uint8_t *__restrict__ q, int N, int row_bytes,
                                                           int wbits, int K, const void *scales, int sdt,
                                                           const void *zeros, int zdt, int groupsize,
                                                           int64_t stride_n, int64_t stride_g, void *out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(N) * K) return;
  const int k = static_cast<int>(idx % K);
  const int n = static_cast<int>(idx / K);
  const int per = 8 / wbits;
  const int code = (q[static_cast<int64_t>(n) * row_bytes + k / per] >> (wbits * (k % per))) & ((1 << wbits) - 1);
  const int64_t gi = static_cast<int64_t>(n) * stride_n + (groupsize > 0 ? static_cast<int64_t>(k / groupsize) * stride_g : 0);
  const float sv = load_any_f32(scales, gi, sdt);
  const float zv = load_any_f32(zeros, gi, zdt);
  // rounded to fp32 before the output conversion (see opaque())
  const float v = opaque(__fmul_rn(__fsub_rn(static_cast<float>(code), zv), sv));
  store_out<ODT>(out, idx, v);
}

inline unsigned grid_for(int64_t n, int block = 256) {
  return static_cast<unsigned>((n + block - 1) / block);
}

}  // namespace oc

using namespace oc;

extern "C" {

const char *oc_status_string(int status) {
  switch (status) {
    case OC_OK: return "OC_OK";
    case OC_ERR_INVALID_ARGUMENT: return "OC_ERR_INVALID_ARGUMENT";
    case OC_ERR_SHAPE: return "OC_ERR_SHAPE";
    case OC_ERR_UNSUPPORTED: return "OC_ERR_UNSUPPORTED";
    case OC_ERR_WORKSPACE: return "OC_ERR_WORKSPACE";
    case OC_ERR_HIP: return "OC_ERR_HIP";
    default: return "OC_ERR_UNKNOWN";
  }
}

const char *oc_last_error(void) { return g_last_error; }

int oc_version(void) { return 100; }

int oc_int4_plan_groups(const int64_t *g_idx, int32_t K, int32_t groupsize, int32_t *kmap_out,
                        int64_t kmap_capacity, int32_t *k_phys_out, int32_t *group_rows_out,
                        int32_t *num_groups_out, int32_t *identity_out) {
  clear_error();
  if (K <= 0) return fail(OC_ERR_SHAPE, "K must be positive, got %d", K);
  if (!k_phys_out || !group_rows_out || !num_groups_out || !identity_out)
    return fail(OC_ERR_INVALID_ARGUMENT, "output pointers must not be NULL");
  int64_t G = 0;
  std::vector<int64_t> group(K);
  if (g_idx) {
    for (int32_t k = 0; k < K; ++k) {
      if (g_idx[k] < 0 || g_idx[k] >= K)
        return fail(OC_ERR_INVALID_ARGUMENT, "g_idx[%d] = %lld outside [0, K)", k,
                    static_cast<long long>(g_idx[k]));
      group[k] = g_idx[k];
      G = std::max<int64_t>(G, g_idx[k] + 1);
    }
  } else {
    if (groupsize <= 0) return fail(OC_ERR_INVALID_ARGUMENT, "groupsize must be positive");
    for (int32_t k = 0; k < K; ++k) group[k] = k / groupsize;
    G = (K + groupsize - 1) / groupsize;
  }
  std::vector<int32_t> count(G, 0);
  for (int32_t k = 0; k < K; ++k) ++count[group[k]];
  int32_t max_count = 0;
  for (int32_t c : count) max_count = std::max(max_count, c);
  const int64_t rows = (static_cast<int64_t>(max_count) + 31) / 32 * 32;
  const int64_t k_phys = G * rows;
  if (k_phys > 8 * static_cast<int64_t>(K) + 256 || k_phys > (1LL << 30))
    return fail(OC_ERR_UNSUPPORTED,
                "groups are too uneven: %lld groups of up to %d members need %lld physical rows "
                "for K=%d",
                static_cast<long long>(G), max_count, static_cast<long long>(k_phys), K);
  *k_phys_out = static_cast<int32_t>(k_phys);
  *group_rows_out = static_cast<int32_t>(rows);
  *num_groups_out = static_cast<int32_t>(G);
  std::vector<int32_t> kmap(k_phys, -1);
  std::vector<int32_t> cursor(G, 0);
  for (int32_t k = 0; k < K; ++k) {
    const int64_t g = group[k];
    kmap[g * rows + cursor[g]++] = k;
  }
  int32_t identity = k_phys == K ? 1 : 0;
  for (int64_t i = 0; identity && i < k_phys; ++i) identity = kmap[i] == i;
  *identity_out = identity;
  if (kmap_out) {
    if (kmap_capacity < k_phys)
      return fail(OC_ERR_SHAPE, "kmap capacity %lld < K_phys %lld",
                  static_cast<long long>(kmap_capacity), static_cast<long long>(k_phys));
    std::memcpy(kmap_out, kmap.data(), sizeof(int32_t) * k_phys);
  }
  return OC_OK;
}

int oc_unpack_rows(const int32_t *packed, int32_t packed_rows, int32_t cols, int32_t wbits,
                   int32_t num_rows, int32_t *out, void *stream) {
  clear_error();
  if (wbits != 2 && wbits != 4 && wbits != 8)
    return fail(OC_ERR_UNSUPPORTED, "wbits must divide 32 and be 2, 4 or 8, got %d", wbits);
  if (packed_rows < 0 || cols < 0 || num_rows < 0 ||
      static_cast<int64_t>(num_rows) > static_cast<int64_t>(packed_rows) * (32 / wbits))
    return fail(OC_ERR_SHAPE, "num_rows=%d exceeds %d packed rows x %d", num_rows, packed_rows, 32 / wbits);
  const int64_t total = static_cast<int64_t>(num_rows) * cols;
  if (total == 0) return OC_OK;
  if (!packed || !out) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  hipLaunchKernelGGL(unpack_rows_kernel, dim3(grid_for(total)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), packed, cols, wbits, num_rows, out);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_int4_dequant(const int32_t *qweight, const void *scales, int32_t scale_dtype,
                    const int32_t *qzeros, int32_t zero_mode, const int32_t *g_idx,
                    int32_t groupsize, int32_t wbits, int32_t K, int32_t N, void *out,
                    int32_t out_dtype, void *stream) {
  clear_error();
  if (!qweight || !scales || !qzeros || !out) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (wbits != 4 && wbits != 8) return fail(OC_ERR_UNSUPPORTED, "wbits must be 4 or 8, got %d", wbits);
  if (!is_float_dtype(scale_dtype) || !is_float_dtype(out_dtype))
    return fail(OC_ERR_INVALID_ARGUMENT, "scale/out dtype must be F16, BF16 or F32");
  if (zero_mode != OC_ZERO_V1 && zero_mode != OC_ZERO_V2)
    return fail(OC_ERR_INVALID_ARGUMENT, "zero_mode must be OC_ZERO_V1 or OC_ZERO_V2");
  const int per_word = 32 / wbits;
  if (K <= 0 || N <= 0 || N % per_word != 0)
    return fail(OC_ERR_SHAPE, "bad shape K=%d N=%d (N %% %d == 0 required)", K, N, per_word);
  if (!g_idx && groupsize <= 0) return fail(OC_ERR_INVALID_ARGUMENT, "groupsize must be positive");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool fast = wbits == 4 && !g_idx && groupsize % 8 == 0 && K % 8 == 0 &&
                    is_half_dtype(scale_dtype) && is_half_dtype(out_dtype) && aligned(out, 16);
  if (fast) {
    const int64_t total = static_cast<int64_t>(K / 8) * N;
    auto kern = out_dtype == OC_DTYPE_BF16 ? gptq_dequant4_kernel<OC_DTYPE_BF16>
                                           : gptq_dequant4_kernel<OC_DTYPE_F16>;
    hipLaunchKernelGGL(kern, dim3(grid_for(total)), dim3(256), 0, s, qweight,
                       static_cast<const uint16_t *>(scales), scale_dtype, qzeros, zero_mode,
                       groupsize, K, N, static_cast<uint4 *>(out));
  } else {
    const int64_t total = static_cast<int64_t>(K) * N;
    auto kern = out_dtype == OC_DTYPE_BF16   ? gptq_dequant_generic_kernel<OC_DTYPE_BF16>
                : out_dtype == OC_DTYPE_F16 ? gptq_dequant_generic_kernel<OC_DTYPE_F16>
                                            : gptq_dequant_generic_kernel<OC_DTYPE_F32>;
    hipLaunchKernelGGL(kern, dim3(grid_for(total)), dim3(256), 0, s, qweight, scales, scale_dtype,
                       qzeros, zero_mode, g_idx, groupsize, wbits, K, N, out);
  }
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_rtn_dequant(const uint8_t *qweight_u8, int32_t rows, int32_t row_bytes, const void *scales,
                   int32_t scale_dtype, const void *zeros, int32_t zero_dtype, int32_t G, int32_t K,
                   void *out, int32_t out_dtype, void *stream) {
  clear_error();
  if (!qweight_u8 || !scales || !zeros || !out) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_float_dtype(scale_dtype) || !is_float_dtype(out_dtype) || dtype_bytes(zero_dtype) == 0)
    return fail(OC_ERR_INVALID_ARGUMENT, "unsupported dtype");
  if (rows <= 0 || K <= 0 || G <= 0 || row_bytes < (K + 1) / 2)
    return fail(OC_ERR_SHAPE, "bad shape rows=%d K=%d G=%d row_bytes=%d", rows, K, G, row_bytes);
  if (K % G != 0)
    return fail(OC_ERR_SHAPE, "in_features=%d not divisible by num_groups=%d", K, G);
  const int64_t total = static_cast<int64_t>((K + 1) / 2) * rows;
  auto kern = out_dtype == OC_DTYPE_BF16   ? rtn_dequant_kernel<OC_DTYPE_BF16>
              : out_dtype == OC_DTYPE_F16 ? rtn_dequant_kernel<OC_DTYPE_F16>
                                          : rtn_dequant_kernel<OC_DTYPE_F32>;
  hipLaunchKernelGGL(kern, dim3(grid_for(total)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     qweight_u8, rows, row_bytes, scales, scale_dtype, zeros, zero_dtype, G, K, out);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_dsv4_dequant(const uint8_t *qweight, int32_t N, int32_t row_bytes, int32_t wbits, int32_t K,
                    const void *scales, int32_t scale_dtype, const void *zeros, int32_t zero_dtype,
                    int32_t groupsize, int64_t sz_stride_n, int64_t sz_stride_g, void *out, int32_t out_dtype,
                    void *stream) {
  clear_error();
  if (!qweight || !scales || !zeros || !out) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (wbits != 2 && wbits != 4 && wbits != 8) return fail(OC_ERR_INVALID_ARGUMENT, "wbits must be 2, 4 or 8");
  if (!is_float_dtype(scale_dtype) || !is_float_dtype(zero_dtype) || !is_float_dtype(out_dtype))
    return fail(OC_ERR_INVALID_ARGUMENT, "unsupported dtype");
  const int per = 8 / wbits;
  if (N <= 0 || K <= 0 || row_bytes < (K + per - 1) / per)
    return fail(OC_ERR_SHAPE, "bad shape N=%d K=%d row_bytes=%d", N, K, row_bytes);
  const int64_t total = static_cast<int64_t>(N) * K;
  auto kern = out_dtype == OC_DTYPE_BF16   ? dsv4_dequant_kernel<OC_DTYPE_BF16>
              : out_dtype == OC_DTYPE_F16 ? dsv4_dequant_kernel<OC_DTYPE_F16>
                                          : dsv4_dequant_kernel<OC_DTYPE_F32>;
  hipLaunchKernelGGL(kern, dim3(grid_for(total)), dim3(256), 0, static_cast<hipStream_t>(stream), qweight, N,
                     row_bytes, wbits, K, scales, scale_dtype, zeros, zero_dtype, groupsize, sz_stride_n,
                     sz_stride_g, out);
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

int oc_rtn_embedding(const int64_t *ids, int64_t T, const uint8_t *qweight_u8, int64_t V,
                     int32_t row_bytes, const void *scales, int32_t scale_dtype, const void *zeros,
                     int32_t zero_dtype, int32_t G, int32_t D, void *out, int32_t out_dtype,
                     int32_t *bad_id_flag, void *stream) {
  clear_error();
  if (T == 0) return OC_OK;
  if (!ids || !qweight_u8 || !scales || !zeros || !out)
    return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!is_float_dtype(scale_dtype) || !is_float_dtype(out_dtype) || dtype_bytes(zero_dtype) == 0)
    return fail(OC_ERR_INVALID_ARGUMENT, "unsupported dtype");
  if (T < 0 || V <= 0 || D <= 0 || G <= 0 || row_bytes < (D + 1) / 2)
    return fail(OC_ERR_SHAPE, "bad shape T=%lld V=%lld D=%d G=%d row_bytes=%d",
                static_cast<long long>(T), static_cast<long long>(V), D, G, row_bytes);
  if (D % G != 0) return fail(OC_ERR_SHAPE, "in_features=%d not divisible by num_groups=%d", D, G);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int gs = D / G;
  const bool vec = is_half_dtype(out_dtype) && D % 16 == 0 && gs % 16 == 0 && row_bytes % 8 == 0 &&
                   aligned(qweight_u8, 8) && aligned(out, 16);
  if (vec) {
    const int64_t total = T * (D / 16);
    auto kern = out_dtype == OC_DTYPE_BF16 ? rtn_embedding_vec_kernel<OC_DTYPE_BF16>
                                           : rtn_embedding_vec_kernel<OC_DTYPE_F16>;
    hipLaunchKernelGGL(kern, dim3(grid_for(total)), dim3(256), 0, s, ids, T, qweight_u8, V,
                       row_bytes, scales, scale_dtype, zeros, zero_dtype, G, D,
                       static_cast<uint4 *>(out), bad_id_flag);
  } else {
    const int64_t total = T * D;
    auto kern = out_dtype == OC_DTYPE_BF16   ? rtn_embedding_scalar_kernel<OC_DTYPE_BF16>
                : out_dtype == OC_DTYPE_F16 ? rtn_embedding_scalar_kernel<OC_DTYPE_F16>
                                            : rtn_embedding_scalar_kernel<OC_DTYPE_F32>;
    hipLaunchKernelGGL(kern, dim3(grid_for(total)), dim3(256), 0, s, ids, T, qweight_u8, V,
                       row_bytes, scales, scale_dtype, zeros, zero_dtype, G, D, out, bad_id_flag);
  }
  OC_RETURN_LAUNCH_STATUS();
  return OC_OK;
}

}  // extern "C"
