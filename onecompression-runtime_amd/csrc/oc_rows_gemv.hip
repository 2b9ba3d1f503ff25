// Small-batch GEMV (M <= 4) over row-major packed weights: RTN nibble rows
// (quant_utils.py:72-103, PackedRTNLinear) and DSV4 int4 / int2 rows
// (layers/dsv4_packed_linear.py:22-56), for gfx950.
//
// The weight of output n is one contiguous byte row (codes along K, code i
// of a word at bits BITS * i), so one wave owns one output row and each wave
// instruction reads 1 KB of it (16 bytes per lane). A row's loads (up to 4
// per lane, then batch by batch) and their group parameters are issued
// before the activation rows are staged into LDS, so the weight stream's
// latency covers the staging. Each octet is dequantized
// exactly as the tiled kernels do it (RTN: per-op rounding; DSV4: fp32
// subtract and multiply, one rounding), and multiplied with the matching 8
// activations in fp32 pairs (v_dot2_f32_{bf16,f16}); the lanes' sums are
// added with a fixed butterfly, so results are deterministic.
#include <hip/hip_runtime.h>

#include "oc_gemm_common.h"

namespace oc {
namespace {

// Output rows per workgroup: each workgroup stages the activation rows once,
// so more rows per workgroup stage less in total (measured on DSV4 K=7168
// N=2048 M=1: 2 / 4 / 8 rows 11.5 / 8.6 / 7.4 us).
constexpr int RG_WAVES = 8;
constexpr int RG_BATCH = 4;  // 16-byte weight loads per lane in flight (4 beat 8: 8.6 vs 9.0 us)

// V octets per lane per load (16 bytes: V = 4 at 4 bits, 8 at 2 bits), so a
// wave instruction reads 1 KB of the row. Lane l of load i holds octets
// 64 V i + V l + j (j < V), all in one group (host: the group size is a
// multiple of 8 V): one scale and zero load per lane and load. Activation
// octet o of row m sits in LDS at m * NOP + 64 V (o / 64 V) + 64 j + l, so
// the lanes' reads of octet j are consecutive 16-byte chunks.
template <int DT, int FMT, int MR, int SDT>
__global__ __launch_bounds__(64 * RG_WAVES) void rows_gemv_kernel(GemmParams p) {
  constexpr int BITS = FMT == FMT_DSV4_2 ? 2 : 4;
  constexpr int V = 16 / BITS;       // octets per lane per load
  constexpr int OB = 64 * V;         // octets per wave load
  static_assert(FMT == FMT_RTN || FMT == FMT_DSV4_4 || FMT == FMT_DSV4_2, "row formats");
  extern __shared__ __attribute__((aligned(16))) uint4 xs[];  // [MR][NOP] activation octets, permuted
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroups of neighbouring rows on one XCD: they share the lines of the
  // [groups][N] scales and zeros.
  const int n = xcd_block(blockIdx.x, gridDim.x) * RG_WAVES + wave;
  const int nr = min(n, p.N - 1);  // rows past N load a valid row; nothing is stored for them
  const int K = p.K_logical, NO = K >> 3;
  const int NL = (NO + OB - 1) / OB;  // wave loads per row
  const int NOP = NL * OB;            // octets per LDS row (padded to whole loads)
  const uint8_t *qrow = static_cast<const uint8_t *>(p.qw) + static_cast<int64_t>(nr) * p.row_bytes;
  const int row_bytes_used = NO * BITS;  // bytes of the row's codes
  const uint16_t *sc = static_cast<const uint16_t *>(p.scales);
  const uint16_t *zr = static_cast<const uint16_t *>(p.zeros);
  const int64_t sz_row = static_cast<int64_t>(nr) * p.sz_stride_n;

  uint4 q[RG_BATCH];
  uint32_t sv[RG_BATCH], zv[RG_BATCH];
  auto load_batch = [&](int b0) {
#pragma unroll
    for (int i = 0; i < RG_BATCH; ++i) {
      // Loads past the row re-read its last 16 bytes (their octets are masked).
      const int byte = min((OB * (b0 + i) + V * lane) * BITS, row_bytes_used - 16);
      q[i] = *reinterpret_cast<const uint4 *>(qrow + byte);
      const uint32_t x = static_cast<uint32_t>(8 * (byte / BITS));  // first K row of the lane's octets
      const uint32_t g = p.rtn_gs_magic ? __umulhi(x, p.rtn_gs_magic) : x / static_cast<uint32_t>(p.rtn_gs);
      const int64_t e = sz_row + static_cast<int64_t>(g) * p.sz_stride_g;
      sv[i] = sc[e];
      zv[i] = zr[e];
    }
  };
  load_batch(0);

  // Activation rows into LDS, permuted: every load first, then the stores
  // (rows past M and octets past K are zeros).
  constexpr int XB = 4096 / (64 * RG_WAVES);  // chunks per thread (host: MR * NOP * 16 <= 64 KB)
  const int nx = MR * NOP;
  const uint16_t *a = static_cast<const uint16_t *>(p.a);
  uint4 xr[XB];
#pragma unroll
  for (int jj = 0; jj < XB; ++jj) {
    const int i = tid + 64 * RG_WAVES * jj;
    const int m = i / NOP, o = i - m * NOP;
    xr[jj] = i < nx && m < p.M && o < NO
                 ? *reinterpret_cast<const uint4 *>(a + static_cast<int64_t>(m) * p.lda + 8 * o)
                 : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int jj = 0; jj < XB; ++jj) {
    const int i = tid + 64 * RG_WAVES * jj;
    if (i < nx) {
      const int m = i / NOP, o = i - m * NOP;
      const int r = o % OB;
      xs[m * NOP + (o - r) + 64 * (r % V) + r / V] = xr[jj];
    }
  }
  __syncthreads();

  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.f;
  auto consume = [&](int b0) {
#pragma unroll
    for (int i = 0; i < RG_BATCH; ++i) {
      const int ld = b0 + i;
      if (ld >= NL) break;  // wave-uniform
      const float s = half_to_f32<SDT>(sv[i]), z = half_to_f32<SDT>(zv[i]);
      const uint32_t words[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int o = OB * ld + V * lane + j;
        if (o >= NO) break;
        const uint32_t code8 = BITS == 4 ? words[j] : (words[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
        uint4 w;
        if constexpr (FMT == FMT_RTN) {
          RtnParam rp;
          rp.sq = round_to<DT>(s);
          rp.zq = round_to<DT>(z);
          w = rtn_dequant8<DT>(code8, rp);
        } else {
          w = dsv4_dequant8<DT, BITS>(code8, s, z);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const uint4 xv = xs[m * NOP + OB * ld + 64 * j + lane];
          float d = acc[m];
          d = dot2acc<DT>(w.x, xv.x, d);
          d = dot2acc<DT>(w.y, xv.y, d);
          d = dot2acc<DT>(w.z, xv.z, d);
          d = dot2acc<DT>(w.w, xv.w, d);
          acc[m] = d;
        }
      }
    }
  };
  consume(0);
  for (int b0 = RG_BATCH; b0 < NL; b0 += RG_BATCH) {
    load_batch(b0);
    consume(b0);
  }
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float v = acc[m];
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
    acc[m] = v;
  }
  if (lane != 0 || n >= p.N) return;
  const float bv = bias_at(p, n);
#pragma unroll
  for (int m = 0; m < MR; ++m)
    if (m < p.M) store_c<DT>(p.c, static_cast<int64_t>(m) * p.ldc + n, acc[m] + bv);
}

// LDS bytes of the activation rows (rows padded to whole wave loads).
size_t rows_lds_bytes(int MR, int K, int bits) {
  const int OB = 64 * (16 / bits), NO = K / 8;
  return static_cast<size_t>(MR) * ((NO + OB - 1) / OB) * OB * 16;
}

template <int DT, int FMT, int SDT>
void launch_rows_m(const GemmParams &p, hipStream_t s) {
  constexpr int BITS = FMT == FMT_DSV4_2 ? 2 : 4;
  const dim3 grid((p.N + RG_WAVES - 1) / RG_WAVES), block(64 * RG_WAVES);
  if (p.M == 1)
    hipLaunchKernelGGL((rows_gemv_kernel<DT, FMT, 1, SDT>), grid, block, rows_lds_bytes(1, p.K_logical, BITS), s, p);
  else if (p.M == 2)
    hipLaunchKernelGGL((rows_gemv_kernel<DT, FMT, 2, SDT>), grid, block, rows_lds_bytes(2, p.K_logical, BITS), s, p);
  else
    hipLaunchKernelGGL((rows_gemv_kernel<DT, FMT, 4, SDT>), grid, block, rows_lds_bytes(4, p.K_logical, BITS), s, p);
}

template <int DT, int FMT>
void launch_rows_s(const GemmParams &p, hipStream_t s) {
  if (p.scale_dtype == OC_DTYPE_BF16) launch_rows_m<DT, FMT, OC_DTYPE_BF16>(p, s);
  else launch_rows_m<DT, FMT, OC_DTYPE_F16>(p, s);
}

template <int FMT>
void launch_rows_x(const GemmParams &p, int x_dtype, hipStream_t s) {
  if (x_dtype == OC_DTYPE_BF16) launch_rows_s<OC_DTYPE_BF16, FMT>(p, s);
  else launch_rows_s<OC_DTYPE_F16, FMT>(p, s);
}

}  // namespace

bool rows_gemv_applies(int M, int K, int groupsize, int bits, int scale_dtype, int zero_dtype, int64_t row_bytes,
                       const void *qweight) {
  // ONECOMP_HIP_ROWS_GEMV=0 (read per call; tests) keeps these shapes on the tiled kernel.
  if (env_int("ONECOMP_HIP_ROWS_GEMV", 1) == 0) return false;
  const int MR = M <= 1 ? 1 : M <= 2 ? 2 : 4;
  const int lane_k = 8 * (16 / bits);  // K rows of one lane's 16-byte load
  // Whole 16-byte loads: rows of K / lane_k loads at 16-byte aligned addresses.
  return M >= 1 && M <= 4 && K % lane_k == 0 && groupsize > 0 && groupsize % lane_k == 0 &&
         row_bytes % 16 == 0 && reinterpret_cast<uintptr_t>(qweight) % 16 == 0 &&
         rows_lds_bytes(MR, K, bits) <= 64 * 1024 && scale_dtype == zero_dtype &&
         (scale_dtype == OC_DTYPE_F16 || scale_dtype == OC_DTYPE_BF16);
}

void launch_rows_gemv(const GemmParams &p_in, int x_dtype, int fmt, hipStream_t s) {
  GemmParams p = p_in;
  // floor(x / gs) = umulhi(x, ceil(2^32 / gs)) for every x < K when K gs < 2^32.
  const uint64_t gs = static_cast<uint64_t>(p.rtn_gs);
  p.rtn_gs_magic = gs >= 2 && static_cast<uint64_t>(p.K_logical) * gs < (uint64_t{1} << 32)
                       ? static_cast<uint32_t>(((uint64_t{1} << 32) + gs - 1) / gs)
                       : 0;
  if (fmt == FMT_RTN) launch_rows_x<FMT_RTN>(p, x_dtype, s);
  else if (fmt == FMT_DSV4_4) launch_rows_x<FMT_DSV4_4>(p, x_dtype, s);
  else launch_rows_x<FMT_DSV4_2>(p, x_dtype, s);
}

}  // namespace oc
