// Kernel parameters and device helpers shared by the GEMM translation units
// (oc_gemm.hip, oc_gemm_wide.hip): the launch-parameter block, epilogue
// helpers, the buffer-resource DMA path into LDS and its wait/barrier
// primitives.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "oc_device.h"
#include "oc_internal.h"

namespace oc {

// Weight formats of the tiled GEMM: 4-bit GPTQ tile16, RTN uint8 nibbles
// [N, K/2], 8-bit GPTQ tile16 (32 code bytes per column and K step).
// DSV4: uint8 [N, K / per] codes along the in-dim (int4: the RTN nibble
// order; int2: 4 codes per byte, low bits first), fp32 dequant (q - z) * s.
// RTN_T: RTN nibbles of a transposed weight (rows = output columns n, K
// along each row) whose scales and zeros vary along K: one per (K row, group
// of n), stored [groups][K] (the packed ConvTranspose1d weight).
enum { FMT_GPTQ = 0, FMT_RTN = 1, FMT_GPTQ8 = 2, FMT_DSV4_4 = 3, FMT_DSV4_2 = 4, FMT_RTN_T = 5 };
constexpr bool fmt_rows(int f) { return f == FMT_RTN || f == FMT_DSV4_4 || f == FMT_DSV4_2 || f == FMT_RTN_T; }

struct GemmParams {
  const void *a;
  int64_t lda;
  int64_t a_bytes;  // bytes of the activation block the large-M kernel may read
  int M;
  int K_logical;
  const void *qw;      // GPTQ: tile16 words; RTN: uint8 [N, row_bytes]
  const void *scales;  // GPTQ: tile16 16-bit scales; RTN: [N, G] of scale_dtype
  const void *zeros;   // GPTQ: tile16 zero words; RTN: [N, G] of zero_dtype
  int scale_dtype;     // RTN (runtime)
  int zero_dtype;      // RTN (runtime)
  int rtn_gs;          // RTN / DSV4: columns per group
  uint32_t rtn_gs_magic;  // ceil(2^32 / rtn_gs) when floor(x / rtn_gs) = umulhi(x, magic) for every
                          // K offset x of the layer, else 0 (set by the tiled launch)
  int rtn_G;           // RTN: groups per row
  int row_bytes;       // RTN / DSV4
  int64_t sz_stride_n;  // RTN / DSV4: scale/zero element offset per output row ...
  int64_t sz_stride_g;  // ... and per group
  int N;
  int K_phys;
  int KS;              // K_phys / 32
  int G;               // K_phys / group_rows
  int group_rows;
  int gshift;          // log2(group_rows / 32), or -1
  const uint16_t *kinv;  // decode regime: logical -> physical row (NULL: identity)
  const void *bias;
  int bias_dtype;
  void *c;
  int64_t ldc;
  float *partials;  // fp32 partial sums [ksplit, M, N] (split-K)
  int out_f32;      // 1: the tiled kernel writes fp32 partials even without a K split
  int ksplit;
  int ksteps_per_split;
  // grouped (MoE) launch
  const int32_t *expert_offsets;
  const int32_t *sorted_pairs;
  int topk;
  int64_t qw_expert_stride;  // 32-bit words per expert
  int64_t s_expert_stride;   // 16-bit scales per expert
  int64_t z_expert_stride;   // zero words per expert
  // decode (split GEMV)
  const int32_t *kmap;  // physical -> logical row (-1: padding), NULL: identity
  int *counters;        // per tile group arrival counters (zero between calls)
  int stream_slots;     // stream GEMV: most tiles one workgroup's range touches
};

__device__ __forceinline__ int group_of(const GemmParams &p, int ks) {
  return p.gshift >= 0 ? (ks >> p.gshift) : (32 * ks) / p.group_rows;
}

template <int SDT>
__device__ __forceinline__ float scale_f32(uint32_t bits) {
  return SDT == OC_DTYPE_BF16 ? bf16_to_f32(static_cast<uint16_t>(bits)) : f16_to_f32(static_cast<uint16_t>(bits));
}

template <int DT>
__device__ __forceinline__ void store_c(void *c, int64_t i, float v) {
  static_cast<uint16_t *>(c)[i] = static_cast<uint16_t>(pack2<DT>(v, 0.f));
}

__device__ __forceinline__ float bias_at(const GemmParams &p, int n) {
  return p.bias ? load_any_f32(p.bias, n, p.bias_dtype) : 0.f;
}

// Workgroup order -> tile, keeping neighbouring tiles on one XCD (workgroups
// are handed to the 8 XCDs round-robin); identity unless 8 divides the count.
__device__ __forceinline__ int xcd_block(int bid, int nblocks) {
  if (nblocks % 8 != 0) return bid;
  return (bid & 7) * (nblocks >> 3) + (bid >> 3);
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Buffer DMA: lane l's bytes at (resource base + voffset + soffset) land at
// lds + size * l (lds and soffset wave-uniform). Addresses are 32-bit offsets
// from a per-tensor resource, so the loop advances them with scalar adds;
// reads outside the resource's range return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, int64_t bytes) {
  const int n = static_cast<int>(bytes < 0x7fffffff ? bytes : 0x7fffffff);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, n, 0x00020000);
}
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void *lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)(lds), 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void *lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)(lds), 4, voff, soff, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x0F70);
}

// Workgroup barrier without the release fence of __syncthreads (which would
// wait for every DMA in flight). This wave's LDS reads are complete first, so
// no other wave's DMA issued after the barrier can overwrite data they read.
__device__ __forceinline__ void barrier_no_fence() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int I>
using ic = std::integral_constant<int, I>;

// f(ic<k>) for k = K0 .. E - 1, unrolled at compile time (stage arrays stay
// in registers even where the unroller would give up on a large body).
template <int K0, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (K0 < E) {
    f(ic<K0>{});
    static_for<K0 + 1, E>(f);
  }
}

// 16-byte chunk swizzle of the LDS activation rows (64 bytes each): chunk q
// of row r sits at position q ^ big_swz(r). An MFMA operand read (rows
// r0..r0+15, one chunk) then touches distinct banks within every group of 8
// or 16 lanes the LDS serves together (32 or 64 banks of 4 bytes).
__device__ __forceinline__ int big_swz(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

// ---- decode inner-product helpers (x-pair staging) ----

template <int DT>
__device__ __forceinline__ float dot2acc(uint32_t b, uint32_t x, float acc) {
  if constexpr (DT == OC_DTYPE_BF16) {
    return __builtin_amdgcn_fdot2_f32_bf16(bitcast<v2bf16>(b), bitcast<v2bf16>(x), acc, false);
  } else {
    return __builtin_amdgcn_fdot2(bitcast<v2f16>(b), bitcast<v2f16>(x), acc, false);
  }
}

// Cache policy of the weight, scale and zero loads of the stream and
// whole-tile MFMA GEMV kernels (the aux operand of the buffer loads): nt,
// non-temporal. Each of those bytes is read once per call. Measured on a
// decode sweep of four layers: 5 % faster per step; a single layer replayed
// back to back is ~4 % slower with it.
constexpr int CPOL_WEIGHT_STREAM = 2;

template <int DT>
__device__ __forceinline__ float half_to_f32(uint32_t h16) {
  if constexpr (DT == OC_DTYPE_BF16) return bf16_to_f32(static_cast<uint16_t>(h16));
  else return f16_to_f32(static_cast<uint16_t>(h16));
}

template <int DT>
constexpr float dot_base() {
  return DT == OC_DTYPE_BF16 ? 128.f : 1024.f;
}

// Physical row r of activation row m -> its 16-bit slot in an x-pair block
// (rows of K_phys values; octet pairs (i, i + 4) adjacent).
__device__ __forceinline__ int xpair_slot(int m, int K_phys, int r) {
  return m * K_phys + (r & ~7) + ((r & 3) << 1) + ((r >> 2) & 1);
}

// Pair words of one octet given as 4 raw words {x0|x1<<16, x2|x3<<16, ...},
// and the octet's sum (fp32, in row order).
template <int DT>
__device__ __forceinline__ uint4 octet_pairs(uint4 raw, float &sum) {
  const uint32_t lo = 0x05040100u, hi = 0x07060302u;  // v_perm selectors: low / high halves of two words
  uint4 r;
  r.x = __builtin_amdgcn_perm(raw.z, raw.x, lo);  // x0 | x4 << 16
  r.y = __builtin_amdgcn_perm(raw.z, raw.x, hi);  // x1 | x5 << 16
  r.z = __builtin_amdgcn_perm(raw.w, raw.y, lo);  // x2 | x6 << 16
  r.w = __builtin_amdgcn_perm(raw.w, raw.y, hi);  // x3 | x7 << 16
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += half_to_f32<DT>(w[i] & 0xFFFFu);
    s += half_to_f32<DT>(w[i] >> 16);
  }
  sum = s;
  return r;
}


// Host helpers.
int env_int(const char *name, int dflt);
int device_cus();          // compute units of the current device
int ilog2_exact(int v);    // log2(v) for a power of two, else -1

// LDS-tiled kernel over RTN nibble rows (oc_gemm.hip): tile shape and K split
// for an M x N x K problem, and a launch of FMT_RTN (transposed = false) or
// FMT_RTN_T. With p.out_f32 (or a K split) the kernel writes fp32 partials
// [ksplit][M][N] to p.partials and nothing else.
void plan_tiled(int M, int N, int K, int *wm, int *wn, int *kg, int *ksplit, int *ksteps_per_split);
void launch_rtn_tiled(const GemmParams &p, int x_dtype, bool transposed, int wm, int wn, int kg, hipStream_t s);

// Row-format GEMV for M <= 4 (oc_rows_gemv.hip): RTN nibble rows (fmt
// FMT_RTN) and DSV4 int4 / int2 rows (FMT_DSV4_4 / FMT_DSV4_2), one wave per
// output row, no workspace. rows_gemv_applies: M <= 4; K and the group size
// multiples of one lane's 16 bytes of codes (32 columns at 4 bits, 64 at 2);
// 16-byte aligned rows; 16-bit scales and zeros of one dtype; the activation
// rows within 64 KB of LDS.
bool rows_gemv_applies(int M, int K, int groupsize, int bits, int scale_dtype, int zero_dtype, int64_t row_bytes,
                       const void *qweight);
void launch_rows_gemv(const GemmParams &p, int x_dtype, int fmt, hipStream_t s);

// Large-M kernel with 256-row wave tiles (oc_gemm_wide.hip): one launch over
// ceil(M / 256) x ceil(N / (64 wn)) workgroups, wn = 3 or 4 tiles per wave.
void launch_gptq_wide(const GemmParams &p, int a_dtype, int scale_dtype, int wn, hipStream_t s);
// RTN tiles (oc_rtn_tile_prepare) on the large-M kernel into fp32 partials
// [p.ksplit][M][N] (p.out_f32 = 1, p.partials); group steps a power of two
// (p.gshift >= 0), N % 8 == 0, every group fast-dequant eligible; column
// blocks of 64 wn (wn = 2 or 3).
void launch_rtn_wide(const GemmParams &p, int a_dtype, int scale_dtype, int wn, hipStream_t s);
// Transposed-group RTN tiles (oc_rtn_tile_prepare_t, row words in a_dtype)
// on the large-M kernel into fp32 partials, as launch_rtn_wide.
void launch_rtnt_wide(const GemmParams &p, int a_dtype, int wn, hipStream_t s);

// Decode GEMV over work items of T tiles x S K steps (oc_gemv.hip). K is split
// into ksplit = ceil(KS / S) ranges; with ksplit > 1 the launch needs
// p.partials (ksplit * M * N floats) and p.counters (one zeroed int per
// group of T tiles, left zero).
struct GemvPlan {
  int T;       // tiles per item
  int S;       // K steps per item
  int ksplit;  // K ranges
};
GemvPlan plan_gemv(int M, int N, int KS, bool gather, int cus);
size_t gemv_lds_bytes(int MR, int S);
void launch_gptq_gemv(const GemmParams &p, int a_dtype, int scale_dtype, int T, hipStream_t s);

// Small-batch GEMV with one balanced weight range per workgroup
// (oc_gemv_stream.hip; dot2 for M <= 2, MFMA for M <= 16). gemv_stream_wgs
// gives the launch width for a layer (0: not applicable: M > 16, activation
// rows beyond LDS, fewer tiles than workgroups, or more swap cells than
// cell_bytes hold). The launch needs p.counters: nwg * MR * 16 zeroed 64-bit
// cells (MR = M rounded up to 1, 2, 4, 8 or 16), left zero.
int gemv_stream_wgs(int M, int N, int KS, int cus, size_t cell_bytes);
// The same ranges for 3..16 rows read from global memory in physical row order
// (no staging; for rows beyond LDS when whole tiles would load CUs unevenly).
int gemv_stream_global_wgs(int M, int N, int KS, int cus, size_t cell_bytes);
// 8-bit tile16x8 layers at M <= 16: launch width of the global form (0: not
// applicable) and its launch (activation rows in physical order).
int gemv_stream_global8_wgs(int M, int N, int KS, int cus, size_t cell_bytes);
void launch_gptq8_gemv_stream(const GemmParams &p, int a_dtype, int scale_dtype, int nwg, hipStream_t s);
void launch_gptq_gemv_stream(const GemmParams &p, int a_dtype, int scale_dtype, int nwg, bool global_rows,
                             hipStream_t s);

}  // namespace oc
