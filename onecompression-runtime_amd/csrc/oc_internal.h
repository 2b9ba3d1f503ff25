// Host-side helpers shared by the library's translation units: the public
// ABI, status reporting and launch-argument checks.
#pragma once

#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>

#include "onecomp_hip.h"

namespace oc {

// Records a formatted error message for oc_last_error() and returns `status`.
int fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the thread's last error.
void clear_error();

inline bool is_half_dtype(int dt) { return dt == OC_DTYPE_F16 || dt == OC_DTYPE_BF16; }
inline bool is_float_dtype(int dt) { return is_half_dtype(dt) || dt == OC_DTYPE_F32; }
inline size_t dtype_bytes(int dt) {
  switch (dt) {
    case OC_DTYPE_F16:
    case OC_DTYPE_BF16: return 2;
    case OC_DTYPE_F32:
    case OC_DTYPE_I32: return 4;
    case OC_DTYPE_U8: return 1;
    default: return 0;
  }
}
// Activations into physical row order (oc_layout.hip): through kinv when
// given (coalesced), else through kmap.
void launch_gather_cols(const void *a, int64_t lda, int M, int K_logical, const int32_t *kmap,
                        const uint16_t *kinv, int K_phys, void *out, void *stream);

inline bool aligned(const void *p, size_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// GEMM workspace layout, every regime: [counter area][gathered activations]
// [fp32 partials]. The counter area holds the small-batch kernels' arrival
// counters and swap cells; it must be zero when a workspace is first used and
// every call leaves it zero, so no regime writes anything else there.
constexpr size_t COUNTER_BYTES = 512 * 1024;

// Workspace of one GEMM call: the caller's buffer, or (scratch_cap > 0) a
// static scratch array whose capacity bounds the call.
struct WorkspaceArg {
  void *ptr;
  size_t bytes;
  size_t scratch_cap;
};

// The body of oc_int4_gemm (oc_gemm.hip), shared by the entry points that
// bring their own workspace and by the allocation-free one.
int gemm_impl(const void *a, int64_t lda, int32_t a_dtype, int32_t M, int32_t K_logical, const int32_t *qt,
              const void *st, int32_t scale_dtype, const int32_t *zt, int32_t N, int32_t K_phys,
              int32_t group_rows, const int32_t *kmap, const uint16_t *kinv, const void *bias,
              int32_t bias_dtype, void *c, int64_t ldc, WorkspaceArg ws, int32_t regime, void *stream);

}  // namespace oc

// Returns OC_ERR_HIP (with the HIP error string) from the enclosing function
// when a HIP call fails.
#define OC_HIP_RETURN_IF_ERROR(expr)                                                   \
  do {                                                                                 \
    hipError_t oc_err_ = (expr);                                                       \
    if (oc_err_ != hipSuccess)                                                         \
      return ::oc::fail(OC_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(oc_err_)); \
  } while (0)

// Checks the launch that was just enqueued.
#define OC_RETURN_LAUNCH_STATUS() OC_HIP_RETURN_IF_ERROR(hipGetLastError())
