// The allocation-free GEMM entry point (oc_int4_gemm_noalloc): oc_int4_gemm
// with its scratch in a static device array instead of a caller workspace,
// for callers that cannot allocate.
#include <hip/hip_runtime.h>

#include <mutex>

#include "oc_internal.h"

namespace oc {
namespace {

// One array per device (each GPU the library runs on holds it until the
// process ends). Its device address is looked up once per device with
// hipGetSymbolAddress, with that device current; host code uses only that
// address, never the array's name.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t{32} << 20;
static_assert(NOALLOC_SCRATCH_BYTES > COUNTER_BYTES, "scratch must hold the counter area");
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

// The counter area must start at zero (every call leaves it zero again): a
// fill kernel clears it at set-up (a kernel, not a memset, so a set-up that
// happens under graph capture records a node that replays correctly).
__global__ __launch_bounds__(256) void clear_counters_kernel(uint4 *__restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = make_uint4(0, 0, 0, 0);
}

constexpr int SCRATCH_MAX_DEVICES = 64;
struct ScratchSlot {
  std::once_flag once;
  void *ptr = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot scratch_slots[SCRATCH_MAX_DEVICES];

// Device address of the current device's scratch; the first call on a device
// looks it up and clears the counter area on `s`.
int scratch_of_current_device(hipStream_t s, void **out) {
  int dev = -1;
  OC_HIP_RETURN_IF_ERROR(hipGetDevice(&dev));
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) return fail(OC_ERR_UNSUPPORTED, "device %d out of range", dev);
  ScratchSlot &slot = scratch_slots[dev];
  std::call_once(slot.once, [&] {
    void *ptr = nullptr;
    slot.err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (slot.err != hipSuccess || !ptr) return;
    constexpr int n = static_cast<int>(COUNTER_BYTES / sizeof(uint4));
    hipLaunchKernelGGL(clear_counters_kernel, dim3((n + 255) / 256), dim3(256), 0, s, static_cast<uint4 *>(ptr), n);
    slot.err = hipGetLastError();
    if (slot.err == hipSuccess) slot.ptr = ptr;
  });
  if (slot.err != hipSuccess || !slot.ptr)
    return fail(OC_ERR_HIP, "static scratch set-up failed: %s", hipGetErrorString(slot.err));
  *out = slot.ptr;
  return OC_OK;
}

}  // namespace
}  // namespace oc

using namespace oc;

extern "C" {

int oc_int4_gemm_noalloc(const void *a, int64_t lda, int32_t a_dtype, int32_t M, int32_t K_logical,
                         const int32_t *qt, const void *st, int32_t scale_dtype, const int32_t *zt, int32_t N,
                         int32_t K_phys, int32_t group_rows, const int32_t *kmap, const uint16_t *kinv,
                         const void *bias, int32_t bias_dtype, void *c, int64_t ldc, int32_t regime, void *stream) {
  clear_error();
  if (M == 0) return OC_OK;
  void *ptr = nullptr;
  const int status = scratch_of_current_device(static_cast<hipStream_t>(stream), &ptr);
  if (status != OC_OK) return status;
  return gemm_impl(a, lda, a_dtype, M, K_logical, qt, st, scale_dtype, zt, N, K_phys, group_rows, kmap, kinv, bias,
                   bias_dtype, c, ldc, WorkspaceArg{ptr, NOALLOC_SCRATCH_BYTES, NOALLOC_SCRATCH_BYTES}, regime,
                   stream);
}

size_t oc_int4_gemm_noalloc_scratch_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

}  // extern "C"
