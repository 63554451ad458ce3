/*
 * The static device scratch behind tm_launch_noalloc: device memory that
 * exists from the moment this library's code object is loaded on a device
 * until the process ends, so a launch that needs a work buffer (the fp32 dQ
 * accumulator of attn_bwd_fused) can run without allocating.
 *
 * Host code never uses the array's name as a device address (on the host it
 * names a stand-in, not the device copy): tm_scratch_address resolves the
 * device copy with hipGetSymbolAddress, once per device while that device is
 * current, and every later use takes the resolved pointer.
 */
#include <hip/hip_runtime.h>

#include <mutex>

#include "scratch.h"

static __device__ __align__(256) float scratch[TM_SCRATCH_BYTES / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch_ptr[kMaxDevices];
}  // namespace

hipError_t tm_scratch_address(void **ptr) {
  int device = -1;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return status;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    status = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (status != hipSuccess) return status;
    g_scratch_ptr[device] = p;
  }
  *ptr = g_scratch_ptr[device];
  return hipSuccess;
}
