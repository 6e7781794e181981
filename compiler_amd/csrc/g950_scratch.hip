// The library's static device scratch for g950_launch_noalloc: workspace
// for callers that cannot allocate device memory (code
// under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
//
// Each GPU the library runs on holds its own copy of the array at its own
// address from the first lookup until the process ends.  In host code the
// array's name is only a stand-in for the symbol: its device address comes
// from hipGetSymbolAddress, looked up once per device with that device
// current, and only that address is handed to kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/g950rt.h"

static __device__ __align__(256) char scratch[G950_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];
hipError_t g_err[kMaxDevices];
bool g_done[kMaxDevices];
}  // namespace

// Device address of this device's scratch array (the current device must be
// `device`).  The lookup runs once per device; later calls return its result.
__attribute__((visibility("hidden"))) hipError_t g950_scratch_address(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_done[device]) {
    void* ptr = nullptr;
    g_err[device] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_ptr[device] = g_err[device] == hipSuccess ? ptr : nullptr;
    g_done[device] = true;
  }
  *out = g_ptr[device];
  return g_err[device];
}
