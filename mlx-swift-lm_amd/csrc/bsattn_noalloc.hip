// bsattn_noalloc.hip -- the fixed device scratch of bsattn_decode_noalloc.
//
// The decode's workspaces (block scores, MFMA score bounds, selected
// indices, split partials) normally belong to the cache handle.  For callers
// that cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid allocation) the no-allocation decode places them in
// `scratch`, a file-scope device array of kNoAllocScratchBytes that every
// call on a device shares; each GPU the library runs on holds its own copy
// until the process ends.  In host code the array's name is only a host-side
// stand-in: host code uses the address hipGetSymbolAddress returns for the
// current device, never the name.
#include <hip/hip_runtime.h>

#include <mutex>

#include "bsattn_internal.h"

namespace bsattn {

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t noalloc_scratch(int device, void** out) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device] == nullptr) {
    // once per device, with that device current (the caller's DeviceGuard)
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return hipSuccess;
}

}  // namespace bsattn
