// Static device scratch of fmlp_bwd_noalloc, in a translation unit of its own.
//
// The backward's workspace (the dW programs' fp32 partials of a B split and, in the
// stored-dZ form, dZ) lives in this file-scope device array instead of caller memory. The
// array is the only object of this file's code object, which the HIP runtime loads onto a
// device the first time the array's address is looked up there (scratch_current_device,
// called by fmlp_bwd_noalloc only): the 64 MiB are reserved on a device from the first
// no-alloc call on it until the process ends, and not at all in processes that never make
// one. Every call on a device shares that device's copy, so calls that overlap on one
// device race. The kernels write every byte they later read: nothing in it has to start at
// zero.
#include "fmlp_launch.h"

#include <mutex>

namespace fmlp {

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

hipError_t scratch_current_device(void** ptr) {
  constexpr int kDevices = 64;
  static std::mutex mu;
  static void* addr[kDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    // the host-side name `scratch` is not a device address: only this lookup yields one
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return hipSuccess;
}

}  // namespace fmlp
