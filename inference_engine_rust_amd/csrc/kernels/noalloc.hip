// Device scratch for the no-allocation decode attention entry point: one file-scope array per
// device, resolved to its device address once per device with hipGetSymbolAddress. The host-side
// name `scratch` is not a device address; only the resolved pointer is passed to kernels.
#include <mutex>

#include "../iek_internal.h"

namespace iek {

static __device__ __align__(256) char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};
}  // namespace

// The scratch of the device the work runs on: the stream's device (the current device for the
// null stream). The first call on a device resolves the array's address with that device current.
void* noalloc_scratch(hipStream_t st) {
  int cur = 0, dev = 0;
  IEK_HIP(hipGetDevice(&cur));
  dev = cur;
  if (st) IEK_HIP(hipStreamGetDevice(st, &dev));
  if (dev < 0 || dev >= kMaxDevices) fail(ST_DEVICE, "device index out of range");
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    if (dev != cur) IEK_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) IEK_HIP(hipSetDevice(cur));
    IEK_HIP(e);
    if (!p) fail(ST_DEVICE, "hipGetSymbolAddress returned a null scratch address");
    g_ptr[dev] = p;
  }
  return g_ptr[dev];
}

}  // namespace iek
