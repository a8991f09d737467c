// Scratch memory of the allocation-free entry point (gs_linear_dot_noalloc): a file-scope
// device array, one copy on every GPU that calls that entry point, held until the process
// ends.  It lives in a translation unit of its own, so its code object -- and with it the
// array's reservation -- is loaded on a device only when noalloc_scratch() first looks the
// array up there, not by the other entry points' kernels.  Host code never uses the array's
// name as an address (on the host it is only a stand-in for the symbol): the device address
// comes from hipGetSymbolAddress, looked up once per device with that device current.
#include <mutex>
#include <string>

#include "gs_common.h"

static __device__ __align__(256) unsigned char scratch[GS_LINEAR_NOALLOC_SCRATCH_BYTES];

namespace gs {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

int noalloc_scratch(hipStream_t s, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(GS_ERR_LAUNCH, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(GS_ERR_UNSUPPORTED, "gs_linear_dot_noalloc: device index above 63");
  if (s != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(s, &sdev);
    if (e != hipSuccess)
      return fail(GS_ERR_LAUNCH, std::string("hipStreamGetDevice: ") + hipGetErrorString(e));
    if (sdev != dev)
      return fail(GS_ERR_INVALID,
                  "gs_linear_dot_noalloc: the stream belongs to another device than the "
                  "current one");
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(GS_ERR_LAUNCH, std::string("hipGetSymbolAddress(scratch): ") +
                                     hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GS_OK;
}

}  // namespace gs
