// noalloc.hip — the fixed device scratch of the allocation-free forward
// entry (pfhip_model_forward_device_noalloc, include/pfhip.h).
//
// The array lives in the library's code object: each GPU the library runs on
// holds its own copy from the first symbol lookup on that device until the
// process ends. Host code must not pass `scratch` itself to a kernel or a
// copy (in host code the name is only a stand-in for the device symbol);
// noalloc_scratch() returns the array's address on a device, looked up once
// per device with that device current.
#include <mutex>

#include "pfhip_internal.h"

namespace pf {

namespace {

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void* g_ptr[MAX_DEVICES] = {};

}  // namespace

void* noalloc_scratch(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  PF_CHECK(device >= 0 && device < MAX_DEVICES, "noalloc scratch: device ordinal out of range");
  if (!g_ptr[device]) {
    int cur = 0;
    PF_HIP(hipGetDevice(&cur));
    if (cur != device) PF_HIP(hipSetDevice(device));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != device) PF_HIP(hipSetDevice(cur));
    PF_HIP(e);
    PF_CHECK(p != nullptr, "noalloc scratch: hipGetSymbolAddress returned no address");
    g_ptr[device] = p;
  }
  return g_ptr[device];
}

}  // namespace pf
