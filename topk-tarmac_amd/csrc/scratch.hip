// Library-held device workspace, for entry points whose callers cannot
// allocate device memory (code under graph capture, serving loops that forbid
// hipMalloc). One fixed array per GPU, resident until the process ends; every
// call on a GPU shares it, so calls that overlap on one GPU race on it.
//
// The array's name is a host-side stand-in in host code: its device address
// is looked up once per device with hipGetSymbolAddress (each GPU holds its
// own copy at its own address) and only that address is handed to kernels.
#include <mutex>

#include "tarmac_internal.hpp"

namespace tarmac {

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

hipError_t scratch_address(void** out) {
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace tarmac
