// Launch-floor probe: one thread writes one float (scripts/launch_overhead.py:28-30).
#include "tarmac_internal.hpp"

namespace tarmac {

__global__ void noop_kernel(float* out) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *out = 1.0f;
}

hipError_t run_noop(float* out, void* stream) {
  hipLaunchKernelGGL(noop_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), out);
  return hipGetLastError();
}

}  // namespace tarmac
