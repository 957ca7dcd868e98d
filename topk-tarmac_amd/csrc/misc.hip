// Diagnostics: the launch-floor probe (one thread writes one float,
// scripts/launch_overhead.py:28-30) and a probe of the bf16 MFMA's fp32
// accumulation, whose error bound the exact bf16 / split-bf16 top-k proofs
// rely on.
#include "common.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

__global__ void noop_kernel(float* out) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *out = 1.0f;
}

hipError_t run_noop(float* out, void* stream) {
  hipLaunchKernelGGL(noop_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), out);
  return hipGetLastError();
}

// One wave per tile: chain v_mfma_f32_16x16x32_bf16 products from +0 and
// store the 16 x 16 result. a, b: [T][chain][64 lanes][8] bf16 operands in
// the instruction's lane layout; out: [T][64 lanes][4].
__global__ void __launch_bounds__(64)
mfma_bf16_probe_kernel(const bf16* __restrict__ a, const bf16* __restrict__ b,
                       float* __restrict__ out, int T, int chain) {
  const int lane = threadIdx.x;
  for (int t = blockIdx.x; t < T; t += gridDim.x) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < chain; ++c) {
      const size_t off = (static_cast<size_t>(t) * chain + c) * 64 * 8 + static_cast<size_t>(lane) * 8;
      acc = mfma_bf16_16x16x32(*reinterpret_cast<const bf16x8*>(a + off),
                               *reinterpret_cast<const bf16x8*>(b + off), acc);
    }
    *reinterpret_cast<f32x4*>(out + (static_cast<size_t>(t) * 64 + lane) * 4) = acc;
  }
}

hipError_t run_mfma_bf16_probe(const void* a, const void* b, float* out, int T, int chain,
                               void* stream) {
  const int grid = T < 4096 ? T : 4096;
  hipLaunchKernelGGL(mfma_bf16_probe_kernel, dim3(grid), dim3(64), 0,
                     static_cast<hipStream_t>(stream), static_cast<const bf16*>(a),
                     static_cast<const bf16*>(b), out, T, chain);
  return hipGetLastError();
}

}  // namespace tarmac
