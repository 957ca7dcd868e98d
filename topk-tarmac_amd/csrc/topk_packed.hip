// Packed top-k (k <= 8) for head widths 8 .. 64, and the entry that routes
// d = 128 to topk_packed_d128.hip. The kernel is in topk_packed.hpp.
#include "topk_packed.hpp"

namespace tarmac {

size_t packed_lds_bytes(int dtype, int d, int kc, bool split) {
  const int row = dtype == kF32 ? (split ? (3 * d + 8) * 2 : (d + 4) * 4) : (d + 8) * 2;
  const int kcb = (kc + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
  return 16 + static_cast<size_t>(kcb) * row;
}

bool packed_split_supported(int dtype, int d) { return dtype == kF32 && d == 16; }

hipError_t run_topk_packed(const TopkArgs& a, bool split) {
  if (a.d == 128) return split ? hipErrorInvalidValue : run_topk_packed_d128(a);
  if (a.dtype == kF32) {
    if (split) return a.d == 16 ? launch_packed<float, 16, true>(a) : hipErrorInvalidValue;
    switch (a.d) {
      case 8: return launch_packed<float, 8, false>(a);
      case 16: return launch_packed<float, 16, false>(a);
      case 32: return launch_packed<float, 32, false>(a);
      case 64: return launch_packed<float, 64, false>(a);
    }
  } else {
    switch (a.d) {
      case 16: return launch_packed<bf16, 16, false>(a);
      case 32: return launch_packed<bf16, 32, false>(a);
      case 64: return launch_packed<bf16, 64, false>(a);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace tarmac
