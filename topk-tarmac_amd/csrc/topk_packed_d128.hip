// Packed top-k (k <= 8) at head width 128 (msg_dim 65 .. 128 after the
// module's zero padding): the kernel of topk_packed.hpp, instantiated in its
// own translation unit.
#include "topk_packed.hpp"

namespace tarmac {

hipError_t run_topk_packed_d128(const TopkArgs& a) {
  return a.dtype == kF32 ? launch_packed<float, 128, false>(a) : launch_packed<bf16, 128, false>(a);
}

}  // namespace tarmac
