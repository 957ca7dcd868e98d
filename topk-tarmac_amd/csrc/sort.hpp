// Workgroup bitonic sort (ascending) of P = R * T keys held in registers:
// thread t (t < T) holds positions t*R + r, r = 0..R-1.
//
// A compare-exchange stage of stride s runs
//   * in registers when s < R (partner r ^ s in the same thread),
//   * across lanes when R <= s < 64R (partner lane t ^ (s/R), same r: DPP or
//     ds_bpermute, no barrier),
//   * through LDS only when s >= 64R (partner in another wavefront),
// so a 512-key sort by 256 threads (R = 2) has 3 LDS stages instead of 45.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"

namespace tarmac {

// The value of lane (l ^ M), on the VALU: DPP inside a 16-lane row (quad
// permutes for M = 1, 2; row shifts for 4; a row rotation for 8) and the
// gfx950 row / half swaps for 16, 32 (v_permlane16_swap swaps the odd rows
// of its first operand with the even rows of its second; v_permlane32_swap
// the upper half of the first with the lower half of the second).
template <int M>
__device__ __forceinline__ uint32_t lane_xor(uint32_t x) {
  const int v = static_cast<int>(x);
  if constexpr (M == 1) {
    return static_cast<uint32_t>(dpp_mov<kDppQuadXor1>(v));
  } else if constexpr (M == 2) {
    return static_cast<uint32_t>(dpp_mov<kDppQuadXor2>(v));
  } else if constexpr (M == 4) {
    const int up = dpp_mov<0x104>(v);  // row_shl:4 -> lane l + 4
    const int dn = dpp_mov<0x114>(v);  // row_shr:4 -> lane l - 4
    return static_cast<uint32_t>((threadIdx.x & 4) ? dn : up);
  } else if constexpr (M == 8) {
    return static_cast<uint32_t>(dpp_mov<dpp_row_ror(8)>(v));
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (threadIdx.x & 16) ? r[0] : r[1];
  } else {
    static_assert(M == 32, "lane_xor: M must be a power of two below 64");
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (threadIdx.x & 32) ? r[0] : r[1];
  }
}

// Partner value for a cross-lane stage: DPP where one move per 32-bit half
// does it (xor 1, 2, 8), ds_bpermute otherwise (fewer VALU operations than
// the DPP shift pair or the lane swaps).
template <int M>
__device__ __forceinline__ uint32_t partner32(uint32_t x) {
  if constexpr (M == 1 || M == 2 || M == 8) return lane_xor<M>(x);
  else return static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), M));
}
template <int M>
__device__ __forceinline__ uint32_t key_xor(uint32_t x) { return partner32<M>(x); }
template <int M>
__device__ __forceinline__ uint64_t key_xor(uint64_t x) {
  const uint32_t lo = partner32<M>(static_cast<uint32_t>(x));
  const uint32_t hi = partner32<M>(static_cast<uint32_t>(x >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Compare-exchange with the partner's key: keep the min when take_min (the
// lower position of a block sorting up, or the upper of one sorting down).
template <typename K>
__device__ __forceinline__ K bitonic_keep(K mine, K other, bool take_min) {
  return ((mine < other) == take_min) ? mine : other;
}

// For strides >= R the direction is the same for all R keys of a thread.
__device__ __forceinline__ bool bitonic_take_min(int base, int stride, int size) {
  return ((base & size) == 0) == ((base & stride) == 0);
}

// In-register stages of one merge (strides R/2 .. 1, those below `size`).
template <typename K, int R>
__device__ __forceinline__ void bitonic_register_stages(K (&key)[R], int base, int size) {
#pragma unroll
  for (int s = R / 2; s >= 1; s >>= 1) {
    if (s < size) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if ((r & s) == 0) {
          const int pos = base + r;
          const bool up = (pos & size) == 0;
          const K a = key[r], b = key[r | s];
          const bool swap = (a > b) == up;
          key[r] = swap ? b : a;
          key[r | s] = swap ? a : b;
        }
      }
    }
  }
}

template <typename K, int R, int M>
__device__ __forceinline__ void bitonic_lane_stage(K (&key)[R], int base, int stride, int size) {
  const bool take_min = bitonic_take_min(base, stride, size);
  K other[R];
#pragma unroll
  for (int r = 0; r < R; ++r) other[r] = key_xor<M>(key[r]);
#pragma unroll
  for (int r = 0; r < R; ++r) key[r] = bitonic_keep(key[r], other[r], take_min);
}

// All threads of the workgroup call this (it has barriers); threads with
// t >= T pass active = false. lds: scratch of P keys.
template <typename K, int R>
__device__ void block_bitonic_sort(K (&key)[R], K* lds, int P, int t, bool active) {
  const int base = t * R;
  for (int size = 2; size <= P; size <<= 1) {
    int stride = size >> 1;
    for (; stride >= 64 * R; stride >>= 1) {  // partner in another wavefront
      __syncthreads();
      if (active) {
#pragma unroll
        for (int r = 0; r < R; ++r) lds[base + r] = key[r];
      }
      __syncthreads();
      if (active) {
        const bool take_min = bitonic_take_min(base, stride, size);
#pragma unroll
        for (int r = 0; r < R; ++r) key[r] = bitonic_keep(key[r], lds[(base + r) ^ stride], take_min);
      }
    }
    for (; stride >= R; stride >>= 1) {  // partner lane t ^ (stride / R)
      switch (stride / R) {
        case 1: bitonic_lane_stage<K, R, 1>(key, base, stride, size); break;
        case 2: bitonic_lane_stage<K, R, 2>(key, base, stride, size); break;
        case 4: bitonic_lane_stage<K, R, 4>(key, base, stride, size); break;
        case 8: bitonic_lane_stage<K, R, 8>(key, base, stride, size); break;
        case 16: bitonic_lane_stage<K, R, 16>(key, base, stride, size); break;
        default: bitonic_lane_stage<K, R, 32>(key, base, stride, size); break;
      }
    }
    if (active) bitonic_register_stages<K, R>(key, base, size);
  }
}

// Bitonic sort (ascending) of 64 * R keys by one wavefront: lane l holds
// positions l*R .. l*R+R-1. Every stage is a register or lane stage (no LDS,
// no barrier); sizes and strides are compile-time, so the stages unroll into
// straight-line code and the R exchanges of a lane stage overlap.
template <typename K, int R>
__device__ __forceinline__ void wave_bitonic_sort(K (&key)[R], int lane) {
  const int base = lane * R;
#pragma unroll
  for (int size = 2; size <= 64 * R; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride >= R; stride >>= 1) {
      if constexpr (R <= 32) {
        switch (stride / R) {
          case 1: bitonic_lane_stage<K, R, 1>(key, base, stride, size); break;
          case 2: bitonic_lane_stage<K, R, 2>(key, base, stride, size); break;
          case 4: bitonic_lane_stage<K, R, 4>(key, base, stride, size); break;
          case 8: bitonic_lane_stage<K, R, 8>(key, base, stride, size); break;
          case 16: bitonic_lane_stage<K, R, 16>(key, base, stride, size); break;
          default: bitonic_lane_stage<K, R, 32>(key, base, stride, size); break;
        }
      }
    }
    bitonic_register_stages<K, R>(key, base, size);
  }
}

}  // namespace tarmac
