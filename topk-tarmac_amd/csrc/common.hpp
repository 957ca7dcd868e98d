// Shared device helpers for the TarMAC attention-core kernels (gfx950 / CDNA4).
//
// Layout conventions used by every kernel in this directory:
//   * q, k, v, out are row-major contiguous [B, N, d] (fp32 or bf16);
//   * one wavefront (64 lanes) owns a tile of 16 query rows;
//   * scores are formed as an S^T tile (16 keys x 16 queries) with MFMA, so
//     after the instruction lane l holds the four scores of query (l % 16)
//     against keys 4*(l/16) + r, r = 0..3 -- every lane works on exactly one
//     query and selection / softmax state stays in that lane's registers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tarmac {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t bf16;  // raw bfloat16 storage

constexpr int kWave = 64;
constexpr int kCUs = 256;  // compute units of an MI355X (8 XCDs x 32)

__device__ __forceinline__ float bf16_to_f32(bf16 h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// a.lo * b.lo + a.hi * b.hi + c for bf16 pairs in 32-bit words (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Round-to-nearest-even fp32 -> bf16 (the rounding Tensor.to(torch.bfloat16) uses).
__device__ __forceinline__ bf16 f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16>(u >> 16);
}

// D += A(16x4) * B(4x16), fp32. Lane l supplies A[l%16][l/16] and B[l/16][l%16];
// returns D[4*(l/16)+r][l%16] in element r. Rounds like a sequential fmaf chain
// over the four contraction slots, in slot order.
__device__ __forceinline__ f32x4 mfma_f32_16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// D += A(16x16) * B(16x16), bf16 inputs, fp32 accumulate. Lane l supplies
// A[l%16][4*(l/16)+e] and B[4*(l/16)+e][l%16], e = 0..3.
__device__ __forceinline__ f32x4 mfma_bf16_16x16x16(i16x4 a, i16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// D += A(16x32) * B(32x16), bf16 inputs (gfx950). Lane l supplies
// A[l%16][8*(l/16)+e] and B[8*(l/16)+e][l%16], e = 0..7.
__device__ __forceinline__ f32x4 mfma_bf16_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Workgroups are dispatched round-robin over the 8 XCDs (id % 8). Remap the
// hardware id so that consecutive logical ids run on the same XCD and share
// its L2 (all query tiles of one batch row read the same K and V).
__device__ __forceinline__ int xcd_logical_block(int hw, int nblocks) {
  constexpr int X = 8;
  const int q = nblocks / X, r = nblocks % X;
  const int x = hw % X, local = hw / X;
  return (x < r) ? x * (q + 1) + local : r * (q + 1) + (x - r) * q + local;
}

// 2^x on the transcendental unit (v_exp_f32), without the denormal-range
// fix-up exp2f adds: softmax terms below 2^-126 of the row maximum flush to 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2eF = 1.4426950408889634f;

__device__ __forceinline__ bool is_pow2_scale(float s) {
  uint32_t u = __float_as_uint(s);
  return (u & 0x007fffffu) == 0u;
}

// Ask the scheduler for a pipeline of NM groups {1 MFMA, VPM VALU}, preceded
// by NDS LDS reads, within the current basic block.
template <int NDS, int NM, int VPM>
__device__ __forceinline__ void interleave_mfma_valu() {
  if constexpr (NDS > 0) __builtin_amdgcn_sched_group_barrier(0x100, NDS, 0);
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
  }
}

// Lane moves inside a 16-lane row with DPP: VALU operations, no LDS traffic
// (a __shfl_xor becomes ds_bpermute, an LDS-pipeline instruction).
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int dpp_row_ror(int n) { return 0x120 + n; }

template <int CTRL>
__device__ __forceinline__ int dpp_mov(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(dpp_mov<CTRL>(__float_as_int(x)));
}

// Sum over the 4 lanes of a quad; every lane gets the same value.
__device__ __forceinline__ float quad_sum(float x) {
  x += dpp_mov<kDppQuadXor1>(x);
  return x + dpp_mov<kDppQuadXor2>(x);
}

// Sum over aligned groups of G consecutive lanes (G = 1, 2, 4, 8 or 16);
// every lane of a group gets the group's sum. Within quads by DPP (VALU),
// beyond by ds_swizzle in xor mode (no lane-index arithmetic).
template <int G>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "group of 1..16 lanes");
  if constexpr (G >= 2) x += dpp_mov<kDppQuadXor1>(x);
  if constexpr (G >= 4) x += dpp_mov<kDppQuadXor2>(x);
  if constexpr (G >= 8)
    x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x1f | (4 << 10)));
  if constexpr (G >= 16)
    x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x1f | (8 << 10)));
  return x;
}

// x of this lane plus x of the lane 16 (xor 16) or 32 (xor 32) away:
// v_permlane16_swap / v_permlane32_swap, VALU only.
__device__ __forceinline__ float add_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Reductions over the 16 lanes of a row (rotations by 8, 4, 2, 1: each step
// adds a lane's partner's partial, so every lane ends with the same value).
template <typename T, typename Op>
__device__ __forceinline__ T row16_reduce(T x, Op op) {
  x = op(x, dpp_mov<dpp_row_ror(8)>(x));
  x = op(x, dpp_mov<dpp_row_ror(4)>(x));
  x = op(x, dpp_mov<dpp_row_ror(2)>(x));
  return op(x, dpp_mov<dpp_row_ror(1)>(x));
}
// Over the lanes of a row that agree in (lane % 4): rotations by 8 and 4.
template <typename T, typename Op>
__device__ __forceinline__ T row16_reduce_stride4(T x, Op op) {
  x = op(x, dpp_mov<dpp_row_ror(8)>(x));
  return op(x, dpp_mov<dpp_row_ror(4)>(x));
}

// +inf in an SGPR, from an instruction the compiler cannot fold (a scalar
// copy: VALU work stays visible to the compiler, which inserts the wait
// states that DPP, lane swaps and MFMA results need after it).
__device__ __forceinline__ float opaque_inf() {
  float r;
  asm("s_mov_b32 %0, 0x7f800000" : "=s"(r));
  return r;
}

// max of two non-NaN floats as one v_med3_f32 against an opaque +inf,
// without the canonicalising copies fmaxf adds for operands the compiler
// cannot prove canonical (lane moves, MFMA results).
__device__ __forceinline__ float max_plain(float a, float b) {
  return __builtin_amdgcn_fmed3f(a, b, opaque_inf());
}

// (a, ia) ranks before (b, ib): higher score first, lower index on ties.
__device__ __forceinline__ bool ranks_before(float a, int ia, float b, int ib) {
  return a > b || (a == b && ia < ib);
}

}  // namespace tarmac
