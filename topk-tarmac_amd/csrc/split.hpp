// Split-bf16 operands for fp32 scores on bf16 MFMA: x = hi + mid + lo (bf16
// each), the query fragment and key rows of the S^T tile in split form, and
// the staging of split key rows into LDS. Used by the filter and packed top-k
// kernels.
#pragma once

#include "frag.hpp"

namespace tarmac {

// bf16 score error bound, relative to |q| |k_j|: bf16 MFMA sums exact
// products with an fp32 accumulation error that is measured, not derived
// (at most 2^-20.25 of the sum of their magnitudes, the worst seen 2^-20.5:
// one dominant product among small ones, on 16x16x32 and 32x32x16 chains of
// up to 128 products); the canonical fp32 chain adds <= d 2^-24 of it (one
// rounding per step); split scores drop three products of <= 2^-24 each;
// sum_c |q_c k_c| <= |q| |k_j|. 2^-18 (d <= 32), 2^-17 (d = 64) and 2^-16
// (d = 128) cover the sum with a margin of 1.25 or more, including the fp32
// rounding of the bound itself.
template <int D>
constexpr float packed_eps() {
  static_assert(D <= 128, "the bound covers chains of up to 128 products");
  return D <= 32 ? 1.0f / 262144.0f : (D <= 64 ? 1.0f / 131072.0f : 1.0f / 65536.0f);
}
constexpr float kPackedNormLimit = 1.329228e36f;  // 2^120: |q| max|k| at or above fails the proof

// An upper bound on |q| max_j |k_j| from the squared norms: one v_sqrt_f32
// (within 1 ulp) of the product (one rounding), raised by 2^-21 (more than
// both errors and the raise's own rounding). Products below 2^-100 give +inf,
// which fails the proof (the exact pass decides such queries: their scores
// could sit among denormals, where the MFMA and the fmaf chain may flush
// differently); an overflowing product gives +inf too.
__device__ __forceinline__ float proof_norm(float qn2, float kmax2) {
  const float p = qn2 * kmax2;
  return p >= 7.88860905e-31f ? __builtin_amdgcn_sqrtf(p) * 1.00000048f : INFINITY;
}

// ---------------------------------------------------------------------------
// split-bf16 fragments: S^T tile (16 keys x 16 queries) of split products
// ---------------------------------------------------------------------------

// x = hi + mid + lo (bf16 each, round to nearest) with |x - hi - mid - lo| <= 2^-24 |x|.
__device__ __forceinline__ void split3_bf16(float x, __bf16& hi, __bf16& mid, __bf16& lo) {
  hi = static_cast<__bf16>(x);
  const float r1 = x - static_cast<float>(hi);
  mid = static_cast<__bf16>(r1);
  lo = static_cast<__bf16>(r1 - static_cast<float>(mid));
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two elements at a time: one packed conversion per part (v_cvt_pk_bf16_f32),
// results already packed as bf16 pairs. exact: both elements satisfy
// x == hi + mid + lo exactly (the last residual is representable in bf16;
// then the fp32 sums (hi + mid) + lo rebuild x bit for bit). It fails only
// near the ends of the fp32 range, or for NaN.
__device__ __forceinline__ void split3_pair(float x0, float x1, uint32_t& hi, uint32_t& mid,
                                            uint32_t& lo, bool& exact) {
  bf16x2_t h = {static_cast<__bf16>(x0), static_cast<__bf16>(x1)};
  hi = __builtin_bit_cast(uint32_t, h);
  // the halves come from the packed word (an opaque copy keeps the compiler
  // from converting x0 a second time for the low half): 11 VALU per pair
  asm("" : "+v"(hi));
  const float r0 = x0 - __uint_as_float(hi << 16), r1 = x1 - __uint_as_float(hi & 0xffff0000u);
  bf16x2_t m = {static_cast<__bf16>(r0), static_cast<__bf16>(r1)};
  mid = __builtin_bit_cast(uint32_t, m);
  asm("" : "+v"(mid));
  const float s0 = r0 - __uint_as_float(mid << 16), s1 = r1 - __uint_as_float(mid & 0xffff0000u);
  bf16x2_t l = {static_cast<__bf16>(s0), static_cast<__bf16>(s1)};
  lo = __builtin_bit_cast(uint32_t, l);
  exact = __uint_as_float(lo << 16) == s0 && __uint_as_float(lo & 0xffff0000u) == s1;
}

__device__ __forceinline__ void split3_pair(float x0, float x1, uint32_t& hi, uint32_t& mid,
                                            uint32_t& lo) {
  bool unused;
  split3_pair(x0, x1, hi, mid, lo, unused);
}

// The six products whose size is >= 2^-16 of q.k are formed:
//   hi.hi, hi.mid, mid.hi, mid.mid, hi.lo, lo.hi
// (dropped: mid.lo, lo.mid, lo.lo, each <= 2^-24 |q_c k_c|).
template <int D>
struct SplitFrag;

// d = 16: three 16x16x32 steps over two distinct key operands, from rows
// stored as lo[16] hi[16] mid[16] pad[8] (two 16-byte LDS reads per tile):
//   A1 = [k_hi | k_mid] (halves 16..47), A2 = [k_lo | k_hi] (halves 0..31)
//   step 0: A1 x [q_hi  | q_hi ] = hi.hi + mid.hi
//   step 1: A1 x [q_mid | q_mid] = hi.mid + mid.mid
//   step 2: A2 x [q_hi  | q_lo ] = lo.hi + hi.lo
template <>
struct SplitFrag<16> {
  static constexpr int LDK = 3 * 16 + 8;
  static constexpr int OFF_L = 0, OFF_H = 16, OFF_M = 32;  // part offsets in a row
  static constexpr int NI = 3;
  bf16x8 q[3];
  // Returns the sum of squares of the 8 elements this lane loaded; lane
  // groups g and g ^ 1 together hold the whole row.
  __device__ __forceinline__ float load_q(const float* qrow, int grp) {
    float x[8];
    ld_f32<8>(x, qrow + 8 * (grp & 1));
    const bool lower = grp < 2;
    uint32_t h[4], m[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split3_pair(x[2 * e], x[2 * e + 1], h[e], m[e], l[e]);
    uint32_t w2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) w2[e] = lower ? h[e] : l[e];
    q[0] = __builtin_bit_cast(bf16x8, h);
    q[1] = __builtin_bit_cast(bf16x8, m);
    q[2] = __builtin_bit_cast(bf16x8, w2);
    float n2 = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) n2 = fmaf(x[e], x[e], n2);
    return n2;
  }
  // |q|^2 from the per-lane sums of load_q
  __device__ __forceinline__ static float row_norm2(float part) { return add_xor16(part); }
  struct KF { bf16x8 a[2]; };
  __device__ __forceinline__ static KF load_k(const bf16* krow, int grp) {
    KF f;
    f.a[0] = *reinterpret_cast<const bf16x8*>(krow + OFF_H + 8 * grp);  // [hi | mid]
    f.a[1] = *reinterpret_cast<const bf16x8*>(krow + OFF_L + 8 * grp);  // [lo | hi]
    return f;
  }
  __device__ __forceinline__ f32x4 step(const KF& kf, int i, f32x4 acc) const {
    return mfma_bf16_16x16x32(kf.a[i == 2 ? 1 : 0], q[i], acc);
  }
};

// d = 32 (one 32-wide contraction per product) and d = 64 (two halves).
template <int D>
struct SplitFragWide {
  static_assert(D == 32 || D == 64, "split fragment width");
  static constexpr int NH = D / 32;
  static constexpr int LDK = 3 * D + 8;  // hi[D] mid[D] lo[D] pad
  static constexpr int OFF_H = 0, OFF_M = D, OFF_L = 2 * D;  // part offsets in a row
  static constexpr int NI = 6 * NH;
  bf16x8 qh[NH], qm[NH], ql[NH];
  // Returns the sum of squares of the elements this lane loaded; the four
  // lane groups together hold the whole row.
  __device__ __forceinline__ float load_q(const float* qrow, int grp) {
    float n2 = 0.f;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      float x[8];
      ld_f32<8>(x, qrow + 32 * h + 8 * grp);
#pragma unroll
      for (int e = 0; e < 8; ++e) n2 = fmaf(x[e], x[e], n2);
      uint32_t a[4], b[4], c[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split3_pair(x[2 * e], x[2 * e + 1], a[e], b[e], c[e]);
      qh[h] = __builtin_bit_cast(bf16x8, a);
      qm[h] = __builtin_bit_cast(bf16x8, b);
      ql[h] = __builtin_bit_cast(bf16x8, c);
    }
    return n2;
  }
  __device__ __forceinline__ static float row_norm2(float part) { return add_xor32(add_xor16(part)); }
  struct KF { bf16x8 hi[NH], mid[NH], lo[NH]; };
  __device__ __forceinline__ static KF load_k(const bf16* krow, int grp) {
    KF f;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      f.hi[h] = *reinterpret_cast<const bf16x8*>(krow + 32 * h + 8 * grp);
      f.mid[h] = *reinterpret_cast<const bf16x8*>(krow + D + 32 * h + 8 * grp);
      f.lo[h] = *reinterpret_cast<const bf16x8*>(krow + 2 * D + 32 * h + 8 * grp);
    }
    return f;
  }
  __device__ __forceinline__ f32x4 step(const KF& kf, int i, f32x4 acc) const {
    const int h = i / 6, p = i % 6;
    switch (p) {
      case 0: return mfma_bf16_16x16x32(kf.hi[h], qh[h], acc);
      case 1: return mfma_bf16_16x16x32(kf.hi[h], qm[h], acc);
      case 2: return mfma_bf16_16x16x32(kf.mid[h], qh[h], acc);
      case 3: return mfma_bf16_16x16x32(kf.mid[h], qm[h], acc);
      case 4: return mfma_bf16_16x16x32(kf.hi[h], ql[h], acc);
      default: return mfma_bf16_16x16x32(kf.lo[h], qh[h], acc);
    }
  }
};

template <>
struct SplitFrag<32> : SplitFragWide<32> {};
template <>
struct SplitFrag<64> : SplitFragWide<64> {};

__device__ __forceinline__ uint2 pack_bf16x4(const __bf16 (&v)[4]) {
  uint2 p;
  p.x = __builtin_bit_cast(uint16_t, v[0]) | (uint32_t(__builtin_bit_cast(uint16_t, v[1])) << 16);
  p.y = __builtin_bit_cast(uint16_t, v[2]) | (uint32_t(__builtin_bit_cast(uint16_t, v[3])) << 16);
  return p;
}

// Stage `rows` fp32 key rows as split bf16 rows (zero rows up to rows_pad) and
// return this thread's max squared row norm. exact is cleared if some element
// is not rebuilt bit for bit by (hi + mid + lo) in fp32 (only for values near
// the ends of the fp32 range, or NaN).
template <int D>
__device__ __forceinline__ float stage_split(bf16* lds, const float* src, int rows, int rows_pad,
                                         bool& exact) {
  constexpr int VPR = D / 4;  // float4 per row; VPR consecutive threads share a row
  constexpr int LDK = SplitFrag<D>::LDK;
  constexpr int U = kStageBatch;
  float mx = 0.f;
  const int total = rows_pad * VPR;  // a multiple of 64: whole wavefronts agree on v < total
  const int avail = rows * VPR;      // vectors backed by source rows
  // the rows are contiguous: vector v sits at byte 16 v of the chunk (a 32-bit
  // offset from the uniform base)
  const char* base = reinterpret_cast<const char*>(src);
  for (int v0 = threadIdx.x; v0 < total; v0 += U * blockDim.x) {
    f32x4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * blockDim.x;
      // zero only padding rows (the branch is skipped when no lane pads)
      if (v < avail)
        x[u] = *reinterpret_cast<const f32x4*>(base + static_cast<uint32_t>(v) * 16u);
      else
        x[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * blockDim.x, row = v / VPR, cv = v - row * VPR;
      if (v >= total) break;
      uint2 hi, mid, lo;
      bool e0, e1;
      split3_pair(x[u][0], x[u][1], hi.x, mid.x, lo.x, e0);
      split3_pair(x[u][2], x[u][3], hi.y, mid.y, lo.y, e1);
      exact = exact && e0 && e1;
      bf16* dst = lds + row * LDK + 4 * cv;
      *reinterpret_cast<uint2*>(dst + SplitFrag<D>::OFF_H) = hi;
      *reinterpret_cast<uint2*>(dst + SplitFrag<D>::OFF_M) = mid;
      *reinterpret_cast<uint2*>(dst + SplitFrag<D>::OFF_L) = lo;
      const float n2 = group_sum<VPR>(
          x[u][0] * x[u][0] + x[u][1] * x[u][1] + x[u][2] * x[u][2] + x[u][3] * x[u][3]);
      mx = fmaxf(mx, n2);
    }
  }
  return mx;
}

}  // namespace tarmac
