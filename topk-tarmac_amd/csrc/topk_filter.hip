// Exact top-k attention by filter-and-verify.
//
// Same function as topk_small_kernel on fp32 inputs (scores in the canonical
// fp32 order, top-k with ties to the lower index, k-softmax, gathered
// aggregation). On bf16 inputs (d = 16) the scores are the canonical fp32
// scores of the inputs converted to fp32 (the rule the large-k kernels also
// follow), so the selection is exact there too. The N-wide scoring pass runs
// on bf16 MFMA:
//
//  1. filter: fp32 inputs: every (query, key) dot is formed from three-way
//     split operands x = x_hi + x_mid + x_lo (bf16 each) with the six
//     products of size >= 2^-16, which approximates the fp32 dot to
//     |a - q.k| <= 2^-21 sum_c |q_c k_c| (representation 2^-22, bf16 MFMA
//     accumulation measured <= 2^-21.9 of the term magnitudes). bf16 inputs:
//     one bf16 product (exact products, the same accumulation error). The
//     canonical fp32 dot (d roundings) is within d 2^-24 sum_c |q_c k_c| of
//     q.k. Selection runs on packed values (the
//     filter score with the key's position in its low mantissa bits, see
//     pack8): each lane keeps its k+2 largest with max / med3 only, and the
//     four lane lists of a query merge into k+1 candidates plus the (k+2)-th
//     entry, identically on the four lanes.
//  2. verify: the k+1 candidates are rescored in the canonical fp32 order and
//     their exact top k taken. Every other key's filter score is at most C,
//     the largest value that truncates like the (k+2)-th entry. If C plus
//     eps |q| max_j |k_j| (eps = filter_eps<d>(), >= the sum of the bounds
//     above, with margin; sum_c |q_c k_c| <= |q| |k_j|), scaled, is strictly
//     below the k-th exact score, no other key can reach the top
//     k, so the result IS the exact top k. Rescoring one spare candidate
//     settles near-ties between the k-th and (k+1)-th scores (duplicated keys
//     included) without the fallback.
//  3. fallback: a 16-query tile with any unproven query recomputes exactly
//     (fp32 MFMA over all keys, read from the LDS copy when that holds them
//     all exactly), so the result never depends on the filter -- only the
//     time does.
//
// Reference behaviour: src/kernels/fused_topk_attention.py:211-333 and
// src/kernels/streaming_topk_attention.py:66-258 (including the retained
// index output), as for topk.hip.
#include "frag.hpp"
#include "select.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

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
  const float r0 = x0 - __uint_as_float(hi << 16), r1 = x1 - __uint_as_float(hi & 0xffff0000u);
  bf16x2_t m = {static_cast<__bf16>(r0), static_cast<__bf16>(r1)};
  mid = __builtin_bit_cast(uint32_t, m);
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
  __device__ __forceinline__ static float row_norm2(float part) {
    return part + __shfl_xor(part, 16);
  }
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
  __device__ __forceinline__ static float row_norm2(float part) {
    part += __shfl_xor(part, 16);
    return part + __shfl_xor(part, 32);
  }
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
  for (int v0 = threadIdx.x; v0 < total; v0 += U * blockDim.x) {
    f32x4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * blockDim.x, row = v / VPR, cv = v - row * VPR;
      x[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (v < total && row < rows)
        x[u] = *reinterpret_cast<const f32x4*>(src + static_cast<size_t>(row) * D + 4 * cv);
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
      float n2 = x[u][0] * x[u][0] + x[u][1] * x[u][1] + x[u][2] * x[u][2] + x[u][3] * x[u][3];
#pragma unroll
      for (int o = 1; o < VPR; o <<= 1) n2 += __shfl_xor(n2, o);
      mx = fmaxf(mx, n2);
    }
  }
  return mx;
}

// ---------------------------------------------------------------------------
// bf16 inputs: plain bf16 rows, one product per score
// ---------------------------------------------------------------------------

// Sum of squares of eight packed bf16 values.
__device__ __forceinline__ float sumsq_bf16x8(const uint32_t (&w)[4]) {
  float n2 = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = __uint_as_float(w[e] << 16), hi = __uint_as_float(w[e] & 0xffff0000u);
    n2 = fmaf(lo, lo, n2);
    n2 = fmaf(hi, hi, n2);
  }
  return n2;
}

// The score fragment of topk_small_kernel's bf16 path, with the query left
// unscaled (filter scores are compared unscaled) and |q|^2 for the bound.
template <int D>
struct Bf16FilterFrag : Frag<bf16, D> {
  using Base = Frag<bf16, D>;
  // Returns the sum of squares of the elements this lane loaded; the four
  // lane groups together hold the whole row.
  __device__ __forceinline__ float load_q(const bf16* qrow, int grp) {
    Base::load_q(qrow, grp, 1.f);
    if constexpr (D == 16) {
      float n2 = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = __uint_as_float(static_cast<uint32_t>(static_cast<uint16_t>(this->q[i])) << 16);
        n2 = fmaf(x, x, n2);
      }
      return n2;
    } else {
      float n2 = 0.f;
#pragma unroll
      for (int h = 0; h < Base::NI; ++h) {
        const auto w = __builtin_bit_cast(uint4, this->q[h]);
        const uint32_t a[4] = {w.x, w.y, w.z, w.w};
        n2 += sumsq_bf16x8(a);
      }
      return n2;
    }
  }
  __device__ __forceinline__ static float row_norm2(float part) {
    part += __shfl_xor(part, 16);
    return part + __shfl_xor(part, 32);
  }
};

// Stage `rows` bf16 key rows (zero rows up to rows_pad, a multiple of 64)
// with row stride LDK and return this thread's max squared row norm.
template <int D, int LDK>
__device__ __forceinline__ float stage_bf16_norm(bf16* lds, const bf16* src, int rows, int rows_pad) {
  constexpr int VPR = D / 8;  // 16-byte vectors per row; VPR consecutive threads share a row
  constexpr int U = kStageBatch;
  const char* base = reinterpret_cast<const char*>(src);
  const int total = rows_pad * VPR;  // a multiple of 64: whole wavefronts agree on v < total
  const int avail = rows * VPR;
  float mx = 0.f;
  for (int v0 = threadIdx.x; v0 < total; v0 += U * blockDim.x) {
    uint4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * blockDim.x;
      x[u] = make_uint4(0u, 0u, 0u, 0u);
      if (v < avail) x[u] = *reinterpret_cast<const uint4*>(base + static_cast<uint32_t>(v) * 16u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * blockDim.x, row = v / VPR, cv = v - row * VPR;
      if (v >= total) break;
      *reinterpret_cast<uint4*>(lds + row * LDK + cv * 8) = x[u];
      const uint32_t w[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
      float n2 = sumsq_bf16x8(w);
#pragma unroll
      for (int o = 1; o < VPR; o <<= 1) n2 += __shfl_xor(n2, o);
      mx = fmaxf(mx, n2);
    }
  }
  return mx;
}

// Per input type: the filter fragment, the LDS key row and its staging.
template <typename T, int D>
struct FilterIn;

template <int D>
struct FilterIn<float, D> {
  using SF = SplitFrag<D>;
  static constexpr int LDK = SF::LDK;
  __device__ __forceinline__ static float stage(bf16* lds, const float* src, int rows, int rows_pad,
                                                bool& exact) {
    return stage_split<D>(lds, src, rows, rows_pad, exact);
  }
  // E elements of a staged row, from element e0, rebuilt as fp32
  template <int E>
  __device__ __forceinline__ static void row_f32(float (&dst)[E], const bf16* r, int e0) {
#pragma unroll
    for (int e = 0; e < E; ++e)
      dst[e] = (bf16_to_f32(r[SF::OFF_H + e0 + e]) + bf16_to_f32(r[SF::OFF_M + e0 + e])) +
               bf16_to_f32(r[SF::OFF_L + e0 + e]);
  }
};

template <int D>
struct FilterIn<bf16, D> {
  using SF = Bf16FilterFrag<D>;
  static constexpr int LDK = SF::LDK;
  __device__ __forceinline__ static float stage(bf16* lds, const bf16* src, int rows, int rows_pad,
                                                bool&) {
    return stage_bf16_norm<D, LDK>(lds, src, rows, rows_pad);
  }
  template <int E>
  __device__ __forceinline__ static void row_f32(float (&dst)[E], const bf16* r, int e0) {
    ld_bf16<E>(dst, r + e0);
  }
};

// ---------------------------------------------------------------------------
// exact fp32 pass for one query tile (fallback)
// ---------------------------------------------------------------------------

// The tile's exact top-k lists (merged over the four lanes of each query), in
// the canonical fp32 order (fp32 MFMA on the inputs converted to fp32).
// from_lds (wave-uniform): key rows are rebuilt from the rows resident in LDS
// (all N keys, each rebuilt exactly); otherwise they come from global memory.
template <typename T, int D, int K>
__device__ __forceinline__ void exact_tile(const T* __restrict__ Qb, const T* __restrict__ Kb,
                                           const bf16* Ks, bool from_lds, int N, int qbase,
                                           float scale, int lane, float (&val)[K], int (&ix)[K]) {
  using F = Frag<float, D>;
  constexpr bool POW2 = pow2_scale<D>();
  constexpr int E = F::E;
  constexpr int LDK = FilterIn<T, D>::LDK;
  const int col = lane & 15, grp = lane >> 4;
  const int self = qbase + col;
  F frag;
  ld_row<T, E>(frag.q, Qb + static_cast<size_t>(min(self, N - 1)) * D + grp * E);
  if constexpr (POW2) {
#pragma unroll
    for (int t = 0; t < E; ++t) frag.q[t] *= scale;
  }
#pragma unroll
  for (int m = 0; m < K; ++m) { val[m] = -INFINITY; ix[m] = kIdxSentinel; }
  for (int kb = 0; kb < N; kb += 16) {
    typename F::KF kf;
    if (from_lds) {
      // rows [N, 16 * ceil(N / 16)) are staged zero rows
      FilterIn<T, D>::template row_f32<E>(kf.v, Ks + (kb + col) * LDK, grp * E);
    } else {
      ld_row<T, E>(kf.v, Kb + static_cast<size_t>(min(kb + col, N - 1)) * D + grp * E);
    }
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < F::NI; ++i) s = frag.step(kf, i, s);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = kb + 4 * grp + r;
      float v = POW2 ? s[r] : s[r] * scale;
      if (key >= N || key == self) v = -INFINITY;
      topk_insert<K>(val, ix, v, key);
    }
  }
#pragma unroll
  for (int step = 16; step <= 32; step <<= 1) {
    float pv[K];
    int pi[K];
#pragma unroll
    for (int m = 0; m < K; ++m) {
      pv[m] = __shfl_xor(val[m], step);
      pi[m] = __shfl_xor(ix[m], step);
    }
#pragma unroll
    for (int m = 0; m < K; ++m) topk_insert_lex<K>(val, ix, pv[m], pi[m]);
  }
}

// Canonical fp32 score of one (query row, key row) pair: fmaf chain with
// element kk*(D/4)+t at step t, slot kk (the MFMA chain's order), then scaled.
template <typename T, int D, bool POW2>
// Four steps at a time (4-element runs of each quarter row), so at most 32
// elements are live instead of both whole rows.
__device__ __forceinline__ float canon_pair(const T* qrow, const T* krow, float scale) {
  constexpr int QD = D / 4;
  float acc = 0.f;
#pragma unroll
  for (int t0 = 0; t0 < QD; t0 += 4) {
    float q[4][4], k[4][4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      ld_row<T, 4>(q[kk], qrow + kk * QD + t0);
      ld_row<T, 4>(k[kk], krow + kk * QD + t0);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc = fmaf(POW2 ? q[kk][t] * scale : q[kk][t], k[kk][t], acc);
  }
  return POW2 ? acc : acc * scale;
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------

// Slack of the filter proof, relative to |q| max_j |k_j|: at least the
// filter's error (2^-21) plus the canonical chain's (d 2^-24), with margin
// for the fp32 arithmetic of the bound itself.
template <int D>
constexpr float filter_eps() {
  return D <= 32 ? 1.0f / 262144.0f : 1.0f / 131072.0f;  // 2^-18, 2^-17
}

// Waves per workgroup: every wave of a workgroup shares one staged key chunk,
// so larger groups stage each batch row's keys fewer times and amortise the
// LDS copy over more queries.
constexpr int kFilterMaxWaves = 8;
// 16-key tiles per selection block (the unit of masking and packing)
constexpr int kFilterBlockTiles = 4;

// Packed candidates (pack8, select.hpp): during the scan a lane's filter
// score carries the key's position u = 4 * tile + r within the current
// 1024-key segment (the lane sees keys seg + 16 * tile + 4 * grp + r,
// tile < 64, r < 4).
constexpr int kSegKeys = 1024;
constexpr float kNormLimit = 1.329228e36f;   // 2^120: |q| max|k| at or above fails the proof

// Largest value whose truncation (bits `mask` cleared) is at most trunc(t).
__device__ __forceinline__ float trunc_ceiling(float t, uint32_t mask) {
  const uint32_t b = __float_as_uint(t) & ~mask;
  return __uint_as_float((b & 0x80000000u) ? b : (b | mask));
}

// Decode a lane's packed segment list into (truncated score, key) pairs, fold
// them into its running list and restart the segment list. lane_base is the
// segment's first key plus 4 * grp. The running list stays in (score desc,
// key asc) order, so the four lanes of a query merge to identical lists even
// where truncated scores tie.
template <int QT, int L>
__device__ __forceinline__ void flush_segment(float (&pv)[QT][L], float (&rv)[QT][L],
                                              int (&ri)[QT][L], int lane_base) {
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int m = 0; m < L; ++m) {
      const uint32_t bits = __float_as_uint(pv[qt][m]);
      const int u = static_cast<int>(bits & kLow8);
      topk_insert_lex<L>(rv[qt], ri[qt], __uint_as_float(bits & ~kLow8),
                         lane_base + 16 * (u >> 2) + (u & 3));
      pv[qt][m] = kMasked;
    }
}

// ONESEG: one chunk of at most one segment holds every key (kc >= N, N <= 1024),
// so the lists stay packed until the merge.
// Waves per SIMD the register budget is sized for: 5 (96 VGPRs); at d = 64
// the key and query fragments alone need more, so 4 (128 VGPRs) there.
template <int D>
constexpr int filter_min_waves() {
  return D == 64 ? 4 : 5;
}

template <typename T, int D, int K, int QT, bool ONESEG>
__global__ void __launch_bounds__(kFilterMaxWaves * 64, filter_min_waves<D>())
topk_filter_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
                   T* __restrict__ O, int32_t* __restrict__ Idx, int N, int n_qblk, int kc,
                   float scale, int nblocks) {
  using FI = FilterIn<T, D>;
  using SF = typename FI::SF;
  constexpr int LDK = FI::LDK;
  constexpr int EO = D / 4;
  constexpr int BT = kFilterBlockTiles;
  constexpr int C = K + 1;  // candidates rescored exactly
  constexpr int L = K + 2;  // list length: the candidates and the (k+2)-th
  constexpr bool POW2 = pow2_scale<D>();
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16* Ks = reinterpret_cast<bf16*>(smem_raw + 16);
  unsigned* kmax_slot = reinterpret_cast<unsigned*>(smem_raw);      // max |k|^2 of the chunk
  unsigned* inexact_slot = kmax_slot + 1;  // some staged element is not rebuilt exactly

  const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qblk = blk - b * n_qblk;
  const int q0 = (qblk * nw + wave) * 16 * QT;  // wave-uniform
  const int col = lane & 15, grp = lane >> 4;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const T* Qb = Q + boff;
  const T* Kb = Kx + boff;

  SF frag[QT];
  int self[QT];
  float qn2[QT];  // |q|^2 of this lane's query
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    self[qt] = q0 + 16 * qt + col;
    qn2[qt] = SF::row_norm2(frag[qt].load_q(Qb + static_cast<size_t>(min(self[qt], N - 1)) * D, grp));
  }
  bool self_r[4];  // element r of a diagonal tile is this lane's self pair
#pragma unroll
  for (int r = 0; r < 4; ++r) self_r[r] = (4 * grp + r == col);

  float pv[QT][L];  // packed scores of the current segment
  float rv[QT][L];  // finished segments: truncated scores ...
  int ri[QT][L];    // ... and their keys
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int m = 0; m < L; ++m) {
      pv[qt][m] = kMasked;
      rv[qt][m] = kMasked;
      ri[qt][m] = kIdxSentinel;
    }
  float kmax2 = 0.f;

  for (int c0 = 0; c0 < N; c0 += kc) {
    const int cn = min(kc, N - c0);
    const int cnb = (cn + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
    __syncthreads();
    if (threadIdx.x == 0) {
      *kmax_slot = 0u;
      *inexact_slot = 0u;
    }
    bool exact = true;
    const float mine = FI::stage(Ks, Kb + static_cast<size_t>(c0) * D, cn, cnb, exact);
    if (!exact) atomicOr(inexact_slot, 1u);
    __syncthreads();
    atomicMax(kmax_slot, __float_as_uint(mine));  // non-negative: bit order is value order
    if (q0 < N) {
      const int kend = c0 + cn;
      for (int kb0 = 0; kb0 < cnb; kb0 += 16 * BT) {
        const int kabs = c0 + kb0;
        f32x4 s[QT][BT];
#pragma unroll
        for (int t = 0; t < BT; ++t) {
          const typename SF::KF kf = SF::load_k(Ks + (kb0 + 16 * t + col) * LDK, grp);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) s[qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < SF::NI; ++i)
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) s[qt][t] = frag[qt].step(kf, i, s[qt][t]);
        }
        // raw (unscaled) filter scores: scaling does not change the order
        const uint32_t u0 = static_cast<uint32_t>(kb0 & (kSegKeys - 1)) >> 2;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
          for (int t = 0; t < BT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) s[qt][t][r] = pack8(s[qt][t][r], u0 + 4 * t + r);
        mask_block<QT, BT>(s, self_r, q0, kabs, kend, grp, kMasked);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
          for (int t = 0; t < BT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) vinsert<L>(pv[qt], s[qt][t][r]);
        const int next = kb0 + 16 * BT;
        if (!ONESEG && ((next & (kSegKeys - 1)) == 0 || next >= cnb))
          flush_segment<QT, L>(pv, rv, ri, c0 + (kb0 & ~(kSegKeys - 1)) + 4 * grp);
      }
    }
    __syncthreads();
    kmax2 = fmaxf(kmax2, __uint_as_float(*kmax_slot));
  }
  if (q0 >= N) return;
  // the exact fallback may rebuild keys from LDS: one chunk holds them all
  const bool lds_exact = ONESEG && *inexact_slot == 0u;

  // ---- merge the four lane lists of each query ---------------------------
  // cand: the k+1 candidates (identical on the four lanes of a query;
  // -1 for a masked entry); ceil_f: no other key's filter score exceeds it.
  int cand[QT][C];
  float ceil_f[QT];
  if constexpr (ONESEG) {
    const uint32_t mmask = N <= 256 ? kLow8 : kLow10;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      // repack with the lane group (low bits = 4 * u + grp; u < 64 fits 8 bits
      // when N <= 256) and re-sort: entries equal above those bits may change order
      float p[L];
#pragma unroll
      for (int m = 0; m < L; ++m) p[m] = kMasked;
#pragma unroll
      for (int m = 0; m < L; ++m) {
        const uint32_t bits = __float_as_uint(pv[qt][m]);
        vinsert<L>(p, __uint_as_float((bits & ~mmask) | ((bits & kLow8) << 2) |
                                      static_cast<uint32_t>(grp)));
      }
#pragma unroll
      for (int step = 16; step <= 32; step <<= 1) {
        float o[L];
#pragma unroll
        for (int m = 0; m < L; ++m) o[m] = __shfl_xor(p[m], step);
#pragma unroll
        for (int m = 0; m < L; ++m) vinsert<L>(p, o[m]);
      }
#pragma unroll
      for (int m = 0; m < C; ++m) {
        const int w = static_cast<int>(__float_as_uint(p[m]) & mmask), u = w >> 2;
        cand[qt][m] = p[m] < kMaskedBelow ? -1 : 16 * (u >> 2) + 4 * (w & 3) + (u & 3);
      }
      ceil_f[qt] = trunc_ceiling(p[C], mmask);
    }
  } else {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
      for (int step = 16; step <= 32; step <<= 1) {
        float ov[L];
        int oi[L];
#pragma unroll
        for (int m = 0; m < L; ++m) {
          ov[m] = __shfl_xor(rv[qt][m], step);
          oi[m] = __shfl_xor(ri[qt][m], step);
        }
#pragma unroll
        for (int m = 0; m < L; ++m) topk_insert_lex<L>(rv[qt], ri[qt], ov[m], oi[m]);
      }
#pragma unroll
      for (int m = 0; m < C; ++m) cand[qt][m] = rv[qt][m] < kMaskedBelow ? -1 : ri[qt][m];
      ceil_f[qt] = trunc_ceiling(rv[qt][C], kLow8);
    }
  }

  // ---- verify: rescore the candidates exactly ---------------------------
  const float kmax = sqrtf(kmax2);
  float val[QT][K];
  int ix[QT][K];
  bool ok[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = min(self[qt], N - 1);
    const T* qrow = Qb + static_cast<size_t>(qi) * D;
    // lane group g rescores candidates g, g+4, ...
    float mine[(C + 3) / 4];
#pragma unroll
    for (int u = 0; u < (C + 3) / 4; ++u) {
      const int m = 4 * u + grp;
      int c = -1;
#pragma unroll
      for (int mm = 0; mm < C; ++mm)
        if (mm == m) c = cand[qt][mm];
      const int row = min(max(c, 0), N - 1);
      const float e = canon_pair<T, D, POW2>(qrow, Kb + static_cast<size_t>(row) * D, scale);
      mine[u] = c < 0 ? -INFINITY : e;
    }
    // the exact top k of the candidates, in (score desc, index asc) order
    float cv[C];
#pragma unroll
    for (int m = 0; m < C; ++m) cv[m] = __shfl(mine[m / 4], col + 16 * (m % 4));
    sort_lex<C>(cv, cand[qt]);
#pragma unroll
    for (int m = 0; m < K; ++m) { val[qt][m] = cv[m]; ix[qt][m] = cand[qt][m]; }
    const float nprod = sqrtf(qn2[qt]) * kmax;
    const float bound = (ceil_f[qt] + filter_eps<D>() * nprod) * scale;
    ok[qt] = self[qt] >= N || (nprod < kNormLimit && bound < val[qt][K - 1]);
  }

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    if (!__all(ok[qt]))
      exact_tile<T, D, K>(Qb, Kb, Ks, lds_exact, N, q0 + 16 * qt, scale, lane, val[qt], ix[qt]);
  }

  // ---- k-softmax and gathered aggregation --------------------------------
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = self[qt];
    if (qi >= N) continue;
    const float mx = val[qt][0];
    float acc[EO];
#pragma unroll
    for (int c = 0; c < EO; ++c) acc[c] = 0.f;
    float den = 0.f;
#pragma unroll
    for (int m = 0; m < K; ++m) {
      const float w = fast_exp2((val[qt][m] - mx) * kLog2eF);
      den += w;
      const int row = min(max(ix[qt][m], 0), N - 1);
      float vr[EO];
      ld_row<T, EO>(vr, V + boff + static_cast<size_t>(row) * D + grp * EO);
#pragma unroll
      for (int c = 0; c < EO; ++c) acc[c] = fmaf(w, vr[c], acc[c]);
    }
    const float inv = 1.f / den;
#pragma unroll
    for (int c = 0; c < EO; ++c) acc[c] *= inv;
    st_row<T, EO>(O + boff + static_cast<size_t>(qi) * D + grp * EO, acc);
    if (Idx != nullptr && grp == 0) {
      int32_t* dst = Idx + (static_cast<size_t>(b) * N + qi) * K;
#pragma unroll
      for (int m = 0; m < K; ++m) dst[m] = ix[qt][m];
    }
  }
}

size_t topk_filter_lds_bytes(int dtype, int d, int kc) {
  const int kcb = (kc + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
  const int row = dtype == kF32 ? 3 * d + 8 : d + 8;  // bf16 elements per staged key row
  return 16 + static_cast<size_t>(kcb) * row * sizeof(bf16);
}

template <typename T, int D>
static hipError_t launch_filter(const TopkArgs& a, int kc) {
  constexpr int QT = kTopkQueryTiles;
  const int per_wave = 16 * QT;
  const int waves = (a.N + per_wave - 1) / per_wave;
  // up to N = 256 the 28 KiB key copy is small: four-wave groups keep five
  // groups (20 waves) resident per CU; larger rows share one copy among eight
  // waves, unless that leaves fewer than two workgroups per CU (small batches:
  // B = 32, N = 512 runs 1.4x slower with eight-wave groups)
  const long wide_groups = static_cast<long>(a.B) * ((a.N + 16 * QT * kFilterMaxWaves - 1) /
                                                     (16 * QT * kFilterMaxWaves));
  const int maxw = (a.N <= 256 || wide_groups < 2L * kCUs) ? 4 : kFilterMaxWaves;
  const int nw = waves >= maxw ? maxw : waves;
  const int qb = per_wave * nw;
  const int n_qblk = (a.N + qb - 1) / qb;
  const int nblocks = a.B * n_qblk;
  const size_t lds = topk_filter_lds_bytes(a.dtype, D, kc);
  const T* q = static_cast<const T*>(a.q);
  const T* k = static_cast<const T*>(a.k);
  const T* v = static_cast<const T*>(a.v);
  T* o = static_cast<T*>(a.out);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  const bool oneseg = kc >= a.N && a.N <= kSegKeys;
#define TARMAC_FILTER_CASE(KK)                                                                    \
  case KK:                                                                                        \
    if (oneseg)                                                                                   \
      hipLaunchKernelGGL((topk_filter_kernel<T, D, KK, QT, true>), dim3(nblocks), dim3(64 * nw),  \
                         lds, st, q, k, v, o, a.idx, a.N, n_qblk, kc, a.scale, nblocks);         \
    else                                                                                          \
      hipLaunchKernelGGL((topk_filter_kernel<T, D, KK, QT, false>), dim3(nblocks), dim3(64 * nw), \
                         lds, st, q, k, v, o, a.idx, a.N, n_qblk, kc, a.scale, nblocks);         \
    break;
  switch (a.topk) {
    TARMAC_FILTER_CASE(1)
    TARMAC_FILTER_CASE(2)
    TARMAC_FILTER_CASE(3)
    TARMAC_FILTER_CASE(4)
    TARMAC_FILTER_CASE(5)
    TARMAC_FILTER_CASE(6)
    TARMAC_FILTER_CASE(7)
    TARMAC_FILTER_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef TARMAC_FILTER_CASE
  return hipGetLastError();
}

// fp32: d = 16, 32, 64. bf16: d = 16 only, where one bf16 product per score
// makes the scan cheap (at d = 32 and 64 the plain bf16 pass is faster).
bool topk_filter_supported(int dtype, int d, int topk) {
  const bool shape = dtype == kF32 ? (d == 16 || d == 32 || d == 64) : (dtype == kBf16 && d == 16);
  return shape && topk >= 1 && topk <= kTopkSmallMax;
}

hipError_t run_topk_filter(const TopkArgs& a) {
  if (a.dtype == kBf16) return a.d == 16 ? launch_filter<bf16, 16>(a, a.key_chunk) : hipErrorInvalidValue;
  switch (a.d) {
    case 16: return launch_filter<float, 16>(a, a.key_chunk);
    case 32: return launch_filter<float, 32>(a, a.key_chunk);
    case 64: return launch_filter<float, 64>(a, a.key_chunk);
  }
  return hipErrorInvalidValue;
}

}  // namespace tarmac
