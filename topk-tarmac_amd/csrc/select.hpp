// Register top-k lists and block masking shared by the top-k kernels.
//
// A lane keeps its best K candidates as a list sorted by (score desc, index
// asc). Keys reach a lane in ascending index order, so a strict '>' insertion
// keeps the lower index ahead on equal scores; lists built from disjoint key
// sets are merged with a lexicographic comparison.
#pragma once

#include "frag.hpp"

namespace tarmac {

constexpr int kIdxSentinel = 0x3fffffff;

// max(a, b) as one v_med3_f32. The compiler's maxnum (fmaxf, or fmed3
// against a literal +inf, which it folds to maxnum) first canonicalises every
// operand it cannot prove canonical: one extra instruction per score here.
// Inputs are never NaN.
__device__ __forceinline__ float vmax(float a, float b) {
  return __builtin_amdgcn_fmed3f(a, b, opaque_inf());
}

// min(a, b) as one v_med3_f32 against an opaque -inf (see vmax).
__device__ __forceinline__ float vmin(float a, float b) {
  return __builtin_amdgcn_fmed3f(a, b, -opaque_inf());
}

template <int K>
__device__ __forceinline__ void topk_insert(float (&val)[K], int (&ix)[K], float s, int j) {
  // New keys arrive in ascending index order, so a strict '>' keeps the
  // earlier (lower-index) entry ahead on equal scores. Values move through
  // max / med3 (list order v[m-1] >= v[m]), indices through the compares.
  bool c[K];
#pragma unroll
  for (int m = 0; m < K; ++m) c[m] = s > val[m];
#pragma unroll
  for (int m = K - 1; m > 0; --m) {
    val[m] = __builtin_amdgcn_fmed3f(val[m - 1], val[m], s);
    ix[m] = c[m - 1] ? ix[m - 1] : (c[m] ? j : ix[m]);
  }
  val[0] = vmax(val[0], s);
  ix[0] = c[0] ? j : ix[0];
}

template <int K>
__device__ __forceinline__ void topk_insert_lex(float (&val)[K], int (&ix)[K], float s, int j) {
#pragma unroll
  for (int m = K - 1; m > 0; --m) {
    const bool cm = ranks_before(s, j, val[m], ix[m]);
    const bool cp = ranks_before(s, j, val[m - 1], ix[m - 1]);
    const float vm = val[m - 1];
    const int im = ix[m - 1];
    val[m] = cp ? vm : (cm ? s : val[m]);
    ix[m] = cp ? im : (cm ? j : ix[m]);
  }
  const bool c0 = ranks_before(s, j, val[0], ix[0]);
  val[0] = c0 ? s : val[0];
  ix[0] = c0 ? j : ix[0];
}

// Sort n (value, index) pairs by (value desc, index asc): odd-even
// transposition network, n rounds of compare-exchange.
template <int n>
__device__ __forceinline__ void sort_lex(float (&v)[n], int (&ix)[n]) {
#pragma unroll
  for (int round = 0; round < n; ++round)
#pragma unroll
    for (int a = round & 1; a + 1 < n; a += 2) {
      const bool sw = ranks_before(v[a + 1], ix[a + 1], v[a], ix[a]);
      const float va = v[a];
      const int ia = ix[a];
      v[a] = sw ? v[a + 1] : va;
      ix[a] = sw ? ix[a + 1] : ia;
      v[a + 1] = sw ? va : v[a + 1];
      ix[a + 1] = sw ? ia : ix[a + 1];
    }
}

constexpr int kBlockTiles = 4;               // 16-key tiles per selection block
constexpr int kBlockKeys = 16 * kBlockTiles;

// Set the self pair and keys at or past kend to `masked`. q0 and kabs are
// wave-uniform, so both tests are scalar branches and only the diagonal and
// ragged blocks pay for the per-element selects. In the 16-key tile holding
// a query tile's diagonal, lane l's element r is the self pair exactly when
// 4*(l/16) + r == l % 16 (the loop-invariant lane predicate self_r[r]).
template <int QT, int BT>
__device__ __forceinline__ void mask_block(f32x4 (&s)[QT][BT], const bool (&self_r)[4], int q0,
                                           int kabs, int kend, int grp, float masked) {
  if (q0 < kabs + 16 * BT && kabs < q0 + 16 * QT) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int t = 0; t < BT; ++t) {
        const bool diag_tile = (q0 + 16 * qt == kabs + 16 * t);  // uniform
#pragma unroll
        for (int r = 0; r < 4; ++r)
          s[qt][t][r] = (diag_tile && self_r[r]) ? masked : s[qt][t][r];
      }
  }
  if (kabs + 16 * BT > kend) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int t = 0; t < BT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kabs + 16 * t + 4 * grp + r >= kend) s[qt][t][r] = masked;
  }
}

// Packed candidates. A score keeps its top 24 bits and carries, in the low 8
// mantissa bits, the key's position u within the lane's stream (u < 256).
// Clearing low bits rounds toward zero, a monotone map, so packed order
// refines the order of the truncated scores and distinct keys give distinct
// packed values: a scan keeps values only (max / med3) and the key comes back
// from the bits.
constexpr uint32_t kLow8 = 0xffu, kLow10 = 0x3ffu;
constexpr float kMasked = -3.40282347e38f;   // -FLT_MAX: stays finite when packed
constexpr float kMaskedBelow = -1.0e38f;     // list entries below this are masked keys

// Bits 8..31 from s, bits 0..7 from u (< 256): one v_perm_b32 (the compiler
// turns the and/or form into two instructions).
__device__ __forceinline__ float pack8(float s, uint32_t u) {
  return __uint_as_float(__builtin_amdgcn_perm(__float_as_uint(s), u, 0x07060500u));
}

// Score s with its low bits (mask m) replaced by field f (f <= m): one
// v_and_or_b32 (with m in a VGPR and f in an SGPR).
__device__ __forceinline__ float pack_field(float s, uint32_t f, uint32_t m) {
  return __uint_as_float((__float_as_uint(s) & ~m) | f);
}

// A wave-uniform value in an SGPR the compiler cannot fold into the
// instructions that read it (a scalar copy).
__device__ __forceinline__ uint32_t opaque_sgpr(uint32_t x) {
  uint32_t r;
  asm("s_mov_b32 %0, %1" : "=s"(r) : "s"(x));
  return r;
}

// The same with the complement of the mask in a VGPR (notm = ~m) and a
// wave-uniform field f: one v_and_or_b32 reading f from an SGPR. With f
// visible the compiler forms it on the VALU instead (an and, then an or3
// with the element's offset: two operations per score).
__device__ __forceinline__ float pack_field_u(float s, uint32_t f, uint32_t notm) {
  return __uint_as_float((__float_as_uint(s) & notm) | opaque_sgpr(f));
}

// Value-only insertion into a descending list: L max/med3 operations.
template <int L>
__device__ __forceinline__ void vinsert(float (&v)[L], float s) {
#pragma unroll
  for (int m = L - 1; m > 0; --m) v[m] = __builtin_amdgcn_fmed3f(v[m - 1], v[m], s);
  v[0] = vmax(v[0], s);
}

// Scale (non power-of-two 1/sqrt(d)) and mask one block's scores: the self
// pair and keys past the chunk end. Branches are wave-uniform. In the 16-key
// tile holding a query tile's diagonal, lane l's element r is the self pair
// exactly when 4*(l/16) + r == l % 16 (the loop-invariant lane predicate
// self_r[r]), so the self mask is one select per element of that block.
template <int QT, int BT, bool POW2>
__device__ __forceinline__ void prepare_block(f32x4 (&s)[QT][BT], float scale,
                                              const bool (&self_r)[4], int q0, int kabs, int kend,
                                              int grp) {
  if constexpr (!POW2) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int t = 0; t < BT; ++t) s[qt][t] *= scale;
  }
  mask_block<QT, BT>(s, self_r, q0, kabs, kend, grp, -INFINITY);
}

template <int QT, int K>
__device__ __forceinline__ void rebase_list(int (&ix)[QT][K], int delta) {
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int m = 0; m < K; ++m) ix[qt][m] -= delta;
}


// As topk_insert, plus the value (no index) of the (K+1)-th best in val[K]:
// values move through max / med3, indices through the compares.
template <int K>
__device__ __forceinline__ void topk_insert_x(float (&val)[K + 1], int (&ix)[K], float s, int j) {
  bool c[K];
#pragma unroll
  for (int m = 0; m < K; ++m) c[m] = s > val[m];
  val[K] = __builtin_amdgcn_fmed3f(val[K - 1], val[K], s);
#pragma unroll
  for (int m = K - 1; m > 0; --m) {
    val[m] = __builtin_amdgcn_fmed3f(val[m - 1], val[m], s);
    ix[m] = c[m - 1] ? ix[m - 1] : (c[m] ? j : ix[m]);
  }
  val[0] = vmax(val[0], s);
  ix[0] = c[0] ? j : ix[0];
}

// Lexicographic insertion into a (K+1)-list whose last slot carries only a
// value. Entries with index kIdxSentinel lose every tie.
template <int K>
__device__ __forceinline__ void topk_insert_lex_x(float (&val)[K + 1], int (&ix)[K], float s, int j) {
  // slot K (value only): the (K+1)-th best of the union
  const bool ck = ranks_before(s, j, val[K - 1], ix[K - 1]);
  val[K] = ck ? val[K - 1] : vmax(val[K], s);
#pragma unroll
  for (int m = K - 1; m > 0; --m) {
    const bool cm = ranks_before(s, j, val[m], ix[m]);
    const bool cp = ranks_before(s, j, val[m - 1], ix[m - 1]);
    const float vm = val[m - 1];
    const int im = ix[m - 1];
    val[m] = cp ? vm : (cm ? s : val[m]);
    ix[m] = cp ? im : (cm ? j : ix[m]);
  }
  const bool c0 = ranks_before(s, j, val[0], ix[0]);
  val[0] = c0 ? s : val[0];
  ix[0] = c0 ? j : ix[0];
}

}  // namespace tarmac
