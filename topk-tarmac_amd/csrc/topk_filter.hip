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
//     |a - q.k| < 2^-19.9 sum_c |q_c k_c| (three dropped products of
//     <= 2^-24 each; the bf16 MFMA accumulation, measured at most 2^-20.25
//     of the term magnitudes). bf16 inputs:
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
//  3. fallback: an unproven query is recomputed exactly by the whole wave
//     (exact_query_topk_lanes: its row's canonical scores on the VALU, one
//     key row per lane, per-lane lists, a six-step merge), so the result
//     never depends on the filter -- only the time does.
//
// Reference behaviour: src/kernels/fused_topk_attention.py:211-333 and
// src/kernels/streaming_topk_attention.py:66-258 (including the retained
// index output), as for topk.hip.
#include "exact.hpp"
#include "frag.hpp"
#include "select.hpp"
#include "split.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

// ---------------------------------------------------------------------------
// bf16 inputs: plain bf16 rows, one product per score
// ---------------------------------------------------------------------------

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
  __device__ __forceinline__ static float row_norm2(float part) { return add_xor32(add_xor16(part)); }
};

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
// the kernel
// ---------------------------------------------------------------------------

// Slack of the filter proof, relative to |q| max_j |k_j|: at least the
// filter's error (< 2^-19.9) plus the canonical chain's (d 2^-24), with
// margin for the fp32 arithmetic of the bound itself.
template <int D>
constexpr float filter_eps() {
  static_assert(D <= 64, "the filter serves d <= 64");
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
    if (threadIdx.x == 0) *kmax_slot = 0u;
    bool exact = true;  // (whether the LDS rows rebuild the inputs exactly: not needed here)
    const float mine = FI::stage(Ks, Kb + static_cast<size_t>(c0) * D, cn, cnb, exact);
    // one LDS atomic per wave (a per-lane atomic compiles to a 64-step
    // readlane loop); non-negative floats order like their bits
    const float wmax = wave_max_rows(mine);
    __syncthreads();
    if (lane == 0) atomicMax(kmax_slot, __float_as_uint(wmax));
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
    const float nprod = proof_norm(qn2[qt], kmax2);
    const float bound = (ceil_f[qt] + filter_eps<D>() * nprod) * scale;
    ok[qt] = self[qt] >= N || (nprod < kNormLimit && bound < val[qt][K - 1]);
  }

  // unproven queries: recomputed exactly one at a time across the whole wave
  // (the tile's proven queries keep their sets)
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    unsigned long long todo = __ballot(grp == 0 && !ok[qt]);
    while (todo != 0ull) {
      const int c = __builtin_ctzll(todo);
      todo &= todo - 1ull;
      float ev[K];
      int ei[K];
      const int qi = q0 + 16 * qt + c;
      exact_query_topk_lanes<T, D, K, QT == 1 ? exact_wide_rows<T, D>() : 1>(
          Qb + static_cast<size_t>(qi) * D, [&](int j) { return Kb + static_cast<size_t>(j) * D; }, N,
          qi, scale, lane, ev, ei);
      if (col == c) {
#pragma unroll
        for (int m = 0; m < K; ++m) { val[qt][m] = ev[m]; ix[qt][m] = ei[m]; }
      }
    }
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

template <typename T, int D, int QT>
static hipError_t launch_filter_q(const TopkArgs& a, int kc) {
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

// bf16 batches too small to give every SIMD a wave at two query tiles per
// wave (B * N / 32 below 4 * kCUs) take one tile per wave: twice the waves.
template <typename T, int D>
static hipError_t launch_filter(const TopkArgs& a, int kc) {
  if constexpr (sizeof(T) == 2) {
    if (one_query_tile(a.B, a.N)) return launch_filter_q<T, D, 1>(a, kc);
  }
  return launch_filter_q<T, D, kTopkQueryTiles>(a, kc);
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
