// Score-then-select top-k attention, fused: scores, selection, k-softmax and
// the gathered aggregation in one launch; no score row, index tensor or
// gathered value tensor reaches HBM.
//
// Reference behaviour: src/kernels/fused_topk_attention.py:211-333
// (fused_topk_attention_tiled) and src/kernels/streaming_topk_attention.py:
// 66-258 (streaming_topk_attention, incl. the optional retained-index output).
//
// Small k (1..8), one launch shape for both the resident and the streamed
// variants:
//   * workgroup = (batch row b, block of 16*nw queries), nw waves;
//   * keys are staged through LDS in chunks of `kc` rows (kc >= N: the whole
//     K[b] is resident; otherwise the chunks stream);
//   * each wave forms 16x16 S^T tiles with MFMA; lane l owns query l%16 and,
//     per tile, the 4 keys 4*(l/16)+r, so the four lanes l, l^16, l^32, l^48
//     see disjoint interleaved key subsets of one query, each in ascending key
//     order;
//   * every lane keeps a sorted (score desc, index asc) list of its best k in
//     registers; strict '>' insertion keeps the lower index on ties;
//   * two xor-shuffle merge steps (16, 32) combine the four lists, after which
//     the 4 lanes of a query each compute d/4 output channels from the k
//     gathered V rows.
//
// Large k (> 8): one wave per query, the score row in LDS, an exact threshold
// found by bisection on the order-preserving integer key, ties at the
// threshold resolved to the lowest indices.
#include "frag.hpp"
#include "select.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

template <typename T, int D, int K, int QT>
__global__ void __launch_bounds__(256)
topk_small_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
                  T* __restrict__ O, int32_t* __restrict__ Idx, int N, int n_qblk, int kc,
                  float scale, int nblocks) {
  using F = Frag<T, D>;
  constexpr int LDK = F::LDK;
  constexpr int EO = D / 4;  // output channels per lane
  constexpr int BT = kBlockTiles;
  constexpr bool POW2 = pow2_scale<D>();
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* Ks = reinterpret_cast<T*>(smem_raw);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qblk = blk - b * n_qblk;
  const int q0 = (qblk * nw + wave) * 16 * QT;  // first query of this wave
  const int col = lane & 15, grp = lane >> 4;
  const size_t boff = static_cast<size_t>(b) * N * D;

  F frag[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = q0 + 16 * qt + col;
    frag[qt].load_q(Q + boff + static_cast<size_t>(min(qi, N - 1)) * D, grp,
                    POW2 ? scale : 1.f);
  }

  float val[QT][K];
  int ix[QT][K];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int m = 0; m < K; ++m) { val[qt][m] = -INFINITY; ix[qt][m] = kIdxSentinel; }

  bool self_r[4];  // element r of a diagonal tile is this lane's self pair
#pragma unroll
  for (int r = 0; r < 4; ++r) self_r[r] = (4 * grp + r == col);
  // Stored indices are kept relative to the base of the block being
  // selected, so a new candidate's index is the inline constant 16t+r; the
  // lane-group offset 4*(l/16) is added at the end.
  int base = 0;

  for (int c0 = 0; c0 < N; c0 += kc) {
    const int cn = min(kc, N - c0);
    const int cnb = (cn + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
    __syncthreads();
    stage_rows<T, D, LDK>(Ks, Kx + boff + static_cast<size_t>(c0) * D, cn, cnb);
    __syncthreads();
    if (q0 >= N) continue;
    const int kend = c0 + cn;  // rows past the chunk end are zero padding
    for (int kb0 = 0; kb0 < cnb; kb0 += kBlockKeys) {
      const int kabs = c0 + kb0;
      f32x4 s[QT][BT];
      block_scores<F, QT, BT>(frag, Ks, kb0, LDK, lane, s);
      prepare_block<QT, BT, POW2>(s, scale, self_r, q0, kabs, kend, grp);
      rebase_list<QT, K>(ix, kabs - base);
      base = kabs;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int t = 0; t < BT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) topk_insert<K>(val[qt], ix[qt], s[qt][t][r], 16 * t + r);
    }
  }
  rebase_list<QT, K>(ix, -base);  // back to absolute key indices
  if (q0 >= N) return;

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int m = 0; m < K; ++m) ix[qt][m] += 4 * grp;
#pragma unroll
    for (int step = 16; step <= 32; step <<= 1) {
      float pv[K];
      int pi[K];
#pragma unroll
      for (int m = 0; m < K; ++m) {
        pv[m] = __shfl_xor(val[qt][m], step);
        pi[m] = __shfl_xor(ix[qt][m], step);
      }
#pragma unroll
      for (int m = 0; m < K; ++m) topk_insert_lex<K>(val[qt], ix[qt], pv[m], pi[m]);
    }
  }

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = q0 + 16 * qt + col;
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

// ---------------------------------------------------------------------------
// large k: one wave per query row
// ---------------------------------------------------------------------------

__device__ __forceinline__ int ordered_key(float x) {
  // Monotone fp32 -> int32 (src/kernels/fused_topk_attention.py:113-124).
  const int i = __float_as_int(x);
  return i ^ ((i >> 31) & 0x7fffffff);
}

__device__ __forceinline__ int wave_sum(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

template <typename T, int D>
__device__ __forceinline__ float canon_score(const float (&q)[D], const T* krow) {
  // Same fmaf order as the MFMA chain: slot kk of step t holds c = kk*(D/4)+t.
  float kf[D];
  ld_row<T, D>(kf, krow);
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < D / 4; ++t)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = fmaf(q[kk * (D / 4) + t], kf[kk * (D / 4) + t], acc);
  return acc;
}

__device__ __forceinline__ int wave_min_int(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = min(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ int wave_max_int(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = max(x, __shfl_xor(x, o));
  return x;
}

// Selection rules of the wide kernel:
//   kSelTopk   exactly k, ties at the k-th score keep the lowest indices
//              (the standard rule, src/kernels/streaming_topk_attention.py:37-44);
//   kSelMasked every peer whose key is >= the threshold left by `bisect`
//              halvings of the reference's integer bisection
//              (src/kernels/fused_topk_attention.py:127-208): exact top-k plus
//              every peer tied at the k-th score once bisect >= 32;
//   kSelSort   exactly k, ties at the k-th score keep the highest indices (the
//              descending sort of key << 32 | index, :405-504).
// One wave per query row; the score row and the selected indices live in LDS
// (the selected list holds up to `cap` entries: k, or N for kSelMasked).
template <typename T, int D>
__global__ void __launch_bounds__(256)
topk_wide_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
                 T* __restrict__ O, int32_t* __restrict__ Idx, int B, int N, int topk, float scale,
                 int mode, int bisect, int cap) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const long row_raw = static_cast<long>(blockIdx.x) * nw + wave;  // (b, i) flattened
  const bool live = row_raw < static_cast<long>(B) * N;  // wave-uniform
  const long row = live ? row_raw : 0;
  const int b = static_cast<int>(row / N), i = static_cast<int>(row - static_cast<long>(b) * N);
  float* S = reinterpret_cast<float*>(smem_raw) + static_cast<size_t>(wave) * (N + cap);
  int* sel = reinterpret_cast<int*>(S + N);
  const size_t boff = static_cast<size_t>(b) * N * D;
  const bool pow2 = is_pow2_scale(scale);

  float q[D];
  ld_row<T, D>(q, Q + boff + static_cast<size_t>(i) * D);
  if (pow2) {
#pragma unroll
    for (int c = 0; c < D; ++c) q[c] *= scale;
  }
  for (int j = lane; j < N; j += kWave) {
    float s = canon_score<T, D>(q, Kx + boff + static_cast<size_t>(j) * D);
    if (!pow2) s *= scale;
    S[j] = (j == i) ? -INFINITY : s;
  }
  __syncthreads();

  int thr;
  if (mode == kSelMasked) {
    // the reference's bisection, step for step: lo starts at the smallest
    // valid key, hi at the row maximum; bisect halvings
    int kmin = 2147483647, kmx = -2147483647 - 1;
    for (int j = lane; j < N; j += kWave) {
      const int key = ordered_key(S[j]);
      kmx = max(kmx, key);
      if (j != i) kmin = min(kmin, key);
    }
    long lo = wave_min_int(kmin), hi = wave_max_int(kmx);
    for (int it = 0; it < bisect; ++it) {
      const long mid = lo + (hi - lo + 1) / 2;
      int cnt = 0;
      for (int j = lane; j < N; j += kWave) cnt += (ordered_key(S[j]) >= mid) ? 1 : 0;
      cnt = wave_sum(cnt);
      if (cnt >= topk) lo = mid; else hi = mid - 1;
    }
    thr = static_cast<int>(lo);
  } else {
    // largest t with count(key >= t) >= topk: the k-th largest key
    long lo = -2147483648L, hi = 2147483647L;
    while (lo < hi) {
      const long mid = lo + (hi - lo + 1) / 2;
      int cnt = 0;
      for (int j = lane; j < N; j += kWave) cnt += (ordered_key(S[j]) >= mid) ? 1 : 0;
      cnt = wave_sum(cnt);
      if (cnt >= topk) lo = mid; else hi = mid - 1;
    }
    thr = static_cast<int>(lo);
  }
  int gt = 0, eq = 0;
  for (int j = lane; j < N; j += kWave) {
    const int key = ordered_key(S[j]);
    gt += key > thr ? 1 : 0;
    eq += key == thr ? 1 : 0;
  }
  gt = wave_sum(gt);
  eq = wave_sum(eq);
  // ties at thr taken: all (masked), the first need_ties in index order
  // (topk) or the last need_ties (sort)
  const int need_ties = mode == kSelMasked ? eq : topk - gt;
  const int skip_ties = mode == kSelSort ? eq - need_ties : 0;

  // Compact the selected indices in ascending index order.
  int taken = 0, ties = 0;
  float mx = -INFINITY;
  for (int j0 = 0; j0 < N; j0 += kWave) {
    const int j = j0 + lane;
    const int key = (j < N) ? ordered_key(S[j]) : -2147483647 - 1;
    const bool is_tie = (j < N) && key == thr;
    const unsigned long long tie_mask = __ballot(is_tie);
    const int tie_rank = ties + __popcll(tie_mask & ((1ull << lane) - 1ull));
    const bool pick = (j < N) && (key > thr || (is_tie && tie_rank >= skip_ties &&
                                                 tie_rank < skip_ties + need_ties));
    const unsigned long long pick_mask = __ballot(pick);
    if (pick) {
      sel[taken + __popcll(pick_mask & ((1ull << lane) - 1ull))] = j;
      mx = fmaxf(mx, S[j]);
    }
    taken += __popcll(pick_mask);
    ties += __popcll(tie_mask);
  }
  mx = wave_max(mx);
  __syncthreads();
  if (!live) return;

  // Lane c < D accumulates channel c over the selected rows.
  if (lane < D) {
    float acc = 0.f, den = 0.f;
    for (int m = 0; m < taken; ++m) {
      const int j = sel[m];
      const float w = expf(S[j] - mx);
      den += w;
      const T* vr = V + boff + static_cast<size_t>(j) * D + lane;
      float x;
      if constexpr (sizeof(T) == 4) x = *reinterpret_cast<const float*>(vr);
      else x = bf16_to_f32(*reinterpret_cast<const bf16*>(vr));
      acc = fmaf(w, x, acc);
    }
    const float o = acc / den;
    T* dst = O + boff + static_cast<size_t>(i) * D + lane;
    if constexpr (sizeof(T) == 4) *reinterpret_cast<float*>(dst) = o;
    else *reinterpret_cast<bf16*>(dst) = f32_to_bf16(o);
  }
  if (Idx != nullptr) {  // never for kSelMasked (the set size varies)
    int32_t* dst = Idx + (static_cast<size_t>(b) * N + i) * topk;
    for (int m = lane; m < topk; m += kWave) dst[m] = sel[m];
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

template <typename T, int D>
static hipError_t launch_small(const TopkArgs& a, int kc) {
  constexpr int QT = kTopkQueryTiles;
  const int per_wave = 16 * QT;
  const int waves = (a.N + per_wave - 1) / per_wave;
  const int nw = waves >= 4 ? 4 : waves;
  const int qb = per_wave * nw;
  const int n_qblk = (a.N + qb - 1) / qb;
  const int nblocks = a.B * n_qblk;
  const size_t lds = topk_lds_bytes(a.dtype, a.d, kc);
  const T* q = static_cast<const T*>(a.q);
  const T* k = static_cast<const T*>(a.k);
  const T* v = static_cast<const T*>(a.v);
  T* o = static_cast<T*>(a.out);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
#define TARMAC_TOPK_CASE(KK)                                                                   \
  case KK:                                                                                     \
    hipLaunchKernelGGL((topk_small_kernel<T, D, KK, QT>), dim3(nblocks), dim3(64 * nw), lds, st, \
                       q, k, v, o, a.idx, a.N, n_qblk, kc, a.scale, nblocks);                 \
    break;
  switch (a.topk) {
    TARMAC_TOPK_CASE(1)
    TARMAC_TOPK_CASE(2)
    TARMAC_TOPK_CASE(3)
    TARMAC_TOPK_CASE(4)
    TARMAC_TOPK_CASE(5)
    TARMAC_TOPK_CASE(6)
    TARMAC_TOPK_CASE(7)
    TARMAC_TOPK_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef TARMAC_TOPK_CASE
  return hipGetLastError();
}

int wide_cap(const TopkArgs& a) { return a.select == kSelMasked ? a.N : a.topk; }

template <typename T, int D>
static hipError_t launch_wide(const TopkArgs& a) {
  // nw waves per workgroup, each holding N + cap words of LDS (<= 64 KiB total)
  const int cap = wide_cap(a);
  int nw = 16384 / (a.N + cap);
  nw = nw < 1 ? 1 : (nw > 4 ? 4 : nw);
  const long rows = static_cast<long>(a.B) * a.N;
  const int grid = static_cast<int>((rows + nw - 1) / nw);
  const size_t lds = static_cast<size_t>(nw) * (a.N + cap) * sizeof(float);
  hipLaunchKernelGGL((topk_wide_kernel<T, D>), dim3(grid), dim3(64 * nw), lds,
                     static_cast<hipStream_t>(a.stream), static_cast<const T*>(a.q),
                     static_cast<const T*>(a.k), static_cast<const T*>(a.v), static_cast<T*>(a.out),
                     a.idx, a.B, a.N, a.topk, a.scale, a.select, a.bisect, cap);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t dispatch_topk(const TopkArgs& a) {
  if (a.topk > kTopkSmallMax || a.select != kSelTopk) return launch_wide<T, D>(a);
  return launch_small<T, D>(a, a.key_chunk);
}

int g_topk_filter_mode = kFilterAuto;

// Where the filter-and-verify kernel beats the plain fp32 pass (measured on
// MI355X, d = 16): its fixed per-query cost (split staging, merge, exact
// rescoring) pays off once each query scans 512 keys, or 256 keys when the
// plain pass's per-score selection cost grows with k >= 3.
static bool filter_pays(const TopkArgs& a) { return a.N >= 512 || (a.N >= 256 && a.topk >= 3); }

hipError_t run_topk(const TopkArgs& a) {
  if (a.select == kSelTopk && g_topk_filter_mode != kFilterOff &&
      topk_filter_supported(a.dtype, a.d, a.topk) &&
      (g_topk_filter_mode == kFilterAlways || filter_pays(a)))
    return run_topk_filter(a);
  if (a.dtype == kF32) {
    switch (a.d) {
      case 8: return dispatch_topk<float, 8>(a);
      case 16: return dispatch_topk<float, 16>(a);
      case 32: return dispatch_topk<float, 32>(a);
      case 64: return dispatch_topk<float, 64>(a);
    }
  } else {
    switch (a.d) {
      case 16: return dispatch_topk<bf16, 16>(a);
      case 32: return dispatch_topk<bf16, 32>(a);
      case 64: return dispatch_topk<bf16, 64>(a);
    }
  }
  return hipErrorInvalidValue;
}

size_t topk_lds_bytes(int dtype, int d, int kc) {
  const int row = dtype == kF32 ? (d + 4) * 4 : (d + 8) * 2;
  const int kcb = (kc + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
  const size_t plain = static_cast<size_t>(kcb) * row;
  if (dtype != kF32 || d == 8) return plain;
  const size_t filt = topk_filter_lds_bytes(d, kc);
  return plain > filt ? plain : filt;
}

}  // namespace tarmac
