// Score-then-select top-k attention, fused: scores, selection, k-softmax and
// the gathered aggregation in one launch; no score row, index tensor or
// gathered value tensor reaches HBM.
//
// Reference behaviour: src/kernels/fused_topk_attention.py:211-333
// (fused_topk_attention_tiled) and src/kernels/streaming_topk_attention.py:
// 66-258 (streaming_topk_attention, incl. the optional retained-index output).
//
// Small k (1..8), fp32 register-list pass (topk_small_kernel), one launch
// shape for both the resident and the streamed variants:
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
// The same kernel with RULE serves the reference's masked (>= 32 halvings)
// and sort selection rules at k <= 8 (src/kernels/fused_topk_attention.py:
// 127-208, 405-504); queries the lists cannot settle go to rule_query_exact.
//
// Large k (> 8), and the rules elsewhere: sixteen lanes or one wave per query,
// an exact threshold found by bisection on the order-preserving integer key,
// ties at the threshold resolved by index.
#include <atomic>

#include "frag.hpp"
#include "select.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

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

__device__ __forceinline__ float wave_sumf(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

// One query of the masked rule (bisect >= 32) or the sort rule, by the whole
// wavefront, on the integer keys of its canonical scores: the row's keys
// (j = lane + 64 m) from K in global memory in the MFMA chain's fmaf order,
// kept in the wave's LDS row `skey`; the k-th key by bisection; then every
// key above it and, of the keys equal to it, all (masked) or the
// highest-index ones (sort). The same function as topk_wide_kernel, for the
// rows the register lists cannot settle: a tie across the k-th / (k+1)-th
// score, or non-finite inputs. Runtime loops keep its registers below the
// list pass's. `idx_row` (sort only, may be null) receives the set in
// ascending index order.
template <int D, bool POW2>
__device__ __forceinline__ void rule_query_exact(const float* __restrict__ Qb,
                                                 const float* __restrict__ Kb,
                                                 const float* __restrict__ Vb, float* __restrict__ Ob,
                                                 int32_t* __restrict__ idx_row, int* skey, int qi,
                                                 int N, int topk, float scale, int mode) {
  const int lane = threadIdx.x & 63;
  const unsigned long long below = (1ull << lane) - 1ull;
  const int nm = (N + 63) / 64;  // keys per lane (uniform)
  {
    float q[D];
    ld_f32<D>(q, Qb + static_cast<size_t>(qi) * D);
    if constexpr (POW2) {
#pragma unroll
      for (int c = 0; c < D; ++c) q[c] *= scale;
    }
#pragma unroll 1
    for (int m = 0; m < nm; ++m) {
      const int j = lane + 64 * m;
      const float* krow = Kb + static_cast<size_t>(min(j, N - 1)) * D;
      float acc = 0.f;
#pragma unroll
      for (int t = 0; t < D / 4; ++t)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = fmaf(q[kk * (D / 4) + t], krow[kk * (D / 4) + t], acc);
      if constexpr (!POW2) acc *= scale;
      if (j < N) skey[j] = ordered_key(j == qi ? -INFINITY : acc);
    }
  }
  auto key_at = [&](int m) { return skey[lane + 64 * m]; };  // m < nm, lane + 64 m < N
  auto count_ge = [&](long t) {
    int c = 0;
#pragma unroll 1
    for (int m = 0; m < nm; ++m) c += (lane + 64 * m < N && key_at(m) >= t) ? 1 : 0;
    return wave_sum(c);
  };
  // largest t with count(key >= t) >= topk, or a t with exactly topk keys at
  // or above it: both keep {key >= t_k} for the masked rule
  long lo = -2147483648L, hi = 2147483647L;
  while (lo < hi) {
    const long mid = lo + (hi - lo + 1) / 2;
    const int c = count_ge(mid);
    if (c >= topk) lo = mid; else hi = mid - 1;
    if (c == topk) break;
  }
  const int thr = static_cast<int>(lo);
  int gt = 0, eq = 0;
#pragma unroll 1
  for (int m = 0; m < nm; ++m) {
    if (lane + 64 * m >= N) continue;
    const int key = key_at(m);
    gt += key > thr ? 1 : 0;
    eq += key == thr ? 1 : 0;
  }
  gt = wave_sum(gt);
  eq = wave_sum(eq);
  const int need_ties = mode == kSelMasked ? eq : topk - gt;
  const int skip_ties = mode == kSelSort ? eq - need_ties : 0;
  unsigned picks = 0u;  // bit m: key lane + 64 m is kept
  int taken = 0, ties = 0;
  float mx = -INFINITY;
#pragma unroll 1
  for (int m = 0; m < nm; ++m) {
    const int j = lane + 64 * m;
    const int key = j < N ? key_at(m) : 0;
    const bool is_tie = j < N && key == thr;
    const unsigned long long tmask = __ballot(is_tie);
    const int tie_rank = ties + __popcll(tmask & below);
    const bool pick = j < N && (key > thr || (is_tie && tie_rank >= skip_ties &&
                                              tie_rank < skip_ties + need_ties));
    const unsigned long long pmask = __ballot(pick);
    if (pick) {
      picks |= 1u << m;
      mx = fmaxf(mx, __int_as_float(key ^ ((key >> 31) & 0x7fffffff)));
      if (idx_row != nullptr) idx_row[taken + __popcll(pmask & below)] = j;
    }
    taken += __popcll(pmask);
    ties += __popcll(tmask);
  }
  mx = wave_max(mx);
  auto weight = [&](int m) {
    const int key = key_at(m);
    return fast_exp2((__int_as_float(key ^ ((key >> 31) & 0x7fffffff)) - mx) * kLog2eF);
  };
  float den = 0.f;
#pragma unroll 1
  for (int m = 0; m < nm; ++m)
    if ((picks >> m) & 1u) den += weight(m);
  den = wave_sumf(den);
  constexpr int CH = D < 16 ? D : 16;  // output channels per pass
#pragma unroll 1
  for (int c0 = 0; c0 < D; c0 += CH) {
    float a[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) a[c] = 0.f;
#pragma unroll 1
    for (int m = 0; m < nm; ++m) {
      if ((picks >> m) & 1u) {
        const float w = weight(m);
        float vr[CH];
        ld_f32<CH>(vr, Vb + static_cast<size_t>(lane + 64 * m) * D + c0);
#pragma unroll
        for (int c = 0; c < CH; ++c) a[c] = fmaf(w, vr[c], a[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) a[c] = wave_sumf(a[c]);
    if (lane == 0) {
      const float inv = 1.f / den;
#pragma unroll
      for (int c = 0; c < CH; ++c) a[c] *= inv;
      st_f32<CH>(Ob + static_cast<size_t>(qi) * D + c0, a);
    }
  }
}

// RULE: the reference's masked (bisect >= 32) and sort rules, fp32. Both keep
// exactly the top k when the k-th and (k+1)-th scores differ, so the lists
// also carry the (k+1)-th value (val[K]); a query whose k-th and (k+1)-th
// values are equal, or whose inputs are not all finite (a NaN score is absent
// from a list but ranks in the integer key order), goes to rule_query_exact.
template <typename T, int D, int K, int QT, bool RULE = false>
__global__ void __launch_bounds__(256)
topk_small_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
                  T* __restrict__ O, int32_t* __restrict__ Idx, int N, int n_qblk, int kc,
                  float scale, int nblocks, int mode) {
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

  static_assert(sizeof(T) == 4, "the register-list pass selects on exact fp32 scores");
  constexpr int KV = RULE ? K + 1 : K;  // RULE: val[K] is the (K+1)-th best value
  float val[QT][KV];
  int ix[QT][K];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int m = 0; m < KV; ++m) val[qt][m] = -INFINITY;
#pragma unroll
    for (int m = 0; m < K; ++m) ix[qt][m] = kIdxSentinel;
  }
  // RULE: a non-finite element among the staged keys (one flag word past the
  // key rows) or in this lane's part of a query row
  unsigned* kflag = reinterpret_cast<unsigned*>(
      smem_raw + static_cast<size_t>((kc + kBlockKeys - 1) / kBlockKeys * kBlockKeys) * LDK * sizeof(T));
  int* skey = reinterpret_cast<int*>(kflag + 4) + static_cast<size_t>(wave) * ((N + 63) & ~63);
  bool qbad[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    qbad[qt] = false;
    if constexpr (RULE) {
#pragma unroll
      for (int e = 0; e < F::E; ++e) qbad[qt] = qbad[qt] || !__builtin_isfinite(frag[qt].q[e]);
    }
  }
  if (RULE && threadIdx.x == 0) *kflag = 0u;

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
    if constexpr (RULE) {
      bool kfin = true;  // a quarter row per thread and pass
      for (int u = threadIdx.x; u < cn * (D / 4); u += blockDim.x) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(Ks + (u / (D / 4)) * LDK + 4 * (u % (D / 4)));
#pragma unroll
        for (int e = 0; e < 4; ++e) kfin = kfin && __builtin_isfinite(x[e]);
      }
      if (!__all(kfin) && lane == 0) atomicOr(kflag, 1u);
    }
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
          for (int r = 0; r < 4; ++r) {
            if constexpr (RULE) topk_insert_x<K>(val[qt], ix[qt], s[qt][t][r], 16 * t + r);
            else topk_insert<K>(val[qt], ix[qt], s[qt][t][r], 16 * t + r);
          }
    }
  }
  rebase_list<QT, K>(ix, -base);  // back to absolute key indices
  if constexpr (RULE) __syncthreads();  // every wave's key check is in
  if (q0 >= N) return;

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int m = 0; m < K; ++m) ix[qt][m] += 4 * grp;
#pragma unroll
    for (int step = 16; step <= 32; step <<= 1) {
      float pv[KV];
      int pi[K];
#pragma unroll
      for (int m = 0; m < KV; ++m) pv[m] = __shfl_xor(val[qt][m], step);
#pragma unroll
      for (int m = 0; m < K; ++m) pi[m] = __shfl_xor(ix[qt][m], step);
      if constexpr (RULE) {
#pragma unroll
        for (int m = 0; m < K; ++m) topk_insert_lex_x<K>(val[qt], ix[qt], pv[m], pi[m]);
        val[qt][K] = vmax(val[qt][K], pv[K]);  // the partner's (K+1)-th
      } else {
#pragma unroll
        for (int m = 0; m < K; ++m) topk_insert_lex<K>(val[qt], ix[qt], pv[m], pi[m]);
      }
    }
  }
  bool slow[QT];  // RULE: this lane's query goes to rule_query_exact
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    slow[qt] = false;
    if constexpr (RULE) {
      const unsigned long long bad = __ballot(qbad[qt]);
      slow[qt] = *kflag != 0u || ((bad >> col) & 0x0001000100010001ull) != 0ull ||
                 val[qt][K - 1] == val[qt][K];
    }
  }

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = q0 + 16 * qt + col;
    if (qi >= N || slow[qt]) continue;
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
      for (int m = 0; m < K; ++m) {
        if constexpr (RULE) {  // the rules' sets in ascending index order
          int rank = 0;
#pragma unroll
          for (int u = 0; u < K; ++u) rank += ix[qt][u] < ix[qt][m] ? 1 : 0;
          dst[rank] = ix[qt][m];
        } else {
          dst[m] = ix[qt][m];
        }
      }
    }
  }
  if constexpr (RULE) {
    // the unsettled queries, one at a time across the whole wave
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      unsigned long long todo = __ballot(grp == 0 && slow[qt] && q0 + 16 * qt + col < N);
      while (todo != 0ull) {
        const int qj = q0 + 16 * qt + __builtin_ctzll(todo);
        todo &= todo - 1ull;
        rule_query_exact<D, POW2>(Q + boff, Kx + boff, V + boff, O + boff,
                                  Idx != nullptr ? Idx + (static_cast<size_t>(b) * N + qj) * K : nullptr,
                                  skey, qj, N, K, scale, mode);
      }
    }
  }
}

// Rows of up to 64 keys (N * d <= 2048), k <= 8: the register-list
// selection of topk_small_kernel with every operand fetched in one memory
// round trip. bf16 inputs are converted to fp32 on load, so the fp32 MFMA
// chain gives their canonical fp32 scores and the lists select on those
// exactly (the rule of every bf16 top-k path), with no rescoring. The wave loads its query fragments and the 16-key K fragments
// straight from global memory (16 rows x 64 B per fragment, coalesced) and,
// in the same burst, the batch row's V into LDS; selection then runs while the
// LDS writes land, and the k value rows are gathered from LDS instead of a
// second trip to memory. Selection and arithmetic are those of
// topk_small_kernel, so the results are identical.
template <typename T, int D, int K, int NT>
__global__ void __launch_bounds__(64)
topk_reg_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
                T* __restrict__ O, int32_t* __restrict__ Idx, int N, int n_qblk, float scale,
                int nblocks) {
  using F = Frag<float, D>;
  constexpr int QT = 2;
  constexpr int EO = D / 4;
  constexpr int LDV = D + 4;                 // padded LDS value row (fp32)
  constexpr int VE = 16 / static_cast<int>(sizeof(T));  // elements per 16-byte vector
  constexpr int NV = (NT * 16 * D / VE + 63) / 64;  // 16-byte vectors of V per lane
  constexpr bool POW2 = pow2_scale<D>();
  __shared__ __align__(16) float Vs[NT * 16 * LDV];
  const int lane = threadIdx.x;
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qb = blk - b * n_qblk;
  const int q0 = qb * 16 * QT;
  const int col = lane & 15, grp = lane >> 4;
  const size_t boff = static_cast<size_t>(b) * N * D;

  // query and key fragments as fp32 (bf16 widened exactly): lane group g
  // holds elements g*D/4 .. g*D/4 + D/4 - 1 of its row, the MFMA chain's order
  F frag[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    ld_row<T, F::E>(frag[qt].q,
                    Q + boff + static_cast<size_t>(min(q0 + 16 * qt + col, N - 1)) * D + grp * F::E);
    if constexpr (POW2) {
#pragma unroll
      for (int e = 0; e < F::E; ++e) frag[qt].q[e] *= scale;
    }
  }
  typename F::KF kf[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    ld_row<T, F::E>(kf[t].v, Kx + boff + static_cast<size_t>(min(16 * t + col, N - 1)) * D + grp * F::E);
  uint4 vr[NV];
  const uint4* vsrc = reinterpret_cast<const uint4*>(V + boff);
  const int nvv = N * D / VE;
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int e = lane + 64 * u;
    vr[u] = e < nvv ? vsrc[e] : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int e = lane + 64 * u;
    if (e < nvv) {
      const int row = e / (D / VE), cv = e - row * (D / VE);
      float x[VE];
      ld_row<T, VE>(x, reinterpret_cast<const T*>(&vr[u]));
      st_f32<VE>(Vs + row * LDV + VE * cv, x);
    }
  }

  float val[QT][K];
  int ix[QT][K];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int m = 0; m < K; ++m) { val[qt][m] = -INFINITY; ix[qt][m] = kIdxSentinel; }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < F::NI; ++i) sc = frag[qt].step(kf[t], i, sc);
      if constexpr (!POW2) sc *= scale;
      if (16 * t + 16 > N || 16 * t == q0 + 16 * qt) {  // wave-uniform: the tail or the diagonal tile
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = 16 * t + 4 * grp + r;
          if (key >= N || key == q0 + 16 * qt + col) sc[r] = -INFINITY;
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) topk_insert<K>(val[qt], ix[qt], sc[r], 16 * t + 4 * grp + r);
    }
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
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
  __syncthreads();  // the value rows are in LDS
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
      float vrow[EO];
      ld_f32<EO>(vrow, Vs + row * LDV + grp * EO);
#pragma unroll
      for (int c = 0; c < EO; ++c) acc[c] = fmaf(w, vrow[c], acc[c]);
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
                 T* __restrict__ O, int32_t* __restrict__ Idx, int N, int n_qblk, int topk,
                 float scale, int mode, int bisect, int cap, int k_in_lds) {
  constexpr int KST = D + 16 / static_cast<int>(sizeof(T));  // padded LDS key row
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int blk = xcd_logical_block(blockIdx.x, gridDim.x);  // a batch row's blocks share an XCD
  const int b = blk / n_qblk, qb = blk - b * n_qblk;
  const int i_raw = qb * nw + wave;
  const bool live = i_raw < N;  // wave-uniform
  const int i = live ? i_raw : N - 1;
  T* Ks = reinterpret_cast<T*>(smem_raw);
  const size_t kbytes = k_in_lds ? static_cast<size_t>(N) * KST * sizeof(T) : 0;
  float* S = reinterpret_cast<float*>(smem_raw + kbytes) + static_cast<size_t>(wave) * (N + cap);
  int* sel = reinterpret_cast<int*>(S + N);
  const size_t boff = static_cast<size_t>(b) * N * D;
  const bool pow2 = is_pow2_scale(scale);

  float q[D];
  ld_row<T, D>(q, Q + boff + static_cast<size_t>(i) * D);
  if (pow2) {
#pragma unroll
    for (int c = 0; c < D; ++c) q[c] *= scale;
  }
  if (k_in_lds) {  // uniform: the workgroup's queries share one copy of the batch row's keys
    stage_rows<T, D, KST>(Ks, Kx + boff, N, N);
    __syncthreads();
  }
  for (int j = lane; j < N; j += kWave) {
    // separate calls keep LDS reads as ds_read (a merged pointer would be generic)
    float s = k_in_lds ? canon_score<T, D>(q, Ks + j * KST)
                       : canon_score<T, D>(q, Kx + boff + static_cast<size_t>(j) * D);
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
    // largest t with count(key >= t) >= topk: the k-th largest key (or any t
    // with exactly topk keys at or above it, which selects the same set)
    long lo = -2147483648L, hi = 2147483647L;
    while (lo < hi) {
      const long mid = lo + (hi - lo + 1) / 2;
      int cnt = 0;
      for (int j = lane; j < N; j += kWave) cnt += (ordered_key(S[j]) >= mid) ? 1 : 0;
      cnt = wave_sum(cnt);
      if (cnt >= topk) lo = mid; else hi = mid - 1;
      if (cnt == topk) break;
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

  // Aggregation over the selected rows, all lanes at once: lane = 4 * slot + g
  // takes rows m = slot, slot + 16, ... and channels g*E .. g*E+E-1; the 16
  // slots are then summed with xor shuffles.
  constexpr int E = D / 4;
  const int slot = lane >> 2, g = lane & 3;
  float acc[E];
#pragma unroll
  for (int c = 0; c < E; ++c) acc[c] = 0.f;
  float den = 0.f;
  for (int m = slot; m < taken; m += 16) {
    const int j = sel[m];
    const float w = expf(S[j] - mx);
    den += w;
    float vr[E];
    ld_row<T, E>(vr, V + boff + static_cast<size_t>(j) * D + g * E);
#pragma unroll
    for (int c = 0; c < E; ++c) acc[c] = fmaf(w, vr[c], acc[c]);
  }
#pragma unroll
  for (int o = 4; o < kWave; o <<= 1) {
    den += __shfl_xor(den, o);
#pragma unroll
    for (int c = 0; c < E; ++c) acc[c] += __shfl_xor(acc[c], o);
  }
  if (slot == 0) {
    const float inv = 1.f / den;
    T* dst = O + boff + static_cast<size_t>(i) * D + g * E;
#pragma unroll
    for (int c = 0; c < E; ++c) {
      const float o = acc[c] * inv;
      if constexpr (sizeof(T) == 4) dst[c] = o;
      else dst[c] = f32_to_bf16(o);
    }
  }
  if (Idx != nullptr) {  // never for kSelMasked (the set size varies)
    int32_t* dst = Idx + (static_cast<size_t>(b) * N + i) * topk;
    for (int m = lane; m < topk; m += kWave) dst[m] = sel[m];
  }
}

// ---------------------------------------------------------------------------
// large k, N <= 16 * NS: sixteen lanes per query, keys in registers
// ---------------------------------------------------------------------------

// Same function as topk_wide_kernel (all three selection rules), four
// queries per wavefront and sixteen per workgroup. Lane (16 q + s) holds the
// integer keys of its query's peers j = s + 16 t, t < NS, so every count of
// the bisection is NS compares and a four-step xor reduction over the
// query's sixteen lanes. The selected (index, score) pairs are compacted into
// LDS in ascending index order; four slots x four channel groups then gather
// the value rows.
template <typename T, int D, int NS>
__global__ void __launch_bounds__(256)
topk_wide16_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
                   T* __restrict__ O, int32_t* __restrict__ Idx, int N, int n_qblk, int topk,
                   float scale, int mode, int bisect, int cap, int k_in_lds) {
  constexpr int KST = D + 16 / static_cast<int>(sizeof(T));  // padded LDS key row
  constexpr int kNone = -2147483647 - 1;                       // no peer in this slot
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int qs = lane >> 4, sub = lane & 15;
  const int blk = xcd_logical_block(blockIdx.x, gridDim.x);  // a batch row's blocks share an XCD
  const int b = blk / n_qblk, qb = blk - b * n_qblk;
  const int qslot = 4 * wave + qs;                 // query slot in the workgroup
  const int i_raw = 16 * qb + qslot;
  const bool live = i_raw < N;                     // uniform over the 16 lanes
  const int i = live ? i_raw : N - 1;
  T* Ks = reinterpret_cast<T*>(smem_raw);
  const size_t kbytes = k_in_lds ? static_cast<size_t>(N) * KST * sizeof(T) : 0;
  int* sel = reinterpret_cast<int*>(smem_raw + kbytes) + static_cast<size_t>(qslot) * 2 * cap;
  float* sel_s = reinterpret_cast<float*>(sel + cap);
  const size_t boff = static_cast<size_t>(b) * N * D;
  const bool pow2 = is_pow2_scale(scale);
  const unsigned long long below = (1ull << sub) - 1ull;
  auto seg = [&](unsigned long long m) { return (m >> (16 * qs)) & 0xffffull; };

  float q[D];
  ld_row<T, D>(q, Q + boff + static_cast<size_t>(i) * D);
  if (pow2) {
#pragma unroll
    for (int c = 0; c < D; ++c) q[c] *= scale;
  }
  if (k_in_lds) {
    stage_rows<T, D, KST>(Ks, Kx + boff, N, N);
    __syncthreads();
  }
  int key[NS];
#pragma unroll
  for (int t = 0; t < NS; ++t) {
    const int j = sub + 16 * t;
    key[t] = kNone;
    if (j < N) {
      float sc = k_in_lds ? canon_score<T, D>(q, Ks + j * KST)
                          : canon_score<T, D>(q, Kx + boff + static_cast<size_t>(j) * D);
      if (!pow2) sc *= scale;
      key[t] = ordered_key(j == i ? -INFINITY : sc);
    }
  }
  auto count_ge = [&](long m) {
    int c = 0;
#pragma unroll
    for (int t = 0; t < NS; ++t) c += key[t] >= m ? 1 : 0;
    return row16_reduce(c, [](int a, int b) { return a + b; });
  };

  long lo, hi;
  int iters;
  if (mode == kSelMasked) {
    // the reference's bisection, step for step (see topk_wide_kernel)
    int kmin = 2147483647, kmx = kNone;
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      const int j = sub + 16 * t;
      if (j < N) {
        kmx = max(kmx, key[t]);
        if (j != i) kmin = min(kmin, key[t]);
      }
    }
    kmin = row16_reduce(kmin, [](int a, int b) { return min(a, b); });
    kmx = row16_reduce(kmx, [](int a, int b) { return max(a, b); });
    lo = kmin;
    hi = kmx;
    iters = bisect;
  } else {
    lo = -2147483648L;
    hi = 2147483647L;
    iters = 32;  // closes the full 32-bit range
  }
  // Exactly topk keys at or above lo also settles the top-k rules (every key
  // >= lo is taken, no tie straddles lo); the masked rule runs all its
  // halvings, as the reference does. The loop ends when the wave's four
  // queries are all settled.
  bool settled = false;
  for (int it = 0; it < iters; ++it) {
    if (__all(settled)) break;
    const long mid = lo + (hi - lo + 1) / 2;
    const int c = count_ge(mid);
    const bool take = c >= topk;
    if (!settled) {
      lo = take ? mid : lo;
      hi = take ? hi : mid - 1;
    }
    settled = settled || (mode != kSelMasked && take && c == topk);
  }
  const int thr = static_cast<int>(lo);
  int gt = 0, eq = 0;
#pragma unroll
  for (int t = 0; t < NS; ++t) {
    gt += key[t] > thr ? 1 : 0;
    eq += (key[t] == thr && sub + 16 * t < N) ? 1 : 0;
  }
  gt = row16_reduce(gt, [](int a, int b) { return a + b; });
  eq = row16_reduce(eq, [](int a, int b) { return a + b; });
  const int need_ties = mode == kSelMasked ? eq : topk - gt;
  const int skip_ties = mode == kSelSort ? eq - need_ties : 0;

  // compact (index, score) in ascending index order: t-major, lane-minor
  int taken = 0, ties = 0;
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < NS; ++t) {
    const int j = sub + 16 * t;
    const bool is_tie = j < N && key[t] == thr;
    const unsigned long long tmask = seg(__ballot(is_tie));
    const int tie_rank = ties + __popcll(tmask & below);
    const bool pick = j < N && (key[t] > thr || (is_tie && tie_rank >= skip_ties &&
                                                  tie_rank < skip_ties + need_ties));
    const unsigned long long pmask = seg(__ballot(pick));
    if (pick) {
      const int pos = taken + __popcll(pmask & below);
      const float sc = __int_as_float(key[t] ^ ((key[t] >> 31) & 0x7fffffff));
      sel[pos] = j;
      sel_s[pos] = sc;
      mx = fmaxf(mx, sc);
    }
    taken += __popcll(pmask);
    ties += __popcll(tmask);
  }
  mx = row16_reduce(mx, [](float a, float b) { return fmaxf(a, b); });
  __syncthreads();  // the compacted lists, written by other lanes, are read below

  // aggregation: lane s = 4 slot + g takes rows slot, slot + 4, ..., channels g*E..
  constexpr int E = D / 4;
  const int slot = sub >> 2, g = sub & 3;
  float acc[E];
#pragma unroll
  for (int c = 0; c < E; ++c) acc[c] = 0.f;
  float den = 0.f;
  for (int m = slot; m < taken; m += 4) {
    const int j = sel[m];
    const float w = expf(sel_s[m] - mx);
    den += w;
    float vr[E];
    ld_row<T, E>(vr, V + boff + static_cast<size_t>(j) * D + g * E);
#pragma unroll
    for (int c = 0; c < E; ++c) acc[c] = fmaf(w, vr[c], acc[c]);
  }
  den = row16_reduce_stride4(den, [](float a, float b) { return a + b; });
#pragma unroll
  for (int c = 0; c < E; ++c) acc[c] = row16_reduce_stride4(acc[c], [](float a, float b) { return a + b; });
  if (!live) return;
  if (slot == 0) {
    const float inv = 1.f / den;
    T* dst = O + boff + static_cast<size_t>(i) * D + g * E;
#pragma unroll
    for (int c = 0; c < E; ++c) {
      const float o = acc[c] * inv;
      if constexpr (sizeof(T) == 4) dst[c] = o;
      else dst[c] = f32_to_bf16(o);
    }
  }
  if (Idx != nullptr) {  // never for kSelMasked
    int32_t* dst = Idx + (static_cast<size_t>(b) * N + i) * topk;
    for (int m = sub; m < topk; m += 16) dst[m] = sel[m];
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

template <typename T, int D, bool RULE = false>
static hipError_t launch_small(const TopkArgs& a, int kc) {
  constexpr int QT = kTopkQueryTiles;
  const int per_wave = 16 * QT;
  const int waves = (a.N + per_wave - 1) / per_wave;
  const int nw = waves >= 4 ? 4 : waves;
  const int qb = per_wave * nw;
  const int n_qblk = (a.N + qb - 1) / qb;
  const int nblocks = a.B * n_qblk;
  // this kernel's own key copy (topk_lds_bytes also covers the filter
  // kernel's larger split rows; allocating that would cost occupancy)
  // RULE: + the key flag and one key row per wave for rule_query_exact
  const size_t lds = plain_lds_bytes(a.dtype, a.d, kc) +
                     (RULE ? 16 + static_cast<size_t>(nw) * ((a.N + 63) & ~63) * 4 : 0);
  const T* q = static_cast<const T*>(a.q);
  const T* k = static_cast<const T*>(a.k);
  const T* v = static_cast<const T*>(a.v);
  T* o = static_cast<T*>(a.out);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
#define TARMAC_TOPK_CASE(KK)                                                                   \
  case KK:                                                                                     \
    hipLaunchKernelGGL((topk_small_kernel<T, D, KK, QT, RULE>), dim3(nblocks), dim3(64 * nw), lds, \
                       st, q, k, v, o, a.idx, a.N, n_qblk, kc, a.scale, nblocks, a.select);  \
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

template <typename T, int D, int NT>
static hipError_t launch_reg(const TopkArgs& a) {
  const int n_qblk = (a.N + 31) / 32;
  const int nblocks = a.B * n_qblk;
  const T* q = static_cast<const T*>(a.q);
  const T* k = static_cast<const T*>(a.k);
  const T* v = static_cast<const T*>(a.v);
  T* o = static_cast<T*>(a.out);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
#define TARMAC_TOPK_REG_CASE(KK)                                                                  \
  case KK:                                                                                        \
    hipLaunchKernelGGL((topk_reg_kernel<T, D, KK, NT>), dim3(nblocks), dim3(64), 0, st, q, k, v, o, \
                       a.idx, a.N, n_qblk, a.scale, nblocks);                                     \
    break;
  switch (a.topk) {
    TARMAC_TOPK_REG_CASE(1)
    TARMAC_TOPK_REG_CASE(2)
    TARMAC_TOPK_REG_CASE(3)
    TARMAC_TOPK_REG_CASE(4)
    TARMAC_TOPK_REG_CASE(5)
    TARMAC_TOPK_REG_CASE(6)
    TARMAC_TOPK_REG_CASE(7)
    TARMAC_TOPK_REG_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef TARMAC_TOPK_REG_CASE
  return hipGetLastError();
}

// topk_reg_kernel's domain: rows of up to 64 keys with N * d <= 2048 (the V
// row block fits a lane's share of registers on its way to LDS). fp32 honours
// an explicit smaller key chunk (the LDS kernels give identical results);
// bf16 ignores it, so a streamed bf16 call returns the resident call's
// outputs bit for bit (the packed pass's softmax runs on its proof-bounded
// scores, this kernel's on the canonical ones).
static bool topk_reg_supported(const TopkArgs& a) {
  return a.N <= 64 && a.N * a.d <= 2048 && (a.dtype == kBf16 || a.key_chunk >= a.N) &&
         a.topk <= kTopkSmallMax && a.select == kSelTopk;
}

template <typename T, int D>
static bool topk_reg(const TopkArgs& a, hipError_t* e) {
  if (!topk_reg_supported(a)) return false;
  switch ((a.N + 15) / 16) {
    case 1: *e = launch_reg<T, D, 1>(a); return true;
    case 2: *e = launch_reg<T, D, 2>(a); return true;
    case 3: if constexpr (D <= 32) { *e = launch_reg<T, D, 3>(a); return true; } break;
    case 4: if constexpr (D <= 32) { *e = launch_reg<T, D, 4>(a); return true; } break;
  }
  return false;
}

int wide_cap(const TopkArgs& a) { return a.select == kSelMasked ? a.N : a.topk; }

template <typename T, int D, int NS>
static hipError_t launch_wide16(const TopkArgs& a, int cap, size_t kbytes, size_t selbytes) {
  const int k_in_lds = kbytes + selbytes <= 65536 ? 1 : 0;
  const int n_qblk = (a.N + 15) / 16;
  const size_t lds = (k_in_lds ? kbytes : 0) + selbytes;
  hipLaunchKernelGGL((topk_wide16_kernel<T, D, NS>), dim3(a.B * n_qblk), dim3(256), lds,
                     static_cast<hipStream_t>(a.stream), static_cast<const T*>(a.q),
                     static_cast<const T*>(a.k), static_cast<const T*>(a.v), static_cast<T*>(a.out),
                     a.idx, a.N, n_qblk, a.topk, a.scale, a.select, a.bisect, cap, k_in_lds);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_wide(const TopkArgs& a) {
  {
    // sixteen lanes per query while the keys fit registers and the selected
    // lists of sixteen queries fit LDS
    constexpr int KST = D + 16 / static_cast<int>(sizeof(T));
    const int cap = wide_cap(a);
    const size_t selbytes = static_cast<size_t>(16) * 2 * cap * sizeof(int);
    const size_t kbytes = static_cast<size_t>(a.N) * KST * sizeof(T);
    if (selbytes <= 65536) {
      if (a.N <= 64) return launch_wide16<T, D, 4>(a, cap, kbytes, selbytes);
      if (a.N <= 128) return launch_wide16<T, D, 8>(a, cap, kbytes, selbytes);
      if (a.N <= 256) return launch_wide16<T, D, 16>(a, cap, kbytes, selbytes);
      if (a.N <= 512) return launch_wide16<T, D, 32>(a, cap, kbytes, selbytes);
    }
  }
  // nw waves per workgroup (one query each), each holding N + cap words of
  // LDS; the batch row's keys join them in LDS when everything fits 64 KiB
  constexpr size_t kBudget = 65536;
  constexpr int KST = D + 16 / static_cast<int>(sizeof(T));
  const int cap = wide_cap(a);
  const size_t per_wave = static_cast<size_t>(a.N + cap) * sizeof(float);
  const size_t kbytes = static_cast<size_t>(a.N) * KST * sizeof(T);
  int nw = 4, k_in_lds = 1;
  while (nw > 1 && kbytes + nw * per_wave > kBudget) --nw;
  if (kbytes + nw * per_wave > kBudget) {
    k_in_lds = 0;
    nw = static_cast<int>(kBudget / per_wave);
    nw = nw < 1 ? 1 : (nw > 4 ? 4 : nw);
  }
  const int n_qblk = (a.N + nw - 1) / nw;
  const size_t lds = (k_in_lds ? kbytes : 0) + nw * per_wave;
  hipLaunchKernelGGL((topk_wide_kernel<T, D>), dim3(a.B * n_qblk), dim3(64 * nw), lds,
                     static_cast<hipStream_t>(a.stream), static_cast<const T*>(a.q),
                     static_cast<const T*>(a.k), static_cast<const T*>(a.v), static_cast<T*>(a.out),
                     a.idx, a.N, n_qblk, a.topk, a.scale, a.select, a.bisect, cap, k_in_lds);
  return hipGetLastError();
}

// The masked rule after >= 32 halvings and the sort rule, fp32, k <= 8,
// N <= 1024 (the reference's own limit): the register lists with the
// (k+1)-th value, per-query fallback to the exact wave path. 32 halvings close
// any interval of 2^32 integer keys, so the masked threshold is then the k-th
// key itself; fewer halvings (a superset) and bf16 run the wide kernels.
bool topk_rule_lists(const TopkArgs& a) {
  return a.select != kSelTopk && a.dtype == kF32 && a.topk <= kTopkSmallMax && a.N <= 1024 &&
         (a.select == kSelSort || a.bisect >= 32) && a.key_chunk > 0;
}

template <typename T, int D>
static hipError_t dispatch_topk(const TopkArgs& a) {
  if constexpr (sizeof(T) == 4)
    if (topk_rule_lists(a)) return launch_small<T, D, true>(a, a.key_chunk);
  if (a.topk > kTopkSmallMax || a.select != kSelTopk) return launch_wide<T, D>(a);
  hipError_t e;
  if (topk_reg<T, D>(a, &e)) return e;
  if constexpr (sizeof(T) == 4) return launch_small<T, D>(a, a.key_chunk);
  return hipErrorInvalidValue;  // bf16 k <= 8 runs the packed or filter kernels
}

// Process-wide choice between equally exact implementations (only the time
// differs); atomic so that concurrent calls and a concurrent setter do not race.
static std::atomic<int> g_topk_filter_mode{kFilterAuto};

int topk_filter_mode() { return g_topk_filter_mode.load(std::memory_order_relaxed); }
int set_topk_filter_mode(int mode) { return g_topk_filter_mode.exchange(mode); }

// Process-wide override of the query tiles per wave (also exact either way).
static std::atomic<int> g_query_tiles_mode{kTilesAuto};

int set_query_tiles_mode(int mode) { return g_query_tiles_mode.exchange(mode); }
int query_tiles_mode() { return g_query_tiles_mode.load(std::memory_order_relaxed); }

bool one_query_tile(int B, int N) {
  switch (g_query_tiles_mode.load(std::memory_order_relaxed)) {
    case kTilesOne: return true;
    case kTilesTwo: return false;
    default: break;
  }
  // two tiles per wave halve the per-query staging and merge cost, unless the
  // batch is then too small to give every SIMD a wave (B * N / 32 < 4 * kCUs)
  return static_cast<long>(B) * ((N + 31) / 32) < 4L * kCUs;
}

enum TopkPath { kPathPacked, kPathPackedSplit, kPathSplit32, kPathFilter, kPathLists };

// The implementation for k <= 8 (all return identical results). Automatic
// choice from interleaved timings on MI355X (B = 1024 for fp32 d = 16, the
// configs[1] sweep; the configs[2] bf16 grid), us:
//   fp32, d = 16: split-bf16 scores on 32 x 32 tiles (topk_split32.hip)
//     for k <= 4 and N = 128 .. 256 at batches of two query tiles per wave;
//     otherwise the packed pass on split-bf16 scores from N = 160, and
//     at N = 128 for k >= 3 with B >= 1024 (see choose_path) (N=256
//     k=1: 28.4 vs lists 30.4; k=2: 31.1 vs 37.1 lists, 34.5 filter; k=4:
//     38.1 vs 44.1 filter, 56.5 lists; N=512 k=2: 83.5 vs 96.2 filter, 117.4
//     lists); below that the register lists for k <= 2 (N=64 k=1: 5.9 vs
//     6.7 packed, 9.2 split) and the fp32-MFMA packed pass above (N=128 k=4:
//     17.9 vs 19.9 lists), except at N <= 32, where the one-round-trip list
//     kernel wins at every k (rocprof, B=1024 N=32 k=4: 7.4 vs 7.8 packed).
//   fp32, d = 8, 32, 64: register lists for k <= 2 (every k at N <= 32), packed above.
//   bf16: packed, the 32 x 32 kernel at d = 16 with two query tiles per wave
//     (k = 4, N = 193 .. 256; k = 2, 3, N = 193 .. 384, B <= 1024), or the bf16
//     filter at d = 16 with N >= 256 and k >= 4
//     (B=1024 N=256 k=4: 35.1 vs 40.4) or k = 2, 3 with B <= 1024; at d = 16, rows of up to 64 keys
//     with k <= 2 and rows of up to 32 keys take the one-round-trip register
//     lists, which widen bf16 to fp32 and select on the canonical scores
//     directly.
static TopkPath choose_path(const TopkArgs& a, int mode) {
  const bool filt = topk_filter_supported(a.dtype, a.d, a.topk);
  const bool split = packed_split_supported(a.dtype, a.d);
  switch (mode) {
    case kFilterOff: return kPathPacked;
    case kFilterAlways: return filt ? kPathFilter : kPathPacked;
    case kFilterLegacy: return a.dtype == kF32 ? kPathLists : kPathPacked;
    case kFilterPackedSplit: return split ? kPathPackedSplit : kPathPacked;
    case kFilterSplit32:
      return split32_supported(a) ? kPathSplit32 : (split ? kPathPackedSplit : kPathPacked);
    default: break;
  }
  if (a.dtype == kBf16) {
    // the one-round-trip lists (exact fp32 chain on the widened inputs) at
    // d = 16 where they win: k <= 2, or every k at N <= 32 (B=4096 N=64 k=1:
    // 11.5 vs 12.5 packed; N=32 k=1/4: 5.5/10.5 vs 8.0/12.2; at d = 32 the
    // fp32 chain's 8 steps per tile lose: N=64 k=1 21.9 vs 16.6)
    if (topk_reg_supported(a) && a.d == 16 && (a.topk <= 2 || a.N <= 32)) return kPathLists;
    // k <= 4 (measured per cell at d = 16, B = 32 .. 4096, N = 128 .. 1024,
    // graph-batched calls): the filter where the packed pass's per-query
    // exact tail sets a small launch's time -- rows of 512 keys and more at
    // B <= 128, of 1024 at k >= 3 up to B = 256 (B=32 N=1024 k=3/4: 13.4/15.3
    // vs 21.9/24.7 packed; B=256: 60.7/70.9 vs 65.5/77.3); the 32 x 32
    // kernel's single-product form (one bf16 MFMA per tile, two query tiles
    // per wave) at k = 4 on rows of 193-512 keys up to B = 1024 (B=256
    // N=384: 15.8 vs 16.6 packed, 20.7 filter; B=1024 N=384/512: 50.3/79.4
    // vs 50.3/80.1 packed, 70.2/84.5 filter) and at k = 2, 3 on rows of
    // 193-384 keys up to B = 256 (B=128 N=256 k=2/3: 6.0/6.6 vs 6.4/7.1
    // packed); the packed pass elsewhere (B=1024 N=256 k=2/3: 20.0/23.5 vs
    // 21.3/24.6 on 32 x 32 tiles; B=4096 N=384 k=4: 181.8 vs 185.6, 266.2
    // filter; B=1024 N=1024 k=2/3: 184.6/220.2 vs 189.8/230.2 filter)
    // Where the 32 x 32 kernel would run but the batch takes one query tile
    // per wave, the filter runs: its outputs equal the 32 x 32 kernel's bit
    // for bit (both take the softmax of the exact scores; the packed pass's
    // runs on its proof-bounded ones), so the launch shape never changes a
    // result.
    if (a.topk <= 4) {
      if (filt && a.N >= 512 && (a.B <= 128 || (a.N >= 1024 && a.B <= 256 && a.topk >= 3)))
        return kPathFilter;
      if (split32_supported(a) && a.N > 192 &&
          ((a.topk == 4 && a.N <= 512 && a.B <= 1024) ||
           (a.topk >= 2 && a.topk <= 3 && a.N <= 384 && a.B <= 256)))
        return !one_query_tile(a.B, a.N) ? kPathSplit32 : (filt ? kPathFilter : kPathPacked);
      return kPathPacked;
    }
    // k = 5-8: the filter at small batches (B=32 N=384 k=5: 7.9 vs 10.8
    // packed) and on 1024-key rows up to B = 256 at k <= 6 (B=256 k=5/6:
    // 82.4/91.9 vs 87.2/99.7), the packed pass elsewhere (B=256 N=384
    // k=5/6/8: 19.9/20.9/36.9 vs 28.8/27.2/38.1 filter; B=4096 N=384 k=8:
    // 310.9 vs 451.3)
    if (filt && a.N >= 256 && (a.B <= 128 || (a.N >= 1024 && a.B <= 256 && a.topk <= 6)))
      return kPathFilter;
    return kPathPacked;
  }
  // k <= 4 on batches that take one query tile per wave, rows of 65-256
  // keys or B * N up to 16384: the packed pass on exact fp32 scores (B=32,
  // graph-batched calls: N=128 k=1/2: 4.2/4.4 vs 4.6/5.7 lists; N=256
  // k=1/2/4: 5.5/5.7/6.9 vs 5.9/6.2/7.3 on split-bf16 scores; N=384:
  // 6.9/7.1/8.4 vs 7.2/7.5/8.8; at B=64 N=384 the split-bf16 scores win
  // again, 8.3 vs 9.0 at k = 1)
  if (a.topk <= 4 && a.N > 64 && (a.N <= 256 || a.B * a.N <= 16384) && one_query_tile(a.B, a.N))
    return kPathPacked;
  // k = 1 at d = 32, 64 on rows of 512-1023 keys from B = 256: the filter
  // (B=256 N=512/768 d=32: 44.1/88.1 vs 46.3/95.3 lists; d=64: 80.1/144.2 vs
  // 83.2/167.0; at d = 16 the split-bf16 scores stay ahead, N=768: 40.4 vs
  // 47.7)
  if (filt && a.d >= 32 && a.topk == 1 && a.N >= 512 && a.N < 1024 && a.B >= 256)
    return kPathFilter;
  // d = 64, k >= 3 on rows of 512 keys and more from B = 1024: the register
  // lists (B=1024 N=512 k=3/4/6: 383.1/461.7/524.7 vs 408.1/514.2/580.0
  // packed; B=2048 k=4: 862.8 vs 1016.0; at B = 256 packed stays ahead,
  // 122.9 vs 124.0 at k = 4)
  if (a.d == 64 && a.topk >= 3 && a.N >= 512 && a.B >= 1024) return kPathLists;
  // the lists at k <= 2 on rows of up to 128 keys up to B = 256 (B=256
  // N=128 k=1/2: 4.8/5.9 vs 5.4/6.1 on 32 x 32 tiles)
  if (a.topk <= 2 && a.N <= 128 && a.B <= 256) return kPathLists;
  // split-bf16 scores on 32 x 32 tiles for rows of 128 to 256 keys once the
  // batch gives every SIMD a wave of 32 queries (B=1024 N=256 k=1/2/4:
  // 24.3/27.3/35.2 vs 26.2/28.6/35.9 on 16 x 16 tiles; N=128: 10.4/11.7/16.2
  // vs 10.7 / 13.1 lists and 16.3 packed split; B=4096 N=256 k=2: 96.1 vs
  // 99.5)
  if (split32_supported(a) && a.N >= 128 && !one_query_tile(a.B, a.N)) return kPathSplit32;
  // split-bf16 scores from N = 160 at any k (B=1024 N=192 k=2/4: 26.0/32.3
  // vs 28.0 lists / 36.3 packed; B=4096 N=192 k=4: 111.2 vs 126.9), and at
  // N = 128 for k >= 3 once B >= 1024 (B=4096 N=128 k=3/4: 45.3/52.1 vs
  // 47.0/53.6 packed; k = 2 stays on the lists there, 39.4 vs 40.4)
  if (split && (a.N >= 160 || (a.N >= 128 && a.B >= 1024 && a.topk >= 3))) return kPathPackedSplit;
  return (a.topk <= 2 || a.N <= 32) ? kPathLists : kPathPacked;
}

hipError_t run_topk(const TopkArgs& a) {
  if (a.d == 128) {
    // head width 128: the packed pass for k <= 8 under every filter mode,
    // the wide kernels for larger k and the other selection rules
    if (a.select == kSelTopk && a.topk <= kTopkSmallMax) return run_topk_packed_d128(a);
    return a.dtype == kF32 ? launch_wide<float, 128>(a) : launch_wide<bf16, 128>(a);
  }
  if (a.select == kSelTopk && a.topk <= kTopkSmallMax) {
    switch (choose_path(a, topk_filter_mode())) {
      case kPathPacked: return run_topk_packed(a, false);
      case kPathPackedSplit: return run_topk_packed(a, true);
      case kPathSplit32: return run_topk_split32(a);
      case kPathFilter: return run_topk_filter(a);
      case kPathLists: break;
    }
  }
  if (topk_hist_supported(a)) return run_topk_hist(a);
  switch (a.dtype == kF32 ? a.d : -a.d) {
    case 8: return dispatch_topk<float, 8>(a);
    case 16: return dispatch_topk<float, 16>(a);
    case 32: return dispatch_topk<float, 32>(a);
    case 64: return dispatch_topk<float, 64>(a);
    case -16: return dispatch_topk<bf16, 16>(a);
    case -32: return dispatch_topk<bf16, 32>(a);
    case -64: return dispatch_topk<bf16, 64>(a);
  }
  return hipErrorInvalidValue;
}

size_t plain_lds_bytes(int dtype, int d, int kc) {
  const int row = dtype == kF32 ? (d + 4) * 4 : (d + 8) * 2;
  const int kcb = (kc + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
  return static_cast<size_t>(kcb) * row;
}

size_t topk_lds_bytes(int dtype, int d, int kc) {
  const size_t plain = plain_lds_bytes(dtype, d, kc);
  if (!topk_filter_supported(dtype, d, 1)) return plain;
  const size_t filt = topk_filter_lds_bytes(dtype, d, kc);
  return plain > filt ? plain : filt;
}

}  // namespace tarmac
