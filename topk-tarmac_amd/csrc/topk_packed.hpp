// Exact score-then-select top-k attention (k <= 8) on packed values.
//
// Reference behaviour: src/kernels/fused_topk_attention.py:211-333
// (fused_topk_attention_tiled) and src/kernels/streaming_topk_attention.py:
// 66-258 (streaming_topk_attention, incl. the retained-index output), with the
// tie rule score desc / index asc (:37-44). For bf16 inputs the retained set is
// the exact top k of the canonical fp32 scores of the inputs converted to fp32
// -- the rule the reference's bf16 study ranks by (scripts/bench_precision.py:
// 202-209) -- so fp32 and bf16 follow one exact rule on every shape.
//
// Layout: workgroup = (batch row b, block of 16 * QT * nw queries); keys pass
// through LDS in chunks of kc rows (kc >= N: the row is resident); each wave
// forms 16x16 S^T tiles with MFMA, so lane l owns query l % 16 and, per tile,
// keys 4 * (l / 16) + r (r = 0..3).
//
//  1. scan: a score keeps its high bits and carries, in its low fb mantissa
//     bits, a field naming the key within the current segment of 2^fb keys:
//     bits [4, fb) the 16-key tile, bits 2..3 the row r, bits 0..1 left zero
//     for the lane group (added at the merge). A row of up to 1024 keys is one
//     segment with the fewest bits that name its keys (fb = 8 at N = 256);
//     longer rows use 10-bit segments. One bitfield insert per score,
//     then a value-only insertion into a descending list of K + 2 entries
//     (max / med3): K + 3 VALU operations per score and no index compares.
//     Clearing low bits is a monotone map, so the list holds the K + 2 largest
//     truncated scores (distinct fields make distinct values).
//  2. merge: the lane group goes into bits 0..1 and the four lane lists of a
//     query merge with two xor-shuffle steps; every lane of the query ends with
//     the same K + 2 entries.
//  3. prove: fp32 scores come from fp32 MFMA and ARE the canonical scores, so
//     if trunc(K-th) > trunc((K+1)-th) every key outside the first K has a
//     strictly smaller score and the first K are exactly the top k. bf16 scores
//     come from bf16 MFMA (exact products, fp32 accumulation) and differ from
//     the canonical fp32 chain by at most eps |q| |k_j| (packed_eps): the
//     first K are exactly the top k if, after exact rescoring, the smallest of
//     them exceeds the (K+1)-th entry's largest possible score plus that bound.
//  4. rescore: the K winners are rescored in the canonical fp32 order (their
//     softmax weights are then bit-for-bit those of the oracle's scores) and
//     sorted by (score desc, index asc).
//  5. fallback: an unproven query is recomputed exactly by the whole wave
//     (exact_query_topk_lanes: its row's canonical scores on the VALU, one
//     key row per lane, per-lane lists, a six-step merge) -- the result never depends on the packing, only the
//     time does.
//  6. k-softmax and the gathered aggregation over the K value rows.
//
// The kernel and its launchers, instantiated per head width by
// topk_packed.hip (d <= 64) and topk_packed_d128.hip (d = 128) so the two
// halves compile in parallel.
#pragma once

#include "exact.hpp"
#include "frag.hpp"
#include "select.hpp"
#include "split.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

// 16-key tiles per scan block: two keep the block's scores and key fragments
// at 24 VGPRs (four tiles: 48).
constexpr int kPackedBlockTiles = 2;

// Keys per packing segment for a lane field of FB bits.
template <int FB>
constexpr int seg_keys() {
  return 1 << FB;
}

// The field mask's complement as a VGPR value the compiler cannot fold: the
// packing instruction (pack_field_u) then takes it from a VGPR and the
// (wave-uniform) field from an SGPR, within the one scalar operand a VOP3
// instruction may read.
template <int FB>
__device__ __forceinline__ uint32_t field_nmask_vgpr() {
  uint32_t m;
  asm volatile("v_mov_b32 %0, %1" : "=v"(m) : "i"(~((1u << FB) - 1u)));
  return m;
}

// Key offset within its segment from a merged field (tile | r | grp).
__device__ __forceinline__ int field_key(uint32_t w) {
  return static_cast<int>(16u * (w >> 4) + 4u * (w & 3u) + ((w >> 2) & 3u));
}

// Decode a lane's packed segment lists (NS sub-lists per query tile) into
// (truncated score, key) pairs, fold them into its running lex list and
// restart the segment lists.
template <int QT, int NS, int L, int FB>
__device__ __forceinline__ void flush_packed(float (&pv)[QT][NS][L], float (&rv)[QT][L],
                                             int (&ri)[QT][L], int segbase, int grp) {
  constexpr uint32_t M = (1u << FB) - 1u;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int j = 0; j < NS; ++j)
#pragma unroll
      for (int m = 0; m < L; ++m) {
        const uint32_t bits = __float_as_uint(pv[qt][j][m]);
        const bool live = pv[qt][j][m] >= kMaskedBelow;
        const int key = segbase + field_key((bits & M) | static_cast<uint32_t>(grp));
        topk_insert_lex<L>(rv[qt], ri[qt], live ? __uint_as_float(bits & ~M) : kMasked,
                           live ? key : kIdxSentinel);
        pv[qt][j][m] = kMasked;
      }
}

// Scoring per input: the query fragment, the LDS key row (element type and
// stride) and its staging. fp32: exact fp32 MFMA scores from plain rows, or
// (SPLIT) bf16 MFMA on three-way split operands (x = hi + mid + lo), which
// approximates the fp32 dot to 2^-19.9 sum_c |q_c k_c| at a third of the MFMA
// cycles; bf16: bf16 MFMA on the plain rows.
template <typename T, int D, bool SPLIT>
struct PackedIn;
template <int D>
struct PackedIn<float, D, false> {
  using F = Frag<float, D>;
  using R = float;
  static constexpr int LDK = F::LDK;
};
template <int D>
struct PackedIn<float, D, true> {
  using F = SplitFrag<D>;
  using R = bf16;
  static constexpr int LDK = SplitFrag<D>::LDK;
};
template <int D>
struct PackedIn<bf16, D, false> {
  using F = Frag<bf16, D>;
  using R = bf16;
  static constexpr int LDK = F::LDK;
};

// k-softmax over a query's K retained scores (score desc) and the gathered
// aggregation of their value rows; this lane writes channels grp*D/4 .. of
// query qi, and lane row 0 the retained indices.
template <typename T, int D, int K>
__device__ __forceinline__ void finish_tile(const T* __restrict__ V, T* __restrict__ O,
                                            int32_t* __restrict__ Idx, int b, int N, int qi,
                                            int grp, const float (&val)[K], const int (&ix)[K]) {
  constexpr int EO = D / 4;
  if (qi >= N) return;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const float mx = val[0];
  float acc[EO];
#pragma unroll
  for (int c = 0; c < EO; ++c) acc[c] = 0.f;
  float den = 0.f;
#pragma unroll
  for (int m = 0; m < K; ++m) {
    const float w = fast_exp2((val[m] - mx) * kLog2eF);
    den += w;
    const int row = min(max(ix[m], 0), N - 1);
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
    for (int m = 0; m < K; ++m) dst[m] = ix[m];
  }
}

// ONESEG: every key of the row fits one segment, and the field width is a
// launch argument (fm_arg: the low-bit mask, 2^fb - 1 with 2^fb >= the row
// rounded up to whole 16-key tiles), so short rows truncate less; FB is the
// width of multi-segment rows.
template <typename T, int D, int K, int QT, int NS, int FB, bool ONESEG, bool SPLIT>
__global__ void __launch_bounds__(512)
topk_packed_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
                   T* __restrict__ O, int32_t* __restrict__ Idx, int N, int n_qblk, int kc,
                   float scale, int nblocks, uint32_t fm_arg) {
  using PI = PackedIn<T, D, SPLIT>;
  using F = typename PI::F;
  using R = typename PI::R;  // LDS key row element
  constexpr int LDK = PI::LDK;
  constexpr int BT = kPackedBlockTiles;     // 16-key tiles per scan block
  constexpr int BK = 16 * BT;
  constexpr int C = K + 1;                   // candidates rescored when needed
  constexpr int L = K + 2;                   // list entries: the candidates and the (K+2)-th
  constexpr bool EXACT = sizeof(T) == 4 && !SPLIT;  // fp32 MFMA scores are the canonical scores
  constexpr bool RESCORE = sizeof(T) == 4;  // fp32 softmax needs the canonical scores
  constexpr bool POW2 = pow2_scale<D>();
  const uint32_t FM = ONESEG ? fm_arg : (1u << FB) - 1u;
  constexpr int SEGK = seg_keys<FB>();
  extern __shared__ __align__(16) unsigned char smem_raw[];
  unsigned* kmax_slot = reinterpret_cast<unsigned*>(smem_raw);  // approximate scores: max |k|^2
  R* Ks = reinterpret_cast<R*>(smem_raw + 16);

  const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qblk = blk - b * n_qblk;
  const int q0 = (qblk * nw + wave) * 16 * QT;  // first query of this wave (uniform)
  const int col = lane & 15, grp = lane >> 4;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const T* Qb = Q + boff;
  const T* Kb = Kx + boff;

  F frag[QT];
  float qn2[QT];  // bf16: |q|^2 of this lane's query
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = min(q0 + 16 * qt + col, N - 1);
    // fp32: a power-of-two scale folds into q exactly (canonical order);
    // bf16: raw scores (the bound is scaled instead)
    if constexpr (SPLIT) {
      qn2[qt] = F::row_norm2(frag[qt].load_q(Qb + static_cast<size_t>(qi) * D, grp));
    } else {
      frag[qt].load_q(Qb + static_cast<size_t>(qi) * D, grp, (EXACT && POW2) ? scale : 1.f);
      if constexpr (!EXACT) qn2[qt] = bf16_frag_norm2<D>(frag[qt]);
      else qn2[qt] = 0.f;
    }
  }
  bool self_r[4];  // element r of a diagonal tile is this lane's self pair
#pragma unroll
  for (int r = 0; r < 4; ++r) self_r[r] = (4 * grp + r == col);

  // packed lane lists of the current segment: NS independent sub-lists per
  // query tile (row r of a tile goes to sub-list r % NS), so consecutive
  // insertions do not wait on each other's results
  float pv[QT][NS][L];
  float rv[QT][L];  // finished segments (multi-segment rows): truncated scores ...
  int ri[QT][L];    // ... and their keys
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int m = 0; m < L; ++m) {
#pragma unroll
      for (int j = 0; j < NS; ++j) pv[qt][j][m] = kMasked;
      rv[qt][m] = kMasked;
      ri[qt][m] = kIdxSentinel;
    }
  float kmax2 = 0.f;
  int segbase = 0;  // first key of the current segment (uniform)
  uint32_t nfmask;  // the field mask's complement in a VGPR (pack_field_u)
  if constexpr (ONESEG) asm volatile("v_mov_b32 %0, %1" : "=v"(nfmask) : "s"(~fm_arg));
  else nfmask = field_nmask_vgpr<FB>();

  for (int c0 = 0; c0 < N; c0 += kc) {
    const int cn = min(kc, N - c0);
    const int cnb = (cn + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
    __syncthreads();
    if constexpr (EXACT) {
      stage_rows<T, D, LDK>(Ks, Kb + static_cast<size_t>(c0) * D, cn, cnb);
      __syncthreads();
    } else {
      if (threadIdx.x == 0) *kmax_slot = 0u;
      float mine;
      if constexpr (SPLIT) {
        bool exact_split = true;  // only the LDS rebuild needs it; the fallback reads global rows
        mine = stage_split<D>(Ks, Kb + static_cast<size_t>(c0) * D, cn, cnb, exact_split);
      } else {
        mine = stage_bf16_norm<D, LDK>(reinterpret_cast<bf16*>(Ks),
                                       reinterpret_cast<const bf16*>(Kb) + static_cast<size_t>(c0) * D,
                                       cn, cnb);
      }
      // one LDS atomic per wave (a per-lane atomic compiles to a 64-step
      // readlane loop); non-negative floats order like their bits
      const float wmax = wave_max_rows(mine);
      __syncthreads();
      if (lane == 0) atomicMax(kmax_slot, __float_as_uint(wmax));
    }
    if (q0 < N) {
      const int kend = c0 + cn;  // rows past the chunk end are zero padding
      for (int kb0 = 0; kb0 < cnb; kb0 += BK) {
        const int kabs = c0 + kb0;
        if (!ONESEG && kabs + BK - segbase > SEGK) {
          flush_packed<QT, NS, L, FB>(pv, rv, ri, segbase, grp);
          segbase = kabs;
        }
        f32x4 s[QT][BT];
        block_scores<F, QT, BT>(frag, Ks, kb0, LDK, lane, s);
        if constexpr (EXACT && !POW2) {
#pragma unroll
          for (int qt = 0; qt < QT; ++qt)
#pragma unroll
            for (int t = 0; t < BT; ++t) s[qt][t] *= scale;
        }
        const uint32_t f0 = static_cast<uint32_t>(kabs - segbase);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
          for (int t = 0; t < BT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              s[qt][t][r] = pack_field_u(s[qt][t][r], f0 + 16u * t + 4u * r, nfmask);
        mask_block<QT, BT>(s, self_r, q0, kabs, kend, grp, kMasked);
#pragma unroll
        for (int t = 0; t < BT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) vinsert<L>(pv[qt][r % NS], s[qt][t][r]);
      }
    }
    if constexpr (!EXACT) {
      __syncthreads();
      kmax2 = fmaxf(kmax2, __uint_as_float(*kmax_slot));
    }
  }
  if (q0 >= N) return;
  // rescoring may read keys from LDS: one chunk holds them all
  const bool lds_all = kc >= N;

  // ---- merge the four lane lists of each query ---------------------------
  // Row swaps give every lane its own and its partner's list; both keep the
  // top L of the union, so after the xor-16 and xor-32 steps the four lanes of
  // a query hold identical lists.
  int cand[QT][L];   // candidate keys (identical on the four lanes; -1: masked)
  float pl[QT][L];   // the merged list: packed (one segment) or truncated (several) values
  if constexpr (!ONESEG) flush_packed<QT, NS, L, FB>(pv, rv, ri, segbase, grp);
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    if constexpr (ONESEG) {
#pragma unroll
      for (int j = 1; j < NS; ++j)
#pragma unroll
        for (int m = 0; m < L; ++m) vinsert<L>(pv[qt][0], pv[qt][j][m]);
      float (&pq)[L] = pv[qt][0];
#pragma unroll
      for (int m = 0; m < L; ++m)
        pq[m] = __uint_as_float(__float_as_uint(pq[m]) | static_cast<uint32_t>(grp));
#pragma unroll
      for (int step = 0; step < 2; ++step) {
        float a[L], o[L];
#pragma unroll
        for (int m = 0; m < L; ++m) {
          const uint32_t x = __float_as_uint(pq[m]);
          const LanePair p = step == 0 ? swap_rows16(x) : swap_rows32(x);
          a[m] = __uint_as_float(p.a);
          o[m] = __uint_as_float(p.b);
        }
#pragma unroll
        for (int m = 0; m < L; ++m) vinsert<L>(a, o[m]);
#pragma unroll
        for (int m = 0; m < L; ++m) pq[m] = a[m];
      }
#pragma unroll
      for (int m = 0; m < L; ++m)
        cand[qt][m] = pq[m] < kMaskedBelow ? -1 : field_key(__float_as_uint(pq[m]) & FM);
#pragma unroll
      for (int m = 0; m < L; ++m) pl[qt][m] = pq[m];
    } else {
#pragma unroll
      for (int step = 0; step < 2; ++step) {
        float av[L], ov[L];
        int ai[L], oi[L];
#pragma unroll
        for (int m = 0; m < L; ++m) {
          const uint32_t xv = __float_as_uint(rv[qt][m]), xi = static_cast<uint32_t>(ri[qt][m]);
          const LanePair pv2 = step == 0 ? swap_rows16(xv) : swap_rows32(xv);
          const LanePair pi2 = step == 0 ? swap_rows16(xi) : swap_rows32(xi);
          av[m] = __uint_as_float(pv2.a);
          ov[m] = __uint_as_float(pv2.b);
          ai[m] = static_cast<int>(pi2.a);
          oi[m] = static_cast<int>(pi2.b);
        }
#pragma unroll
        for (int m = 0; m < L; ++m) topk_insert_lex<L>(av, ai, ov[m], oi[m]);
#pragma unroll
        for (int m = 0; m < L; ++m) {
          rv[qt][m] = av[m];
          ri[qt][m] = ai[m];
        }
      }
#pragma unroll
      for (int m = 0; m < L; ++m) cand[qt][m] = rv[qt][m] < kMaskedBelow ? -1 : ri[qt][m];
#pragma unroll
      for (int m = 0; m < L; ++m) pl[qt][m] = rv[qt][m];
    }
  }

  // ---- prove, rescoring where needed -------------------------------------
  // Entries m of the merged list bound their keys' scores: every key outside
  // the first m+1 entries scores at most hi(entry m), the largest value with
  // that truncation. fp32 (exact scores): the first K (or K+1) entries are the
  // exact top K (K+1) when their truncations stay strictly above the next
  // entry's; the K+1 candidates are rescored exactly (the softmax needs full
  // precision) and the top K taken. bf16 (approximate scores, within E =
  // eps |q| max|k| of the canonical ones): when the entries' truncation
  // intervals widened by E are disjoint down to entry K, the first K are the
  // exact top K in exact order and no rescoring is needed (softmax on the
  // truncated scores); otherwise the K+1 candidates are rescored and sorted,
  // which is exact when the intervals separate at entry K-1/K or K/K+1.
  // Lane row g rescores candidates g, g+4, g+8 from its query fragment (the
  // row is gathered across lane rows) and the key row, from LDS when one
  // chunk holds the whole row.
  float val[QT][K];
  int ix[QT][K];
  bool ok[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int self = q0 + 16 * qt + col;
    bool fast = false;  // bf16: proven and ordered without rescoring
    if constexpr (EXACT) {
      ok[qt] = self >= N || trunc_bits(pl[qt][K], FM) < trunc_bits(pl[qt][K - 1], FM) ||
               trunc_bits(pl[qt][K + 1], FM) < trunc_bits(pl[qt][K], FM);
    } else {
      const float nprod = proof_norm(qn2[qt], kmax2);
      const float e = packed_eps<D>() * nprod;
      bool sep[L - 1];  // entry m's interval (widened by e) lies above entry m+1's
#pragma unroll
      for (int m = 0; m + 1 < L; ++m)
        sep[m] = trunc_floor(pl[qt][m], FM) - e > trunc_ceiling(pl[qt][m + 1], FM) + e;
      bool ordered = true;
#pragma unroll
      for (int m = 0; m + 1 < K; ++m) ordered = ordered && sep[m];
      const bool normal = nprod < kPackedNormLimit;
      fast = !SPLIT && (self >= N || (normal && ordered && sep[K - 1]));
      ok[qt] = self >= N || (normal && (sep[K - 1] || sep[K]));
#pragma unroll
      for (int m = 0; m < K; ++m) {
        val[qt][m] = trunc_bits(pl[qt][m], FM) * scale;
        ix[qt][m] = cand[qt][m];
      }
    }
    if (RESCORE || !__all(fast)) {
      float cv[C];
#pragma unroll
      for (int u = 0; u < (C + 3) / 4; ++u) {
        const int m = 4 * u + grp;
        int c = -1;
#pragma unroll
        for (int mm = 0; mm < C; ++mm)
          if (mm == m) c = cand[qt][mm];
        const int row = min(max(c, 0), N - 1);
        float e;
        if constexpr (SPLIT)
          e = canon_pair<T, D, POW2>(Qb + static_cast<size_t>(min(self, N - 1)) * D,
                                     Kb + static_cast<size_t>(row) * D, scale);
        else
          e = lds_all ? canon_from_frag<T, D, POW2>(frag[qt], Ks + row * LDK, scale)
                      : canon_from_frag<T, D, POW2>(frag[qt], Kb + static_cast<size_t>(row) * D, scale);
        uint32_t g4[4];
        gather_rows(__float_as_uint(c < 0 ? -INFINITY : e), g4);
#pragma unroll
        for (int g = 0; g < 4; ++g)
          if (4 * u + g < C) cv[4 * u + g] = __uint_as_float(g4[g]);
      }
      int ci[C];
#pragma unroll
      for (int m = 0; m < C; ++m) ci[m] = cand[qt][m];
      sort_lex<C>(cv, ci);
      if constexpr (SPLIT) {
        // every key outside the candidates scores at most the (K+2)-th
        // entry's ceiling plus the split error
        const float nprod = proof_norm(qn2[qt], kmax2);
        const float bound = (trunc_ceiling(pl[qt][K + 1], FM) + packed_eps<D>() * nprod) * scale;
        ok[qt] = self >= N || (nprod < kPackedNormLimit && bound < cv[K - 1]);
      }
      if (!fast) {
#pragma unroll
        for (int m = 0; m < K; ++m) {
          val[qt][m] = cv[m];
          ix[qt][m] = ci[m];
        }
      }
    }
  }
  // ---- k-softmax and gathered aggregation --------------------------------
  // Proven tiles finish first; a tile's unproven queries are recomputed
  // exactly at the very end, one at a time across the whole wave, where
  // little else is live, so the rare exact pass does not raise the kernel's
  // register count (and cost waves per SIMD).
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
    if (__all(ok[qt])) finish_tile<T, D, K>(V, O, Idx, b, N, q0 + 16 * qt + col, grp, val[qt], ix[qt]);
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    if (!__all(ok[qt])) {
      // one bit per unproven query (its lane in row 0 stands for it)
      unsigned long long todo = __ballot(grp == 0 && !ok[qt]);
      while (todo != 0ull) {
        const int c = __builtin_ctzll(todo);
        todo &= todo - 1ull;
        float ev[K];
        int ei[K];
        const int qi = q0 + 16 * qt + c;
        // plain rows of the whole row in LDS serve it there (split rows do
        // not); the select makes the row pointer generic (flat loads), which
        // keeps one copy of this rare path
        const bool from_lds = lds_all && !SPLIT;  // uniform
        exact_query_topk_lanes<T, D, K, QT == 1 ? exact_wide_rows<T, D>() : 1>(
            Qb + static_cast<size_t>(qi) * D,
            [&](int j) {
              return from_lds ? reinterpret_cast<const T*>(Ks) + j * LDK : Kb + static_cast<size_t>(j) * D;
            },
            N, qi, scale, lane, ev, ei);
        if (col == c) {
#pragma unroll
          for (int m = 0; m < K; ++m) { val[qt][m] = ev[m]; ix[qt][m] = ei[m]; }
        }
      }
      finish_tile<T, D, K>(V, O, Idx, b, N, q0 + 16 * qt + col, grp, val[qt], ix[qt]);
    }
  }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------

// Independent sub-lists per query tile (row r of a 16-key tile goes to
// sub-list r % NS). Two sub-lists measured no faster than one: the scan is not
// bound by the insertion chains' latency.
constexpr int kPackedSubLists = 1;


// Field mask of a one-segment row of N keys: the fewest bits that name
// every key of the row's whole 16-key tiles (at most 10: N <= 1024). Fewer
// bits truncate scores less, so the proof fails on fewer near-ties; the width
// depends on N alone, never on the key chunk, so a streamed row packs exactly
// as a resident one.
static uint32_t packed_field_mask(int N) {
  const int n16 = (N + 15) / 16 * 16;
  int fb = 4;
  while ((1 << fb) < n16) ++fb;
  return (1u << fb) - 1u;
}

template <typename T, int D, int K, int QT, int NS, int FB, bool ONESEG, bool SPLIT>
static void launch_packed_k(const TopkArgs& a, int kc, int nblocks, int n_qblk, int nw, size_t lds) {
  hipLaunchKernelGGL((topk_packed_kernel<T, D, K, QT, NS, FB, ONESEG, SPLIT>), dim3(nblocks),
                     dim3(64 * nw), lds, static_cast<hipStream_t>(a.stream),
                     static_cast<const T*>(a.q), static_cast<const T*>(a.k),
                     static_cast<const T*>(a.v), static_cast<T*>(a.out), a.idx, a.N, n_qblk, kc,
                     a.scale, nblocks, packed_field_mask(a.N));
}

template <typename T, int D, int K, int QT, bool SPLIT>
static hipError_t launch_packed_shape_q(const TopkArgs& a) {
  constexpr int NS = kPackedSubLists;
  const int per_wave = 16 * QT;
  const int waves = (a.N + per_wave - 1) / per_wave;
  // rows of 512 keys and more: eight waves share one staged key copy (half
  // the staging, and a 57 KB split copy at N = 512 leaves eight waves per CU
  // either way), unless that leaves fewer than two workgroups per CU
  const long wide_groups = static_cast<long>(a.B) * ((a.N + 8 * per_wave - 1) / (8 * per_wave));
  const int maxw = (a.N >= 512 && wide_groups >= 2L * kCUs) ? 8 : 4;
  const int nw = waves >= maxw ? maxw : waves;
  const int qb = per_wave * nw;
  const int n_qblk = (a.N + qb - 1) / qb;
  const int nblocks = a.B * n_qblk;
  const int kc = a.key_chunk;
  const size_t lds = packed_lds_bytes(a.dtype, D, kc, SPLIT);
  // rows of up to 1024 keys are one segment whose field width follows N
  // (packed_field_mask: 8 bits at N = 256, a truncation of 2^-15 of the
  // score), resident or streamed alike
  if constexpr (QT == 1) {  // chosen for rows of up to 1024 keys only
    launch_packed_k<T, D, K, QT, NS, 10, true, SPLIT>(a, kc, nblocks, n_qblk, nw, lds);
    return hipGetLastError();
  } else {
  // a row of up to 1024 keys is one segment whether it is resident or
  // streamed in chunks (the fields hold absolute keys): the lists stay packed
  // across chunks, with no per-chunk flush to (score, key) pairs (fp32 B=256
  // N=1024 in 576-key chunks, k = 1 / 2 / 4: 70.6 / 82.4 / 145.2 -> 65.1 /
  // 72.0 / 90.4 us, identical results)
  if (a.N <= 1024)
    launch_packed_k<T, D, K, QT, NS, 10, true, SPLIT>(a, kc, nblocks, n_qblk, nw, lds);
  else
    launch_packed_k<T, D, K, QT, NS, 10, false, SPLIT>(a, kc, nblocks, n_qblk, nw, lds);
  return hipGetLastError();
  }
}

// Two query tiles per wave halve the per-query staging and merge overhead,
// but a batch too small to give every SIMD a wave that way (B * N / 32 below
// 4 * kCUs) leaves SIMDs idle: one tile per wave then doubles the waves
// (k <= 4, which keeps the build's kernel count down).
template <typename T, int D, int K, bool SPLIT>
static hipError_t launch_packed_shape(const TopkArgs& a) {
  if constexpr (K <= 4) {
    if (a.N <= 1024 && one_query_tile(a.B, a.N)) return launch_packed_shape_q<T, D, K, 1, SPLIT>(a);
  }
  return launch_packed_shape_q<T, D, K, kTopkQueryTiles, SPLIT>(a);
}

template <typename T, int D, bool SPLIT>
static hipError_t launch_packed(const TopkArgs& a) {
  switch (a.topk) {
    case 1: return launch_packed_shape<T, D, 1, SPLIT>(a);
    case 2: return launch_packed_shape<T, D, 2, SPLIT>(a);
    case 3: return launch_packed_shape<T, D, 3, SPLIT>(a);
    case 4: return launch_packed_shape<T, D, 4, SPLIT>(a);
    case 5: return launch_packed_shape<T, D, 5, SPLIT>(a);
    case 6: return launch_packed_shape<T, D, 6, SPLIT>(a);
    case 7: return launch_packed_shape<T, D, 7, SPLIT>(a);
    case 8: return launch_packed_shape<T, D, 8, SPLIT>(a);
  }
  return hipErrorInvalidValue;
}

}  // namespace tarmac
