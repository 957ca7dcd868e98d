// Exact fp32 top-k attention by filter-and-verify.
//
// Same function as topk_small_kernel (scores in the canonical fp32 order,
// top-k with ties to the lower index, k-softmax, gathered aggregation), but
// the N-wide scoring pass runs on bf16 MFMA:
//
//  1. filter: every (query, key) dot is formed from three-way split operands
//     x = x_hi + x_mid + x_lo (bf16 each) with the six products of size
//     >= 2^-16, which approximates the fp32 dot to
//     |a - q.k| <= 2^-21 sum_c |q_c k_c| (representation 2^-22, bf16 MFMA
//     accumulation measured <= 2^-21.9 of the term magnitudes); the canonical
//     fp32 dot is within 2^-20 of q.k. Each lane keeps its best k candidates
//     plus the value of the (k+1)-th, as in the exact kernel.
//  2. verify: the k candidates are rescored in the canonical fp32 order. If
//     the (k+1)-th filtered score plus eps = 2^-18 |q| max_j |k_j| (>= the
//     bounds above, with margin) is strictly below every rescored candidate,
//     no other key can reach the top k, so the candidates ARE the exact top k.
//     Equal filtered scores anywhere in the merged list also fail the proof,
//     which keeps the four lanes of a query on identical candidate lists.
//  3. fallback: a wavefront with any unproven query recomputes its queries
//     exactly (fp32 MFMA over all keys), so the result never depends on the
//     filter -- only the time does (near-ties at the k-th score, e.g.
//     duplicated keys, take the fallback).
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
// results already packed as bf16 pairs.
__device__ __forceinline__ void split3_pair(float x0, float x1, uint32_t& hi, uint32_t& mid,
                                            uint32_t& lo) {
  bf16x2_t h = {static_cast<__bf16>(x0), static_cast<__bf16>(x1)};
  hi = __builtin_bit_cast(uint32_t, h);
  const float r0 = x0 - __uint_as_float(hi << 16), r1 = x1 - __uint_as_float(hi & 0xffff0000u);
  bf16x2_t m = {static_cast<__bf16>(r0), static_cast<__bf16>(r1)};
  mid = __builtin_bit_cast(uint32_t, m);
  const float s0 = r0 - __uint_as_float(mid << 16), s1 = r1 - __uint_as_float(mid & 0xffff0000u);
  bf16x2_t l = {static_cast<__bf16>(s0), static_cast<__bf16>(s1)};
  lo = __builtin_bit_cast(uint32_t, l);
}

// The six products whose size is >= 2^-16 of q.k are formed:
//   hi.hi, hi.mid, mid.hi, mid.mid, hi.lo, lo.hi
// (dropped: mid.lo, lo.mid, lo.lo, each <= 2^-24 |q_c k_c|).
template <int D>
struct SplitFrag;

// d = 16: three 16x16x32 steps, each contraction = two 16-wide products:
//   step 0: A = [k_hi  | k_hi ], B = [q_hi  | q_mid]
//   step 1: A = [k_mid | k_lo ], B = [q_hi  | q_hi ]
//   step 2: A = [k_mid | k_hi ], B = [q_mid | q_lo ]
template <>
struct SplitFrag<16> {
  static constexpr int LDK = 3 * 16 + 8;  // bf16 per LDS row: hi[16] mid[16] lo[16] pad
  static constexpr int NI = 3;
  bf16x8 q[3];
  __device__ __forceinline__ void load_q(const float* qrow, int grp) {
    float x[8];
    ld_f32<8>(x, qrow + 8 * (grp & 1));
    const bool lower = grp < 2;
    uint32_t h[4], m[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split3_pair(x[2 * e], x[2 * e + 1], h[e], m[e], l[e]);
    uint32_t w0[4], w2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w0[e] = lower ? h[e] : m[e];
      w2[e] = lower ? m[e] : l[e];
    }
    q[0] = __builtin_bit_cast(bf16x8, w0);
    q[1] = __builtin_bit_cast(bf16x8, h);
    q[2] = __builtin_bit_cast(bf16x8, w2);
  }
  struct KF { bf16x8 a[3]; };
  __device__ __forceinline__ static KF load_k(const bf16* krow, int grp) {
    const int off = 8 * (grp & 1);
    const bool lower = grp < 2;
    KF f;
    f.a[0] = *reinterpret_cast<const bf16x8*>(krow + off);                         // hi
    f.a[1] = *reinterpret_cast<const bf16x8*>(krow + (lower ? 16 : 32) + off);    // mid | lo
    f.a[2] = *reinterpret_cast<const bf16x8*>(krow + (lower ? 16 : 0) + off);     // mid | hi
    return f;
  }
  __device__ __forceinline__ f32x4 step(const KF& kf, int i, f32x4 acc) const {
    return mfma_bf16_16x16x32(kf.a[i], q[i], acc);
  }
};

// d = 32 (one 32-wide contraction per product) and d = 64 (two halves).
template <int D>
struct SplitFragWide {
  static_assert(D == 32 || D == 64, "split fragment width");
  static constexpr int NH = D / 32;
  static constexpr int LDK = 3 * D + 8;  // hi[D] mid[D] lo[D] pad
  static constexpr int NI = 6 * NH;
  bf16x8 qh[NH], qm[NH], ql[NH];
  __device__ __forceinline__ void load_q(const float* qrow, int grp) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      float x[8];
      ld_f32<8>(x, qrow + 32 * h + 8 * grp);
      uint32_t a[4], b[4], c[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split3_pair(x[2 * e], x[2 * e + 1], a[e], b[e], c[e]);
      qh[h] = __builtin_bit_cast(bf16x8, a);
      qm[h] = __builtin_bit_cast(bf16x8, b);
      ql[h] = __builtin_bit_cast(bf16x8, c);
    }
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
// return this thread's max squared row norm.
template <int D>
__device__ __forceinline__ float stage_split(bf16* lds, const float* src, int rows, int rows_pad) {
  constexpr int VPR = D / 4;  // float4 per row; VPR consecutive threads share a row
  constexpr int LDK = SplitFrag<D>::LDK;
  float mx = 0.f;
  const int total = rows_pad * VPR;
  for (int v = threadIdx.x; v < total; v += blockDim.x) {
    const int row = v / VPR, cv = v - row * VPR;
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    if (row < rows) x = *reinterpret_cast<const f32x4*>(src + static_cast<size_t>(row) * D + 4 * cv);
    uint2 hi, mid, lo;
    split3_pair(x[0], x[1], hi.x, mid.x, lo.x);
    split3_pair(x[2], x[3], hi.y, mid.y, lo.y);
    bf16* dst = lds + row * LDK + 4 * cv;
    *reinterpret_cast<uint2*>(dst) = hi;
    *reinterpret_cast<uint2*>(dst + D) = mid;
    *reinterpret_cast<uint2*>(dst + 2 * D) = lo;
    float n2 = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
#pragma unroll
    for (int o = 1; o < VPR; o <<= 1) n2 += __shfl_xor(n2, o);
    mx = fmaxf(mx, n2);
  }
  return mx;
}

// ---------------------------------------------------------------------------
// exact fp32 pass for one wavefront (fallback): keys straight from HBM/L2
// ---------------------------------------------------------------------------

template <int D, int K, int QT>
__device__ __forceinline__ void exact_wave(const float* __restrict__ Qb, const float* __restrict__ Kb,
                                        int N, int q0, float scale, int lane,
                                        float (&val)[QT][K], int (&ix)[QT][K]) {
  using F = Frag<float, D>;
  constexpr bool POW2 = pow2_scale<D>();
  const int col = lane & 15, grp = lane >> 4;
  F frag[QT];
  int self[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    self[qt] = q0 + 16 * qt + col;
    frag[qt].load_q(Qb + static_cast<size_t>(min(self[qt], N - 1)) * D, grp, POW2 ? scale : 1.f);
#pragma unroll
    for (int m = 0; m < K; ++m) { val[qt][m] = -INFINITY; ix[qt][m] = kIdxSentinel; }
  }
  for (int kb = 0; kb < N; kb += 16) {
    typename F::KF kf;
    const int row = min(kb + col, N - 1);
    ld_f32<F::E>(kf.v, Kb + static_cast<size_t>(row) * D + grp * F::E);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < F::NI; ++i) s = frag[qt].step(kf, i, s);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb + 4 * grp + r;
        float v = POW2 ? s[r] : s[r] * scale;
        if (key >= N || key == self[qt]) v = -INFINITY;
        topk_insert<K>(val[qt], ix[qt], v, key);
      }
    }
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
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

// Canonical fp32 score of one (query row, key row) pair: fmaf chain with
// element kk*(D/4)+t at step t, slot kk (the MFMA chain's order), then scaled.
template <int D, bool POW2>
__device__ __forceinline__ float canon_pair(const float* qrow, const float* krow, float scale) {
  float q[D], k[D];
  ld_f32<D>(q, qrow);
  ld_f32<D>(k, krow);
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < D / 4; ++t)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = kk * (D / 4) + t;
      acc = fmaf(POW2 ? q[c] * scale : q[c], k[c], acc);
    }
  return POW2 ? acc : acc * scale;
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------

constexpr float kFilterEps = 1.0f / 262144.0f;  // 2^-18

template <int D, int K, int QT>
__global__ void __launch_bounds__(256)
topk_filter_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                   const float* __restrict__ V, float* __restrict__ O, int32_t* __restrict__ Idx,
                   int N, int n_qblk, int kc, float scale, int nblocks) {
  using SF = SplitFrag<D>;
  constexpr int LDK = SF::LDK;
  constexpr int EO = D / 4;
  constexpr int BT = kBlockTiles;
  constexpr bool POW2 = pow2_scale<D>();
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16* Ks = reinterpret_cast<bf16*>(smem_raw + 16);
  unsigned* kmax_slot = reinterpret_cast<unsigned*>(smem_raw);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qblk = blk - b * n_qblk;
  const int q0 = (qblk * nw + wave) * 16 * QT;
  const int col = lane & 15, grp = lane >> 4;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const float* Qb = Q + boff;
  const float* Kb = Kx + boff;

  SF frag[QT];
  int self[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    self[qt] = q0 + 16 * qt + col;
    frag[qt].load_q(Qb + static_cast<size_t>(min(self[qt], N - 1)) * D, grp);
  }
  bool self_r[4];  // element r of a diagonal tile is this lane's self pair
#pragma unroll
  for (int r = 0; r < 4; ++r) self_r[r] = (4 * grp + r == col);

  float val[QT][K + 1];
  int ix[QT][K];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int m = 0; m <= K; ++m) val[qt][m] = -INFINITY;
#pragma unroll
    for (int m = 0; m < K; ++m) ix[qt][m] = kIdxSentinel;
  }
  int base = 0;
  float kmax2 = 0.f;

  for (int c0 = 0; c0 < N; c0 += kc) {
    const int cn = min(kc, N - c0);
    const int cnb = (cn + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
    __syncthreads();
    if (threadIdx.x == 0) *kmax_slot = 0u;
    const float mine = stage_split<D>(Ks, Kb + static_cast<size_t>(c0) * D, cn, cnb);
    __syncthreads();
    atomicMax(kmax_slot, __float_as_uint(mine));  // non-negative: bit order is value order
    if (q0 < N) {
      const int kend = c0 + cn;
      for (int kb0 = 0; kb0 < cnb; kb0 += kBlockKeys) {
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
        prepare_block<QT, BT, true>(s, 1.f, self_r, q0, kabs, kend, grp);
        rebase_list<QT, K>(ix, kabs - base);
        base = kabs;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
          for (int t = 0; t < BT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              topk_insert_x<K>(val[qt], ix[qt], s[qt][t][r], 16 * t + r);
      }
    }
    __syncthreads();
    kmax2 = fmaxf(kmax2, __uint_as_float(*kmax_slot));
  }
  if (q0 >= N) return;
  rebase_list<QT, K>(ix, -base);

  // ---- merge the four lane lists of each query --------------------------
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int m = 0; m < K; ++m) ix[qt][m] += 4 * grp;
#pragma unroll
    for (int step = 16; step <= 32; step <<= 1) {
      float pv[K + 1];
      int pi[K];
#pragma unroll
      for (int m = 0; m <= K; ++m) pv[m] = __shfl_xor(val[qt][m], step);
#pragma unroll
      for (int m = 0; m < K; ++m) pi[m] = __shfl_xor(ix[qt][m], step);
#pragma unroll
      for (int m = 0; m < K; ++m) topk_insert_x<K>(val[qt], ix[qt], pv[m], pi[m]);
      topk_insert_x<K>(val[qt], ix[qt], pv[K], kIdxSentinel);
    }
  }

  // ---- verify: rescore the candidates exactly ---------------------------
  const float kmax = sqrtf(kmax2);
  float ex[QT][K];
  bool ok = true;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = min(self[qt], N - 1);
    const float* qrow = Qb + static_cast<size_t>(qi) * D;
    // lane group g rescores candidates g, g+4, ...
    float mine[(K + 3) / 4];
#pragma unroll
    for (int u = 0; u < (K + 3) / 4; ++u) {
      const int m = 4 * u + grp;
      int cand = kIdxSentinel;
#pragma unroll
      for (int mm = 0; mm < K; ++mm)
        if (mm == m) cand = ix[qt][mm];
      const int row = min(max(cand, 0), N - 1);
      mine[u] = canon_pair<D, POW2>(qrow, Kb + static_cast<size_t>(row) * D, scale);
    }
    float qn2 = 0.f;
    {
      float qf[D];
      ld_f32<D>(qf, qrow);
#pragma unroll
      for (int c = 0; c < D; ++c) qn2 = fmaf(qf[c], qf[c], qn2);
    }
    float worst = INFINITY;
#pragma unroll
    for (int m = 0; m < K; ++m) {
      ex[qt][m] = __shfl(mine[m / 4], col + 16 * (m % 4));
      worst = fminf(worst, ex[qt][m]);
    }
    const float bound = (val[qt][K] + kFilterEps * sqrtf(qn2) * kmax) * scale;
    bool distinct = true;  // strictly decreasing filtered values: the lane lists agree
#pragma unroll
    for (int m = 0; m < K; ++m) distinct = distinct && val[qt][m] > val[qt][m + 1];
    ok = ok && (self[qt] >= N || (distinct && bound < worst));
  }

  if (__all(ok)) {
    // the candidates are the exact top k: order them by exact score
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float sv[K];
      int si[K];
#pragma unroll
      for (int m = 0; m < K; ++m) { sv[m] = -INFINITY; si[m] = kIdxSentinel; }
#pragma unroll
      for (int m = 0; m < K; ++m) topk_insert_lex<K>(sv, si, ex[qt][m], ix[qt][m]);
#pragma unroll
      for (int m = 0; m < K; ++m) { val[qt][m] = sv[m]; ix[qt][m] = si[m]; }
    }
  } else {
    float ev[QT][K];
    int ei[QT][K];
    exact_wave<D, K, QT>(Qb, Kb, N, q0, scale, lane, ev, ei);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int m = 0; m < K; ++m) { val[qt][m] = ev[qt][m]; ix[qt][m] = ei[qt][m]; }
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
      ld_f32<EO>(vr, V + boff + static_cast<size_t>(row) * D + grp * EO);
#pragma unroll
      for (int c = 0; c < EO; ++c) acc[c] = fmaf(w, vr[c], acc[c]);
    }
    const float inv = 1.f / den;
#pragma unroll
    for (int c = 0; c < EO; ++c) acc[c] *= inv;
    st_f32<EO>(O + boff + static_cast<size_t>(qi) * D + grp * EO, acc);
    if (Idx != nullptr && grp == 0) {
      int32_t* dst = Idx + (static_cast<size_t>(b) * N + qi) * K;
#pragma unroll
      for (int m = 0; m < K; ++m) dst[m] = ix[qt][m];
    }
  }
}

size_t topk_filter_lds_bytes(int d, int kc) {
  const int kcb = (kc + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
  return 16 + static_cast<size_t>(kcb) * (3 * d + 8) * sizeof(bf16);
}

template <int D>
static hipError_t launch_filter(const TopkArgs& a, int kc) {
  constexpr int QT = kTopkQueryTiles;
  const int per_wave = 16 * QT;
  const int waves = (a.N + per_wave - 1) / per_wave;
  const int nw = waves >= 4 ? 4 : waves;
  const int qb = per_wave * nw;
  const int n_qblk = (a.N + qb - 1) / qb;
  const int nblocks = a.B * n_qblk;
  const size_t lds = topk_filter_lds_bytes(D, kc);
  const float* q = static_cast<const float*>(a.q);
  const float* k = static_cast<const float*>(a.k);
  const float* v = static_cast<const float*>(a.v);
  float* o = static_cast<float*>(a.out);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
#define TARMAC_FILTER_CASE(KK)                                                                  \
  case KK:                                                                                      \
    hipLaunchKernelGGL((topk_filter_kernel<D, KK, QT>), dim3(nblocks), dim3(64 * nw), lds, st, \
                       q, k, v, o, a.idx, a.N, n_qblk, kc, a.scale, nblocks);                  \
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

bool topk_filter_supported(int dtype, int d, int topk) {
  return dtype == kF32 && (d == 16 || d == 32 || d == 64) && topk >= 1 && topk <= kTopkSmallMax;
}

hipError_t run_topk_filter(const TopkArgs& a) {
  switch (a.d) {
    case 16: return launch_filter<16>(a, a.key_chunk);
    case 32: return launch_filter<32>(a, a.key_chunk);
    case 64: return launch_filter<64>(a, a.key_chunk);
  }
  return hipErrorInvalidValue;
}

}  // namespace tarmac
