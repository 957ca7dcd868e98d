// Dense attention with the self-diagonal masked, flash-style: online softmax
// over key blocks, nothing but q, k, v and out touches HBM.
//
// Reference behaviour: src/kernels/fused_dense_attention.py:38-152
// (_flash_dense_kernel / fused_dense_attention) and the composed dense path
// scripts/bench_attention_core.py:74-82 (softmax(QK^T/sqrt(d), diag=-inf) V).
//
// Mapping (one wave = 16 queries, lane l owns query l%16):
//   S^T tile  = K_tile * Q_tile^T        (MFMA; lane l gets keys 4*(l/16)+r)
//   O^T      += V^T_tile * P^T_tile      (MFMA; contraction slot kk of step u
//                                         is key 4*kk+u, so lane l's B operand
//                                         is its own probability p[u] -- no
//                                         cross-lane data movement)
// V is staged transposed in LDS so the A operand of the PV product is a
// contiguous read. A row staged in one chunk (the default up to the LDS
// budget) takes a fixed exponent offset per query, c |q| max_j |k_j|, so a
// score costs one exp2 and no maximum: fp32 products start at -offset and
// return the exponent itself (q pre-multiplied by c = scale*log2(e)), bf16
// scores stay raw and take fma(s, c, -offset). A row whose bound sits too far
// above its true maximum (its softmax sum below 2^-64) is run again with the
// online softmax that multi-chunk rows use: per 64-key block a maximum shared
// by the 4 lanes of a query with two row swaps (VALU, no LDS), the running
// offset raised -- rescaling the query's sum and accumulator -- only when a
// block's maximum exceeds it by more than 2^8. bf16 probabilities are rounded
// to bf16 for the PV product, and the row sum adds exactly those weights on
// the matrix core (an all-ones A operand); fp32 sums stay per lane and are
// combined once at the end.
#include "frag.hpp"
#include "select.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kDenseBlockTiles = 4;  // 64 keys per score block
constexpr int kDenseQueryTiles = 2;  // 16-query tiles per wavefront

template <typename T, int D>
struct PvOperand;

// fp32: O^T block h (channels 16h..16h+15) += V^T(16 x 4 keys) * P^T(4 keys x 16 q),
// four steps per 16-key tile. The V^T fragment of a (tile, h) is read once
// and used by every query tile.
template <int D>
struct PvOperand<float, D> {
  static constexpr int NH = (D + 15) / 16;  // output blocks of 16 channels
  static constexpr int CP = NH * 16;        // padded channel count in LDS
  static constexpr int TILES = 1;           // 16-key tiles per step
  template <int QT>
  __device__ __forceinline__ static void pv_step(f32x4 (&acc)[QT][NH], const float* Vt, int ldv,
                                                 int kb, int lane, const float (&p)[QT][TILES][4]) {
    const int col = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const f32x4 vv = *reinterpret_cast<const f32x4*>(Vt + (16 * h + col) * ldv + kb + 4 * grp);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) acc[qt][h] = mfma_f32_16x16x4(vv[u], p[qt][0][u], acc[qt][h]);
    }
  }
};

// Four probabilities as bf16 (round to nearest even, the rounding of
// Tensor.to(torch.bfloat16)), two hardware conversions.
__device__ __forceinline__ bf16x8 pack_p_pair(const float (&a)[4], const float (&b)[4]) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    bf16x2_t lo = {static_cast<__bf16>(a[2 * i]), static_cast<__bf16>(a[2 * i + 1])};
    bf16x2_t hi = {static_cast<__bf16>(b[2 * i]), static_cast<__bf16>(b[2 * i + 1])};
    w[i] = __builtin_bit_cast(uint32_t, lo);
    w[2 + i] = __builtin_bit_cast(uint32_t, hi);
  }
  return __builtin_bit_cast(bf16x8, w);
}

// bf16: one 16x16x32 MFMA per output block and pair of 16-key tiles. The
// contraction index j = 8 (l/16) + e of lane l maps to key 4 (l/16) + e of the
// first tile (e < 4) and of the second (e >= 4): the B operand is the lane's
// own eight probabilities, the A operand two 8-byte V^T reads.
template <int D>
struct PvOperand<bf16, D> {
  static constexpr int NH = D / 16;
  static constexpr int CP = NH * 16;
  static constexpr int TILES = 2;  // 16-key tiles per step
  // pb: each query tile's eight probabilities, packed (pack_p_pair)
  template <int QT>
  __device__ __forceinline__ static void pv_step_packed(f32x4 (&acc)[QT][NH], const bf16* Vt,
                                                        int ldv, int kb, int lane,
                                                        const bf16x8 (&pb)[QT]) {
    const int col = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const bf16* r = Vt + (16 * h + col) * ldv + kb + 4 * grp;
      uint2 w[2] = {*reinterpret_cast<const uint2*>(r), *reinterpret_cast<const uint2*>(r + 16)};
      const bf16x8 vv = __builtin_bit_cast(bf16x8, w);
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) acc[qt][h] = mfma_bf16_16x16x32(vv, pb[qt], acc[qt][h]);
    }
  }
};

// Row sum of eight bf16 probabilities (the PV operand) into an fp32 sum: four
// v_dot2 against (1, 1). The softmax then normalises by the sum of exactly
// the weights the PV product uses.
__device__ __forceinline__ float sum_bf16x8(bf16x8 p, float acc) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const uint4 w = __builtin_bit_cast(uint4, p);
  const bf16x2_t one = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z), one, acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w), one, acc, false);
}

// Maximum over the four lanes of a query (lanes l, l + 16, l + 32, l + 48):
// two row swaps, VALU only.
__device__ __forceinline__ float query_max4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = max_plain(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_plain(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Softmax terms are 2^(c s - off). Where the whole row is staged at once
// (one key chunk), off is fixed per query before the first block:
// off = c |q| max_j |k_j| >= c s for every key (Cauchy-Schwarz), so no term
// exceeds 1 and a block needs no maximum. The bound can sit far above the
// row's true maximum; terms then shrink by 2^-(gap) and the query's sum shows
// it: a sum below 2^-64 (a gap of more than 64 - log2 N) makes the wave run
// the row again with the running maximum below, the path every multi-chunk
// row takes. With the sum at or above 2^-64 the largest term is at least
// 2^-74 (N <= 1024 keys in one chunk), so only terms below 2^-52 of it can
// leave the fp32 (and bf16) normal range.
// The running maximum of c s is only raised when a block's maximum exceeds it
// by more than 2^kDenseLag: terms then stay below 2^kDenseLag (no overflow,
// no loss of precision in fp32), and after the first block a raise -- a
// rescale of the query's sum and accumulator -- is rare.
constexpr float kDenseLag = 8.f;
constexpr float kDenseTinySum = 0x1p-64f;

// All-ones bf16 A operand (0x3f80 = 1.0).
constexpr bf16x8 kOnesBf16x8 = {1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0};

// The query's softmax sum: fp32 lanes hold a quarter each (element 0), bf16
// lanes the whole sum (every element).
template <typename T>
__device__ __forceinline__ float row_total(f32x4 l) {
  if constexpr (sizeof(T) == 2) return l[0];
  float t = l[0] + __shfl_xor(l[0], 16);
  return t + __shfl_xor(t, 32);
}

// Fixed-offset exponents (fp32) of QT query tiles against BT key tiles: the
// fragments hold c q, and every MFMA chain starts at -off, so the product
// returns c s - off itself -- no VALU between the product and exp2. (bf16
// would need c q as a bf16 pair, twice the products: measured slower than the
// fma it saves.)
template <typename F, int QT, int BT, typename T>
__device__ __forceinline__ void block_exponents(const F (&frag)[QT], const T* Ks, int kb, int lane,
                                                const float (&neg)[QT], f32x4 (&s)[QT][BT]) {
  const int col = lane & 15, grp = lane >> 4;
  typename F::KF kf[BT];
#pragma unroll
  for (int t = 0; t < BT; ++t) kf[t] = F::load_k(Ks + (kb + 16 * t + col) * F::LDK, grp);
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int t = 0; t < BT; ++t) s[qt][t] = f32x4{neg[qt], neg[qt], neg[qt], neg[qt]};
#pragma unroll
  for (int i = 0; i < F::NI; ++i)
#pragma unroll
    for (int t = 0; t < BT; ++t)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) s[qt][t] = frag[qt].step(kf[t], i, s[qt][t]);
}

// The block loop over one staged chunk (rows [0, cnp) of Ks / Vt, keys
// c0 + row): scores, the self and chunk-end masks, exponents, row sums and
// the P.V product. ONLINE: off follows the running maximum; otherwise off
// is the fixed per-query bound.
template <bool ONLINE, typename T, int D, int QT>
__device__ __forceinline__ void dense_blocks(const Frag<T, D> (&frag)[QT], const T* Ks, const T* Vt,
                                             int ldv, int c0, int cn, int cnp, int q0,
                                             const bool (&self_r)[4], int lane, int grp, float post,
                                             f32x4 (&acc)[QT][PvOperand<T, D>::NH],
                                             float (&off)[QT], f32x4 (&l_run)[QT]) {
  using F = Frag<T, D>;
  using PV = PvOperand<T, D>;
  constexpr int LDK = F::LDK;
  constexpr int NH = PV::NH;
  constexpr int BT = kDenseBlockTiles;
  constexpr int BK = 16 * BT;
  const int kend = c0 + cn;  // rows past the chunk end are zero padding
  float neg[QT];             // the exponent's offset
  if constexpr (!ONLINE) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) neg[qt] = -off[qt];
  }
  for (int kb0 = 0; kb0 < cnp; kb0 += BK) {
    f32x4 s[QT][BT];
    constexpr bool FOLDED = !ONLINE && sizeof(T) == 4;  // s is already c s - off
    if constexpr (FOLDED) block_exponents<F, QT, BT>(frag, Ks, kb0, lane, neg, s);
    else block_scores<F, QT, BT>(frag, Ks, kb0, LDK, lane, s);
    const int kabs = c0 + kb0;
    // the self pair (one select per element of a diagonal tile, on the
    // loop-invariant lane predicates) and keys past the chunk end
    mask_block<QT, BT>(s, self_r, q0, kabs, kend, grp, -INFINITY);
    if constexpr (ONLINE) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        float mloc = -INFINITY;
#pragma unroll
        for (int t = 0; t < BT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, s[qt][t][r]);
        const float m_blk = query_max4(mloc) * post;
        if (m_blk > off[qt] + kDenseLag) {  // rare after the first block
          const float alpha = fast_exp2(off[qt] - m_blk);  // 0 while nothing has been seen
          l_run[qt] *= alpha;
#pragma unroll
          for (int h = 0; h < NH; ++h) acc[qt][h] *= alpha;
          off[qt] = m_blk;
        }
        neg[qt] = off[qt] == -INFINITY ? 0.f : -off[qt];  // a block of masked keys only
      }
    }
    constexpr int TS = PV::TILES;
    static_assert(BT % TS == 0, "whole PV steps per block");
#pragma unroll
    for (int t0 = 0; t0 < BT; t0 += TS) {
      float p[QT][TS][4];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int t = 0; t < TS; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            p[qt][t][r] = FOLDED ? fast_exp2(s[qt][t0 + t][r])
                                 : fast_exp2(fmaf(s[qt][t0 + t][r], post, neg[qt]));
      if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
          for (int t = 0; t < TS; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) l_run[qt][0] += p[qt][t][r];
        PV::template pv_step<QT>(acc, Vt, ldv, kb0 + 16 * t0, lane, p);
      } else {
        bf16x8 pb[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          pb[qt] = pack_p_pair(p[qt][0], p[qt][1]);
          // the row sum on the matrix core: an all-ones A operand adds the
          // step's 32 weights of the query into every output element
          l_run[qt] = mfma_bf16_16x16x32(kOnesBf16x8, pb[qt], l_run[qt]);
        }
        PV::template pv_step_packed<QT>(acc, Vt, ldv, kb0 + 16 * t0, lane, pb);
      }
    }
  }
}

// A fixed-offset row whose softmax sum is below 2^-64 (the bound sat too far
// above its maximum), above 2N (each term is at most 1) or not a number must
// run again with the online softmax.
template <typename T, int QT>
__device__ __forceinline__ bool sum_out_of_range(const f32x4 (&l_run)[QT], int N) {
  bool out = false;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float l_tot = row_total<T>(l_run[qt]);
    out |= !(l_tot >= kDenseTinySum && l_tot <= 2.f * static_cast<float>(N));
  }
  return out;
}

// Sum of squares of LDS row `row` (D elements, 16-byte aligned).
template <typename T, int D>
__device__ __forceinline__ float row_sumsq(const T* row) {
  constexpr int VE = 16 / sizeof(T);
  float a = 0.f;
#pragma unroll
  for (int c = 0; c < D / VE; ++c) {
    const uint4 w = *reinterpret_cast<const uint4*>(row + c * VE);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (sizeof(T) == 4) {
        const float x = __uint_as_float(ww[e]);
        a = fmaf(x, x, a);
      } else {
        a = dot2_bf16(ww[e], ww[e], a);
      }
    }
  }
  return a;
}

template <typename T, int D, int QT>
__global__ void __launch_bounds__(256)
dense_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
             T* __restrict__ O, float* __restrict__ lse, int N, int n_qblk, int kc, float scale,
             int nblocks) {
  using F = Frag<T, D>;
  using PV = PvOperand<T, D>;
  constexpr int LDK = F::LDK;
  constexpr int NH = PV::NH;
  constexpr int BK = 16 * kDenseBlockTiles;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int kcp = (kc + BK - 1) / BK * BK;  // chunk rows padded to whole blocks
  const int ldv = kcp + 4;
  T* Ks = reinterpret_cast<T*>(smem_raw);
  T* Vt = Ks + static_cast<size_t>(kcp) * LDK;
  // the row's max |k|^2 (bits of a non-negative float), after V^T
  uint32_t* kmax_slot = reinterpret_cast<uint32_t*>(Vt + static_cast<size_t>(PV::CP) * ldv);

  // the wave index in an SGPR, so tile tests on q0 are scalar
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qblk = blk - b * n_qblk;
  const int q0 = (qblk * nw + wave) * 16 * QT;
  const int col = lane & 15, grp = lane >> 4;
  const size_t boff = static_cast<size_t>(b) * N * D;

  // fp32 scores come out pre-multiplied by scale*log2(e), ready for exp2;
  // bf16 scores are scaled inside the exponent (the factor is not exact in bf16).
  F frag[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = q0 + 16 * qt + col;
    frag[qt].load_q(Q + boff + static_cast<size_t>(min(qi, N - 1)) * D, grp,
                    sizeof(T) == 4 ? scale * kLog2e : 1.f);
  }
  // exponent factor c: 1 for fp32 (folded into q), scale*log2(e) for bf16
  const float post = (sizeof(T) == 4) ? 1.f : scale * kLog2e;
  bool self_r[4];  // element r of a diagonal tile is this lane's self pair
#pragma unroll
  for (int r = 0; r < 4; ++r) self_r[r] = (4 * grp + r == col);

  f32x4 acc[QT][NH];
  float off[QT];
  f32x4 l_run[QT];  // fp32: element 0, this lane's share; bf16: the whole sum
  auto reset = [&]() {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
      for (int h = 0; h < NH; ++h) acc[qt][h] = f32x4{0.f, 0.f, 0.f, 0.f};
      off[qt] = -INFINITY;
      l_run[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  reset();

  if (kc >= N) {
    // the whole row in one chunk: fixed offsets from the row's max |k|
    if (threadIdx.x == 0) *kmax_slot = 0u;
    const int cnp = (N + BK - 1) / BK * BK;
    __syncthreads();
    stage_kv<T, D, LDK, PV::CP>(Ks, Vt, ldv, Kx + boff, V + boff, N, cnp);
    __syncthreads();
    float kn2 = 0.f;  // fmaxf drops a NaN row; its scores fail the check below
    for (int r = threadIdx.x; r < N; r += blockDim.x) kn2 = fmaxf(kn2, row_sumsq<T, D>(Ks + r * LDK));
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) kn2 = fmaxf(kn2, __shfl_xor(kn2, m));
    if (lane == 0) atomicMax(kmax_slot, __float_as_uint(kn2));
    __syncthreads();
    if (q0 >= N) return;
    const float kmax2 = __uint_as_float(*kmax_slot);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float qn2 = frag[qt].sumsq();
      qn2 += __shfl_xor(qn2, 16);
      qn2 += __shfl_xor(qn2, 32);
      off[qt] = post * __builtin_amdgcn_sqrtf(qn2 * kmax2);  // v_sqrt_f32, 1 ulp
    }
    dense_blocks<false, T, D, QT>(frag, Ks, Vt, ldv, 0, N, cnp, q0, self_r, lane, grp, post, acc,
                                  off, l_run);
    if (__any(sum_out_of_range<T, QT>(l_run, N))) {  // uniform: the wave runs the row again, online
      reset();
      dense_blocks<true, T, D, QT>(frag, Ks, Vt, ldv, 0, N, cnp, q0, self_r, lane, grp, post, acc,
                                   off, l_run);
    }
  } else {
    // several chunks (d <= 32): the offset is the bound over the keys staged
    // so far, raised with the chunk that holds a longer key (an exact 2^-x
    // rescale of the query's sum and accumulator, before the chunk's first
    // block); a workgroup with a sum out of range runs every chunk again,
    // online. At d = 64 the per-chunk bound costs more than the running
    // maximum it removes (fp32 B=256 N=512: 156 -> 167 us), so those rows run
    // online from the start.
    bool online = D > 32;
    if constexpr (D <= 32) {
      uint32_t* rerun = kmax_slot + 1;
      if (threadIdx.x == 0) {
        *kmax_slot = 0u;
        *rerun = 0u;
      }
      float qn2[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        qn2[qt] = frag[qt].sumsq();
        qn2[qt] += __shfl_xor(qn2[qt], 16);
        qn2[qt] += __shfl_xor(qn2[qt], 32);
      }
      for (int c0 = 0; c0 < N; c0 += kc) {
        const int cn = min(kc, N - c0);
        const int cnp = (cn + BK - 1) / BK * BK;
        __syncthreads();
        stage_kv<T, D, LDK, PV::CP>(Ks, Vt, ldv, Kx + boff + static_cast<size_t>(c0) * D,
                                    V + boff + static_cast<size_t>(c0) * D, cn, cnp);
        __syncthreads();
        float kn2 = 0.f;  // the running maximum in LDS only grows
        for (int r = threadIdx.x; r < cn; r += blockDim.x)
          kn2 = fmaxf(kn2, row_sumsq<T, D>(Ks + r * LDK));
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) kn2 = fmaxf(kn2, __shfl_xor(kn2, m));
        if (lane == 0) atomicMax(kmax_slot, __float_as_uint(kn2));
        __syncthreads();
        if (q0 >= N) continue;
        const float kmax2 = __uint_as_float(*kmax_slot);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const float o = post * __builtin_amdgcn_sqrtf(qn2[qt] * kmax2);
          if (o > off[qt]) {  // first chunk: off = -inf, alpha = 0 on zeros
            const float alpha = fast_exp2(off[qt] - o);
            l_run[qt] *= alpha;
#pragma unroll
            for (int h = 0; h < NH; ++h) acc[qt][h] *= alpha;
            off[qt] = o;
          }
        }
        dense_blocks<false, T, D, QT>(frag, Ks, Vt, ldv, c0, cn, cnp, q0, self_r, lane, grp, post,
                                      acc, off, l_run);
      }
      if (q0 < N && __any(sum_out_of_range<T, QT>(l_run, N)) && lane == 0) atomicOr(rerun, 1u);
      __syncthreads();
      online = *rerun != 0u;  // uniform across the workgroup
    }
    if (online) {
      reset();
      for (int c0 = 0; c0 < N; c0 += kc) {
        const int cn = min(kc, N - c0);
        const int cnp = (cn + BK - 1) / BK * BK;
        __syncthreads();
        // K and V^T in one pass of loads; bf16 rows transpose four at a time
        // (8-byte stores instead of 2-byte ones), fp32 keeps one store per
        // element, measured no slower
        stage_kv<T, D, LDK, PV::CP>(Ks, Vt, ldv, Kx + boff + static_cast<size_t>(c0) * D,
                                    V + boff + static_cast<size_t>(c0) * D, cn, cnp);
        __syncthreads();
        if (q0 >= N) continue;
        dense_blocks<true, T, D, QT>(frag, Ks, Vt, ldv, c0, cn, cnp, q0, self_r, lane, grp, post,
                                     acc, off, l_run);
      }
    }
    if (q0 >= N) return;
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float l_tot = row_total<T>(l_run[qt]);
    const int qi = q0 + 16 * qt + col;
    if (qi >= N) continue;
    // log2-domain logsumexp of the scaled scores, for the backward pass
    if (lse != nullptr && grp == 0) lse[static_cast<size_t>(b) * 2 * N + qi] = off[qt] + log2f(l_tot);
    // lane l holds O^T[c = 16h + 4*(l/16) + r][q = l%16]; one reciprocal
    // per row instead of a division per channel
    const float inv = __builtin_amdgcn_rcpf(l_tot);  // v_rcp_f32, 1 ulp
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const int cbase = 16 * h + 4 * grp;
      if (cbase < D) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = acc[qt][h][r] * inv;
        st_row<T, 4>(O + boff + static_cast<size_t>(qi) * D + cbase, o);
      }
    }
  }
}

// fp32, N <= 64: no LDS, no barrier. Every MFMA operand of a wave (its query
// fragments, the 16-key K fragments, the V^T fragments of the P.V product) is
// loaded from global memory at the start, so the row's q, k and v arrive in
// one memory round trip (the LDS kernel stages K, then V, then waits at a
// barrier). A K fragment is 16 rows x 64 B (coalesced); a V^T fragment element
// is read per lane, 16 consecutive channels per row. One softmax over the
// whole row; for N <= 64 this is the LDS kernel's arithmetic, operation for
// operation (one 64-key block), so the two give identical results.
template <int D, int QT, int NT>
__global__ void __launch_bounds__(64)
dense_reg_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                 const float* __restrict__ V, float* __restrict__ O, float* __restrict__ lse, int N,
                 int n_qblk, float scale, int nblocks) {
  using F = Frag<float, D>;
  constexpr int NH = PvOperand<float, D>::NH;
  const int lane = threadIdx.x;
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qb = blk - b * n_qblk;
  const int q0 = qb * 16 * QT;
  const int col = lane & 15, grp = lane >> 4;
  const size_t boff = static_cast<size_t>(b) * N * D;

  F frag[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
    frag[qt].load_q(Q + boff + static_cast<size_t>(min(q0 + 16 * qt + col, N - 1)) * D, grp,
                    scale * kLog2e);
  typename F::KF kf[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    kf[t] = F::load_k(Kx + boff + static_cast<size_t>(min(16 * t + col, N - 1)) * D, grp);
  f32x4 vv[NT][NH];  // V^T fragment: element u = V[16t + 4 grp + u][16h + col]
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int row = 16 * t + 4 * grp + u, c = 16 * h + col;
        vv[t][h][u] = (row < N && c < D) ? V[boff + static_cast<size_t>(row) * D + c] : 0.f;
      }

  f32x4 s[QT][NT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < F::NI; ++i) acc = frag[qt].step(kf[t], i, acc);
      if (16 * t + 16 > N || 16 * t == q0 + 16 * qt) {  // wave-uniform: the tail or the diagonal tile
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = 16 * t + 4 * grp + r;
          if (key >= N || key == q0 + 16 * qt + col) acc[r] = -INFINITY;
        }
      }
      s[qt][t] = acc;
    }
  f32x4 acc[QT][NH];
  float m_row[QT], l[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    float m = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) m = fmaxf(m, s[qt][t][r]);
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    m_row[qt] = m;
    const float neg = -(m == -INFINITY ? 0.f : m);
    l[qt] = 0.f;
#pragma unroll
    for (int h = 0; h < NH; ++h) acc[qt][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[qt][t][r] = fast_exp2(fmaf(s[qt][t][r], 1.f, neg));
        l[qt] += s[qt][t][r];
      }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
          acc[qt][h] = mfma_f32_16x16x4(vv[t][h][u], s[qt][t][u], acc[qt][h]);
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    float l_tot = l[qt] + __shfl_xor(l[qt], 16);
    l_tot += __shfl_xor(l_tot, 32);
    const int qi = q0 + 16 * qt + col;
    if (qi >= N) continue;
    if (lse != nullptr && grp == 0)
      lse[static_cast<size_t>(b) * 2 * N + qi] = m_row[qt] + log2f(l_tot);
    const float inv = 1.f / l_tot;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const int cbase = 16 * h + 4 * grp;
      if (cbase < D) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = acc[qt][h][r] * inv;
        st_row<float, 4>(O + boff + static_cast<size_t>(qi) * D + cbase, o);
      }
    }
  }
}

template <int D, int NT>
static hipError_t launch_dense_reg(const DenseArgs& a) {
  constexpr int QT = 2;
  const int n_qblk = (a.N + 16 * QT - 1) / (16 * QT);
  const int nblocks = a.B * n_qblk;
  hipLaunchKernelGGL((dense_reg_kernel<D, QT, NT>), dim3(nblocks), dim3(64), 0,
                     static_cast<hipStream_t>(a.stream), static_cast<const float*>(a.q),
                     static_cast<const float*>(a.k), static_cast<const float*>(a.v),
                     static_cast<float*>(a.out), a.stats, a.N, n_qblk, a.scale, nblocks);
  return hipGetLastError();
}

// Register kernel for fp32 rows of up to 64 keys (32 at d = 64, where 64
// keys of K and V fragments would not leave registers for two query tiles).
// B=1024 d=16, rocprof average: N = 32 5.7 -> 3.5 us, N = 64 7.1 -> 6.5 us.
template <int D>
static bool dense_reg(const DenseArgs& a, hipError_t* e) {
  if constexpr (D > 64) {
    return false;  // d = 128 rows take the LDS kernel
  } else {
    if (a.N > (D <= 32 ? 64 : 32) || a.key_chunk < a.N) return false;  // an explicit smaller chunk keeps LDS
    switch ((a.N + 15) / 16) {
      case 1: *e = launch_dense_reg<D, 1>(a); return true;
      case 2: *e = launch_dense_reg<D, 2>(a); return true;
      case 3: *e = launch_dense_reg<D, 3>(a); return true;
      case 4: if constexpr (D <= 32) { *e = launch_dense_reg<D, 4>(a); return true; }
    }
    return false;
  }
}

template <typename T, int D, int QT>
static hipError_t launch_dense_q(const DenseArgs& a) {
  const int per_wave = 16 * QT;
  const int waves = (a.N + per_wave - 1) / per_wave;
  const int nw = waves >= 4 ? 4 : waves;
  const int qb = per_wave * nw;
  const int n_qblk = (a.N + qb - 1) / qb;
  const int nblocks = a.B * n_qblk;
  const size_t lds = dense_lds_bytes(a.dtype, a.d, a.key_chunk);
  hipLaunchKernelGGL((dense_kernel<T, D, QT>), dim3(nblocks), dim3(64 * nw), lds,
                     static_cast<hipStream_t>(a.stream), static_cast<const T*>(a.q),
                     static_cast<const T*>(a.k), static_cast<const T*>(a.v), static_cast<T*>(a.out),
                     a.stats, a.N, n_qblk, a.key_chunk, a.scale, nblocks);
  return hipGetLastError();
}

// A batch too small to give every SIMD a wave at two query tiles per wave
// (B * N / 32 below 4 * kCUs) takes one tile per wave: twice the waves.
// bf16 at d = 16 and 32 on rows of 256 keys or more staged whole, with at
// least four (d = 32: eight) waves per SIMD at four tiles per wave, takes
// four tiles: the staging, bound and epilogue work of a wave is spread over
// twice the scores (B=4096, N=256: d = 16 55.5 -> 51 us, d = 32 76 -> 68.5).
template <typename T, int D>
static hipError_t launch_dense(const DenseArgs& a) {
  if constexpr (sizeof(T) == 4) {
    hipError_t e;
    if (dense_reg<D>(a, &e)) return e;
  }
  if (one_query_tile(a.B, a.N)) return launch_dense_q<T, D, 1>(a);
  if constexpr (sizeof(T) == 2 && D <= 32) {
    if (query_tiles_mode() == kTilesAuto && a.N >= 256 && a.key_chunk >= a.N &&
        static_cast<long>(a.B) * a.N >= (D == 16 ? 4L : 8L) * 64 * 4 * kCUs)
      return launch_dense_q<T, D, 4>(a);
  }
  return launch_dense_q<T, D, kDenseQueryTiles>(a);
}

size_t dense_lds_bytes(int dtype, int d, int kc) {
  const int bk = 16 * kDenseBlockTiles;
  const int kcp = (kc + bk - 1) / bk * bk;
  const int cp = (d + 15) / 16 * 16;
  const size_t es = dtype == kF32 ? 4 : 2;
  const int ldk = dtype == kF32 ? d + 4 : d + 8;
  // K, V^T, and 16 bytes for the row's max |k|^2
  return (static_cast<size_t>(kcp) * ldk + static_cast<size_t>(cp) * (kcp + 4)) * es + 16;
}

hipError_t run_dense(const DenseArgs& a) {
  if (a.dtype == kF32) {
    switch (a.d) {
      case 8: return launch_dense<float, 8>(a);
      case 16: return launch_dense<float, 16>(a);
      case 32: return launch_dense<float, 32>(a);
      case 64: return launch_dense<float, 64>(a);
      case 128: return launch_dense<float, 128>(a);
    }
  } else {
    switch (a.d) {
      case 16: return launch_dense<bf16, 16>(a);
      case 32: return launch_dense<bf16, 32>(a);
      case 64: return launch_dense<bf16, 64>(a);
      case 128: return launch_dense<bf16, 128>(a);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace tarmac
