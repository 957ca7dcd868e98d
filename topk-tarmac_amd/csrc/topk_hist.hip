// Exact top-k attention for large k (fp32 and bf16 inputs; d = 16 and 32
// with N <= 512, d = 64 with N <= 256): every score of a query stays in
// registers, a histogram of them locates the k-th largest, and the kept
// keys' softmax weights drive the MFMA aggregation of the dense kernel (every
// other key weighs 0). bf16 rows are widened to fp32 as they are staged, so
// the scores are the canonical fp32 scores of the widened inputs.
//
// Reference behaviour: the top-k core (src/agents/mappo.py:192-231 topk_gather,
// src/kernels/fused_topk_attention.py:296-355) at the module's k = 0.25 (N - 1)
// (scripts/microbenchmark_comm.py), ties to the lower index
// (src/kernels/streaming_topk_attention.py:37-44); the retained indices come
// out in ascending order.
//
// Layout: workgroup = (batch row b, 64 queries), four waves of 16 queries;
// lane l owns query l % 16 and, in 16-key tile t, keys 16 t + 4 (l / 16) + r.
//  1. scores: fp32 MFMA on the key rows staged in LDS, q pre-multiplied by the
//     power-of-two scale: these ARE the canonical fp32 scores (the MFMA chain
//     rounds like the canonical fmaf chain, in its order).
//  2. histogram: kHistBins bins spanning [min, max] of a query's scores,
//     counted with LDS atomics; a scan from the top finds the bin tb that
//     holds the k-th largest.
//  3. select, in the pass that aggregates: scores above tb's upper edge (plus
//     the binning's rounding slack) are kept, scores below its lower edge are
//     dropped; the scores in between -- bin tb, every tie at the k-th score
//     among them -- are written to per-lane LDS slots as the pass goes.
//  4. aggregate: P = 2^((s - max) log2 e) on the kept keys (0 elsewhere) in
//     the fp32 MFMA P V product of the dense kernel.
//  5. rank the band: the wave's band entries form one flat list (query-major),
//     each as a 64-bit key (ordered score, descending | key index); every lane
//     ranks one or more entries against its query's entries, and a query's
//     best k - |kept| join; their value rows are added by the query's lanes.
//  6. indices (optional): kept and joining keys set bits of a per-query mask;
//     the wave's 16 rows of ascending indices are staged in LDS and stored as
//     one contiguous block.
//  fallback: a wave with a query whose band could overflow the slots (ties,
//     rows of nearly equal scores) or with non-finite inputs or scores takes
//     the queries one at a time over the whole wave: the k-th largest 32-bit
//     ordered key by bisection, ties to the lower index.
#include <type_traits>

#include "exact.hpp"
#include "frag.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

namespace {

constexpr int kHistBins = 128;   // per query
constexpr int kHistSlots = 16;   // band score slots per lane (fast path: fewer entries)
constexpr int kHistWaves = 4;    // 16-query waves per workgroup
constexpr int kHistSel = 16;     // selection bitmask words per query (N <= 512)
constexpr int kHistQWords = kHistBins + kHistSel;  // scratch words per query
constexpr unsigned kHistMaskedBits = 0xffffffffu;  // a NaN; its ordered key is INT_MIN

__device__ __forceinline__ float masked_score() { return __uint_as_float(kHistMaskedBits); }

// Monotone fp32 -> int32 (NaN above +inf, kHistMaskedBits -> INT_MIN).
__device__ __forceinline__ int ordered_key(float x) {
  const int i = __float_as_int(x);
  return i ^ ((i >> 31) & 0x7fffffff);
}

// v_cvt_u32_f32 (NaN, y < 0 -> 0).
__device__ __forceinline__ unsigned cvt_u32(float y) {
  unsigned u;
  asm("v_cvt_u32_f32 %0, %1" : "=v"(u) : "v"(y));
  return u;
}

// Histogram bin of a score (NaN -> 0); monotone in x. The clamp matters only
// when |min| dwarfs the range, where the rounding of c0 can reach bin
// kHistBins (such rows also fail the fast path's margin test).
__device__ __forceinline__ unsigned bin_of(float x, float inv, float c0) {
  return min(cvt_u32(fmaf(x, inv, c0)), static_cast<unsigned>(kHistBins - 1));
}

// x of lane l - N of the same 16-lane row (0 in the row's first N lanes).
template <int N>
__device__ __forceinline__ int dpp_shr(int x) {
  return __builtin_amdgcn_update_dpp(0, x, 0x110 + N, 0xF, 0xF, false);
}

// x, as a value the compiler cannot relate to other expressions: key
// indices recomputed in a later phase then cost an add instead of keeping
// one register per score live from an earlier phase.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Within one wavefront: LDS writes issued before are seen by reads issued after.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sum over the four lane rows (lanes l, l ^ 16, l ^ 32, l ^ 48).
__device__ __forceinline__ unsigned rows_sum(unsigned x) {
  const LanePair p = swap_rows16(x);
  const LanePair q = swap_rows32(p.a + p.b);
  return q.a + q.b;
}
__device__ __forceinline__ float rows_sum(float x) {
  const LanePair p = swap_rows16(__float_as_uint(x));
  const float s = __uint_as_float(p.a) + __uint_as_float(p.b);
  const LanePair q = swap_rows32(__float_as_uint(s));
  return __uint_as_float(q.a) + __uint_as_float(q.b);
}
__device__ __forceinline__ float rows_max(float x) {
  const LanePair p = swap_rows16(__float_as_uint(x));
  const float s = fmaxf(__uint_as_float(p.a), __uint_as_float(p.b));
  const LanePair q = swap_rows32(__float_as_uint(s));
  return fmaxf(__uint_as_float(q.a), __uint_as_float(q.b));
}
__device__ __forceinline__ float rows_min(float x) {
  const LanePair p = swap_rows16(__float_as_uint(x));
  const float s = fminf(__uint_as_float(p.a), __uint_as_float(p.b));
  const LanePair q = swap_rows32(__float_as_uint(s));
  return fminf(__uint_as_float(q.a), __uint_as_float(q.b));
}

// The canonical fp32 chain (element kk*(D/4) + t at step t, slot kk) of the
// query row held in registers (pre-multiplied by a power-of-two scale, or
// not: the caller then scales the result) against key row krow, read in
// chunks of 16 elements.
template <typename T, int D>
__device__ __forceinline__ float canon_row(const float (&qs)[D], const T* krow) {
  constexpr int QD = D / 4, TS = QD < 4 ? QD : 4;
  float acc = 0.f;
#pragma unroll
  for (int t0 = 0; t0 < QD; t0 += TS) {
    float k[4][TS];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) ld_row<T, TS>(k[kk], krow + kk * QD + t0);
#pragma unroll
    for (int t = 0; t < TS; ++t)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc = fmaf(qs[kk * QD + t0 + t], k[kk][t], acc);
  }
  return acc;
}

template <int NT>
constexpr size_t hist_scratch_bytes() {
  return static_cast<size_t>(kHistWaves) * 16 * kHistQWords * 4 + kHistWaves * 32 * 4;
}

template <int NT, int D>
constexpr size_t hist_region_a_bytes() {
  const size_t ks = static_cast<size_t>(16 * NT) * Frag<float, D>::LDK * sizeof(float);
  const size_t sc = hist_scratch_bytes<NT>();
  return ks > sc ? ks : sc;
}

// The key rows (fp32, then the waves' scratch) and the transposed value rows
// (fp32, D channels).
template <int NT, int D>
constexpr size_t hist_lds_bytes() {
  return 16 + hist_region_a_bytes<NT, D>() + static_cast<size_t>(D) * (16 * NT + 4) * sizeof(float);
}

// Stage `rows` bf16 rows of D elements as fp32 into LDS (row stride LDK
// floats), zero rows up to rows_pad: every score of the kernel then comes
// from the fp32 MFMA chain on the exactly widened inputs, the canonical
// score of bf16 inputs.
template <int D, int LDK>
__device__ __forceinline__ void stage_rows_widen(float* lds, const bf16* src, int rows, int rows_pad) {
  constexpr int VPR = D / 8;  // 16-byte source vectors per row
  const int total = rows_pad * VPR, avail = rows * VPR;
  for (int v = threadIdx.x; v < total; v += blockDim.x) {
    const int row = v / VPR, cv = v - row * VPR;
    uint4 x = make_uint4(0u, 0u, 0u, 0u);
    if (v < avail) x = reinterpret_cast<const uint4*>(src)[v];
    const f32x4 a = {__uint_as_float(x.x << 16), __uint_as_float(x.x & 0xffff0000u),
                     __uint_as_float(x.y << 16), __uint_as_float(x.y & 0xffff0000u)};
    const f32x4 c = {__uint_as_float(x.z << 16), __uint_as_float(x.z & 0xffff0000u),
                     __uint_as_float(x.w << 16), __uint_as_float(x.w & 0xffff0000u)};
    *reinterpret_cast<f32x4*>(lds + row * LDK + 8 * cv) = a;
    *reinterpret_cast<f32x4*>(lds + row * LDK + 8 * cv + 4) = c;
  }
}

// Stage V[rows, D] (bf16) transposed into Vt[c][key] as fp32 (row stride
// ldv), zero keys [rows, rows_pad).
template <int D>
__device__ __forceinline__ void stage_vt_widen(float* Vt, int ldv, const bf16* src, int rows,
                                               int rows_pad) {
  constexpr int VPR = D / 8;
  const int total = rows_pad * VPR;
  for (int v = threadIdx.x; v < total; v += blockDim.x) {
    const int row = v / VPR, cv = v - row * VPR;
    uint4 x = make_uint4(0u, 0u, 0u, 0u);
    if (row < rows) x = reinterpret_cast<const uint4*>(src)[v];
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      Vt[(8 * cv + e) * ldv + row] =
          __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
  }
}

// Sums and maximum over the whole wave (DPP row reductions, then row swaps).
__device__ __forceinline__ unsigned wave_sum(unsigned x) {
  const int r = row16_reduce(static_cast<int>(x), [](int a, int b) { return a + b; });
  return rows_sum(static_cast<unsigned>(r));
}
__device__ __forceinline__ float wave_sum(float x) {
  return rows_sum(row16_reduce(x, [](float a, float b) { return a + b; }));
}

// The fallback of a wave: its queries one at a time over all 64 lanes (keys
// j = lane + 64 i), canonical fp32 scores, the k-th largest ordered key by
// bisection over the 32-bit range, ties at it to the lowest indices (a
// ballot prefix in ascending key order), the kept value rows summed across
// the wave. Writes out (and the ascending indices) itself.
template <int NT, typename T, int D>
__device__ __forceinline__ void hist_fallback_wave(const T* Qb, const T* Kb, const T* Vb, T* Ob,
                                                   int32_t* Ib, int N, int q0, int topk,
                                                   float scale, int lane) {
  constexpr bool POW2 = pow2_scale<D>();
  constexpr int NI = (16 * NT + 63) / 64;  // keys per lane
  const unsigned kq = static_cast<unsigned>(topk);
  const uint64_t below = (1ull << lane) - 1ull;
  for (int qq = 0; qq < 16; ++qq) {
    const int qi = q0 + qq;
    if (qi >= N) break;  // uniform
    float qs[D];
    ld_row<T, D>(qs, Qb + static_cast<size_t>(qi) * D);
    if constexpr (POW2) {
#pragma unroll
      for (int c = 0; c < D; ++c) qs[c] *= scale;
    }
    int key[NI];
    float mloc = -INFINITY;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int j = lane + 64 * i;
      const bool valid = j < N && j != qi;
      float c = masked_score();
      if (valid) {
        c = canon_row<T, D>(qs, Kb + static_cast<size_t>(j) * D);
        if constexpr (!POW2) c *= scale;
      }
      mloc = fmaxf(mloc, c);
      key[i] = ordered_key(c);
    }
    const float mq = wave_max_rows(mloc);
    long lo = -2147483647L, hi = 2147483647L;  // INT_MIN (masked) never counts
    for (int it = 0; it < 32; ++it) {
      const long mid = lo + (hi - lo + 1) / 2;
      unsigned c = 0u;
#pragma unroll
      for (int i = 0; i < NI; ++i) c += key[i] >= mid ? 1u : 0u;
      c = wave_sum(c);
      if (c >= kq) lo = mid;
      else hi = mid - 1;
      if (c == kq) break;  // uniform: exactly k keys at or above lo
    }
    const int thr = static_cast<int>(lo);
    unsigned gt = 0u;
#pragma unroll
    for (int i = 0; i < NI; ++i) gt += key[i] > thr ? 1u : 0u;
    const unsigned need_ties = kq - wave_sum(gt);
    unsigned ties = 0u, base = 0u;
    float lsum = 0.f;
    float pw[NI];  // this lane's weights (0: not selected)
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int j = lane + 64 * i;
      const bool tie = key[i] == thr;
      const uint64_t tmask = __ballot(tie);
      const bool sel = key[i] > thr || (tie && ties + __popcll(tmask & below) < need_ties);
      const uint64_t smask = __ballot(sel);
      pw[i] = 0.f;
      if (sel) {
        // the ordered key maps back to the score by the same xor
        const float c = __int_as_float(ordered_key(__int_as_float(key[i])));
        pw[i] = fast_exp2((c - mq) * kLog2eF);  // subtract first: exact near the max
        lsum += pw[i];
        if (Ib != nullptr) {
          const unsigned pos = base + static_cast<unsigned>(__popcll(smask & below));
          if (pos < kq) Ib[static_cast<size_t>(qi) * topk + pos] = j;
        }
      }
      ties += static_cast<unsigned>(__popcll(tmask));
      base += static_cast<unsigned>(__popcll(smask));
    }
    const float il = 1.f / wave_sum(lsum);
    // the kept value rows summed across the wave, 16 channels at a time
#pragma unroll
    for (int c0 = 0; c0 < D; c0 += 16) {
      float acc[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int j = lane + 64 * i;
        if (pw[i] != 0.f) {
          float vr[16];
          ld_row<T, 16>(vr, Vb + static_cast<size_t>(j) * D + c0);
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[e] = fmaf(pw[i], vr[e], acc[e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = wave_sum(acc[e]);
      if (lane < 4) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = 0.f;
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (e == 4 * lane + r) v = acc[e];
          o[r] = v * il;
        }
        st_row<T, 4>(Ob + static_cast<size_t>(qi) * D + c0 + 4 * lane, o);
      }
    }
  }
}

}  // namespace

// Waves per SIMD the register budget is held to (the scores of a query tile
// take NT x 4 registers); without the cap the compiler parks a second copy
// of them in AGPRs and drops to one wave.
template <int NT, int D>
constexpr int hist_waves_per_eu() {
  // wider heads add D/4 query and 12 D/16 value-block registers per lane
  if constexpr (D >= 64) return 2;
  return NT <= 8 ? (D <= 16 ? 4 : 3) : (NT <= 16 ? 3 : 2);
}

// T: the inputs' type (bf16 rows are widened to fp32 as they are staged, so
// every score is the canonical fp32 chain of the widened values); D: the head
// width (16, 32 or 64: D/16 output blocks of 16 channels).
template <int NT, bool WITH_IDX, typename T, int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(hist_waves_per_eu<NT, D>(), hist_waves_per_eu<NT, D>())))
topk_hist_kernel(const T* __restrict__ Q, const T* __restrict__ Kx,
                 const T* __restrict__ V, T* __restrict__ O, int32_t* __restrict__ Idx,
                 int N, int n_qblk, int topk, float scale, int nblocks) {
  using F = Frag<float, D>;
  constexpr int LDK = F::LDK, NP = 16 * NT, LDV = NP + 4, NH = D / 16;
  static_assert(D % 16 == 0, "whole 16-channel output blocks");
  constexpr int BT = 4;  // tiles per score block
  static_assert(NT % BT == 0 && NP <= 32 * kHistSel, "tile count");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  unsigned* flags = reinterpret_cast<unsigned*>(smem_raw);  // [0] a non-finite key element
  unsigned char* region_a = smem_raw + 16;
  float* Ks = reinterpret_cast<float*>(region_a);            // key rows, then scratch
  float* Vt = reinterpret_cast<float*>(region_a + hist_region_a_bytes<NT, D>());

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qblk = blk - b * n_qblk;
  const int q0 = (qblk * kHistWaves + wave) * 16;  // first query of this wave (uniform)
  const int col = lane & 15, grp = lane >> 4;
  const bool live = q0 + col < N;
  const int qi = live ? q0 + col : N - 1;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const T* Kb = Kx + boff;
  // a power-of-two scale (d = 16, 64) is folded into q (exact); any other
  // multiplies each score once, as the canonical score does
  constexpr bool POW2 = pow2_scale<D>();

  // ---- stage the row's keys and transposed values ------------------------
  if (threadIdx.x == 0) flags[0] = 0u;
  if constexpr (sizeof(T) == 4) {
    stage_rows<float, D, LDK>(Ks, Kb, N, NP);
    stage_vt<float, D, D>(Vt, LDV, V + boff, N, NP);
  } else {
    stage_rows_widen<D, LDK>(Ks, Kb, N, NP);
    stage_vt_widen<D>(Vt, LDV, V + boff, N, NP);
  }
  F frag;
  ld_row<T, F::E>(frag.q, Q + boff + static_cast<size_t>(qi) * D + grp * F::E);
  if constexpr (POW2) {
#pragma unroll
    for (int e = 0; e < F::E; ++e) frag.q[e] *= scale;
  }
  bool finite_in = true;  // this lane's query elements
#pragma unroll
  for (int e = 0; e < F::E; ++e) finite_in = finite_in && __builtin_isfinite(frag.q[e]);
  __syncthreads();
  {
    bool kfin = true;  // the staged keys, four elements per thread and pass
    constexpr int V4 = D / 4;
    for (int v = threadIdx.x; v < N * V4; v += blockDim.x) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(Ks + (v / V4) * LDK + 4 * (v % V4));
#pragma unroll
      for (int e = 0; e < 4; ++e) kfin = kfin && __builtin_isfinite(x[e]);
    }
    if (!__all(kfin) && lane == 0) atomicOr(flags, 1u);
  }

  // ---- canonical scores, masked self / padding ----------------------------
  float s[NT][4];
  const int diag = q0 >> 4;  // the tile holding this wave's self pairs
#pragma unroll
  for (int t0 = 0; t0 < NT; t0 += BT) {
    f32x4 acc[1][BT];
    F fr[1] = {frag};
    block_scores<F, 1, BT>(fr, Ks, 16 * t0, LDK, lane, acc);
#pragma unroll
    for (int t = 0; t < BT; ++t) {
      const int tt = t0 + t;
#pragma unroll
      for (int r = 0; r < 4; ++r) s[tt][r] = POW2 ? acc[0][t][r] : acc[0][t][r] * scale;
      if (tt == diag || 16 * tt + 16 > N) {  // wave-uniform
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * tt + 4 * grp + r;
          if (j >= N || j == qi) s[tt][r] = masked_score();
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // one block's key fragments live at a time
  }
  __syncthreads();  // every wave is past its scores: region A becomes the waves' scratch
  if (q0 >= N) return;  // a wave of padding queries (no barrier follows)
  finite_in = finite_in && flags[0] == 0u;

  unsigned* qscr = reinterpret_cast<unsigned*>(region_a) +
                   static_cast<size_t>(wave * 16 + col) * kHistQWords;  // this lane's query
  unsigned* hist = qscr;                   // [kHistBins]
  unsigned* selw = qscr + kHistBins;       // [kHistSel] selection bitmask
  {
    const uint4 z = make_uint4(0u, 0u, 0u, 0u);
    // a query's 144 words: 36 uint4, 9 per lane row
#pragma unroll
    for (int i = 0; i < kHistQWords / 16; ++i)
      reinterpret_cast<uint4*>(qscr)[grp * (kHistQWords / 16) + i] = z;
  }

  // ---- range and histogram ------------------------------------------------
  float mx = -INFINITY, mn = INFINITY;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      mx = fmaxf(mx, s[t][r]);  // NaN (masked) operands are ignored
      mn = fminf(mn, s[t][r]);
    }
  mx = rows_max(mx);
  mn = rows_min(mn);
  const float range = mx - mn;
  const bool finite_s = __builtin_isfinite(range);
  const float inv = (finite_s && range > 0.f) ? (kHistBins * (1.f - 0x1p-20f)) / range : 0.f;
  const float c0 = -mn * inv;
  wave_lds_sync();
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) atomicAdd(hist + bin_of(s[t][r], inv, c0), 1u);
  wave_lds_sync();

  // ---- scan: the bin tb holding the k-th largest -------------------------
  const unsigned n_masked = static_cast<unsigned>(NP - N + 1);  // padding keys and self, in bin 0
  const unsigned kq = static_cast<unsigned>(topk);
  // four-bin group sums of this lane row's 32 bins (32 grp .. 32 grp + 31)
  unsigned q4[8], tot = 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint4 w = reinterpret_cast<const uint4*>(hist)[grp * 8 + i];
    q4[i] = w.x + w.y + w.z + w.w - ((grp == 0 && i == 0) ? n_masked : 0u);
    tot += q4[i];
  }
  uint32_t rt[4];
  gather_rows(tot, rt);
  unsigned above = 0u;  // valid scores in the rows above this lane's
#pragma unroll
  for (int g = 0; g < 4; ++g) above += g > grp ? rt[g] : 0u;
  // the group of four bins, then the bin (scanning downwards)
  int qg = -1;
  unsigned above_g = 0u, run = above;
#pragma unroll
  for (int i = 7; i >= 0; --i) {
    const unsigned nrun = run + q4[i];
    if (run < kq && nrun >= kq) {
      qg = i;
      above_g = run;
    }
    run = nrun;
  }
  int tb_l = -1;
  if (qg >= 0) {
    const uint4 w = reinterpret_cast<const uint4*>(hist)[grp * 8 + qg];
    const unsigned hq[4] = {w.x - ((grp == 0 && qg == 0) ? n_masked : 0u), w.y, w.z, w.w};
    unsigned rr = above_g;
#pragma unroll
    for (int e = 3; e >= 0; --e) {
      const unsigned nr = rr + hq[e];
      if (rr < kq && nr >= kq) tb_l = 32 * grp + 4 * qg + e;
      rr = nr;
    }
  }
  int tb;
  {
    uint32_t tv[4];
    gather_rows(static_cast<uint32_t>(tb_l + 1), tv);
    tb = -1;
#pragma unroll
    for (int g = 0; g < 4; ++g)
      if (tv[g] != 0u) tb = static_cast<int>(tv[g]) - 1;
  }
  // bins tb - 1 .. tb + 1 bound the list (the margin is under half a bin)
  auto bin_count = [&](int bin) -> unsigned {
    if (bin < 0 || bin >= kHistBins) return 0u;
    const unsigned h = hist[bin];
    return bin == 0 ? h - n_masked : h;
  };
  const unsigned n_valid = static_cast<unsigned>(N - 1);
  const unsigned cand_bound = inv > 0.f ? bin_count(tb - 1) + bin_count(tb) + bin_count(tb + 1)
                                        : n_valid;

  // ---- thresholds ---------------------------------------------------------
  // bin tb spans [lo_edge, hi_edge) up to the rounding of the binning (slack)
  const float w = inv > 0.f ? 1.f / inv : 0.f;
  const float lo_edge = inv > 0.f ? fmaf(static_cast<float>(tb), w, mn) : mn;
  const float hi_edge = inv > 0.f ? fmaf(static_cast<float>(tb + 1), w, mn) : mx;
  const float slack = 0x1p-18f * (fabsf(mx) + fabsf(mn) + range);
  const float hiT = hi_edge + slack, loT = lo_edge - slack;
  const bool fast = finite_in && finite_s && cand_bound <= 4 * kHistSlots &&
                    (inv == 0.f || slack < 0.5f * w);

  if (!__all(fast)) {
    hist_fallback_wave<NT, T, D>(Q + boff, Kb, V + boff, O + boff,
                                 Idx ? Idx + static_cast<size_t>(b) * N * topk : nullptr, N, q0,
                                 topk, scale, lane);
    return;
  }

  // ---- kept keys into the product; the band onto per-lane lists -----------
  // exponents: one fma while the maximum is small enough for its rounding in
  // -m log2(e) to be negligible, else subtract first (exact near the maximum)
  const bool small = __all(fabsf(mx) <= 16.f);
  const float nm = -mx * kLog2eF;
  auto expw = [&](float x) {
    return small ? fast_exp2(fmaf(x, kLog2eF, nm)) : fast_exp2((x - mx) * kLog2eF);
  };
  f32x4 acc[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) acc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
  constexpr int NB32 = (NT * 4 + 31) / 32;
  uint32_t kept[NB32];  // bit (4 t + r) % 32 of word (4 t + r) / 32: kept key
#pragma unroll
  for (int i = 0; i < NB32; ++i) kept[i] = 0u;
  uint32_t band[NB32];  // the same for band keys
#pragma unroll
  for (int i = 0; i < NB32; ++i) band[i] = 0u;
  // Band scores go to this lane's kHistSlots slots, in key order (the keys
  // come back from the band bits): every score is written to slot nl mod
  // kHistSlots and only band scores advance nl, so no branch is needed
  // (slots past nl are stale; a lane holds at most kHistSlots - 1 band
  // scores on the fast path). The histogram words the slots reuse are no
  // longer read.
  float* slots = reinterpret_cast<float*>(qscr) + kHistSlots * grp;
  unsigned nl = 0u;
  wave_lds_sync();
  auto pv_pass = [&](auto exp_small) {
    // output block h (channels 16 h .. 16 h + 15): V^T rows 16 h + col
    const float* vrow = Vt + col * LDV + 4 * grp;
    f32x4 vnext[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) vnext[h] = *reinterpret_cast<const f32x4*>(vrow + 16 * h * LDV);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // this tile's value fragments were read a tile ahead: the MFMAs below
      // do not wait on the slot writes
      f32x4 vv[NH];
#pragma unroll
      for (int h = 0; h < NH; ++h) vv[h] = vnext[h];
      if (t + 1 < NT) {
#pragma unroll
        for (int h = 0; h < NH; ++h)
          vnext[h] = *reinterpret_cast<const f32x4*>(vrow + 16 * h * LDV + 16 * (t + 1));
      }
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = s[t][r];
        const bool keep = x > hiT;
        // the select goes on the exponent (2^-inf = 0): no branch around the exp
        const float y = exp_small ? fmaf(x, kLog2eF, nm) : (x - mx) * kLog2eF;
        p[r] = fast_exp2(keep ? y : -INFINITY);
        lsum += p[r];
        const int bit = (4 * t + r) & 31, word = (4 * t + r) >> 5;
        const bool inband = !keep && x >= loT;
        kept[word] |= static_cast<uint32_t>(keep) << bit;
        band[word] |= static_cast<uint32_t>(inband) << bit;
        slots[nl & (kHistSlots - 1)] = x;
        nl += inband ? 1u : 0u;
      }
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[h] = mfma_f32_16x16x4(vv[h][u], p[u], acc[h]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if (small) pv_pass(std::true_type{});
  else pv_pass(std::false_type{});
#pragma unroll
  for (int i = 0; i < NB32; ++i) {  // materialised here: the scores die with the pass
    kept[i] = static_cast<uint32_t>(opaque(static_cast<int>(kept[i])));
    band[i] = static_cast<uint32_t>(opaque(static_cast<int>(band[i])));
  }
  if (!__all(nl < static_cast<unsigned>(kHistSlots))) {  // a lane's share overflowed
    hist_fallback_wave<NT, T, D>(Q + boff, Kb, V + boff, O + boff,
                                 Idx ? Idx + static_cast<size_t>(b) * N * topk : nullptr, N, q0,
                                 topk, scale, lane);
    return;
  }

  // ---- rank the band over the wave's flat list ----------------------------
  // Entry e of the wave's list (at most 512) sits in the upper half of query
  // (e / 32)'s words; a query's entries are contiguous (its four lane rows in
  // order), as (ordered key of the score, descending | key index, query). A
  // query takes its `need` best band entries: k minus the keys kept by the
  // pass.
  unsigned nk = 0u;
#pragma unroll
  for (int i = 0; i < NB32; ++i) nk += __builtin_popcount(kept[i]);
  const unsigned need = kq - rows_sum(nk);
  uint32_t nls[4];
  gather_rows(nl, nls);
  const unsigned cnt = nls[0] + nls[1] + nls[2] + nls[3];
  unsigned rowoff = 0u;
#pragma unroll
  for (int g = 0; g < 4; ++g) rowoff += g < grp ? nls[g] : 0u;
  unsigned incl = cnt;  // prefix over the 16 queries of a row (the four rows agree)
  incl += static_cast<unsigned>(dpp_shr<1>(static_cast<int>(incl)));
  incl += static_cast<unsigned>(dpp_shr<2>(static_cast<int>(incl)));
  incl += static_cast<unsigned>(dpp_shr<4>(static_cast<int>(incl)));
  incl += static_cast<unsigned>(dpp_shr<8>(static_cast<int>(incl)));
  const unsigned qoff = incl - cnt;
  const unsigned total = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(incl), 15));
  if (total > 512u || !__all(need <= 32u)) {  // beyond the flat list's (16 x 32) or a join list's (32) room
    hist_fallback_wave<NT, T, D>(Q + boff, Kb, V + boff, O + boff,
                                 Idx ? Idx + static_cast<size_t>(b) * N * topk : nullptr, N, q0,
                                 topk, scale, lane);
    return;
  }
  unsigned* wscr = reinterpret_cast<unsigned*>(region_a) + kHistWaves * 16 * kHistQWords + wave * 32;
  unsigned* wreg = reinterpret_cast<unsigned*>(region_a) + static_cast<size_t>(wave) * 16 * kHistQWords;
  auto flat = [&](unsigned e) -> uint2* {  // e < 512
    return reinterpret_cast<uint2*>(wreg + (e >> 5) * kHistQWords + 64) + (e & 31u);
  };
  if (grp == 0) wscr[col] = qoff | (cnt << 10) | (need << 20);
  const unsigned mnl = static_cast<unsigned>(wave_max_rows(static_cast<float>(nl)));
  {
    // slot i holds the score of the i-th band key in key order
    uint64_t blo = band[0], bhi = 0u;
    if constexpr (NB32 > 1) blo |= static_cast<uint64_t>(band[1]) << 32;
    if constexpr (NB32 > 2) bhi = band[2];
    if constexpr (NB32 > 3) bhi |= static_cast<uint64_t>(band[3]) << 32;
    for (unsigned i = 0; i < mnl; ++i) {
      if (i < nl) {
        unsigned pos;
        if (blo != 0u) {
          pos = static_cast<unsigned>(__builtin_ctzll(blo));
          blo &= blo - 1u;
        } else {
          pos = 64u + static_cast<unsigned>(__builtin_ctzll(bhi));
          bhi &= bhi - 1u;
        }
        const unsigned j = 16u * (pos >> 2) + 4u * grp + (pos & 3u);
        const uint32_t u = __float_as_uint(slots[i] + 0.f);  // -0 -> +0
        const uint32_t m = static_cast<uint32_t>(static_cast<int>(u) >> 31);
        *flat(qoff + rowoff + i) = make_uint2((u ^ ~m) & (m | 0x7fffffffu), j | (col << 16));
      }
    }
  }
  const unsigned qcmax = static_cast<unsigned>(wave_max_rows(static_cast<float>(cnt)));
  const unsigned needmax = static_cast<unsigned>(wave_max_rows(static_cast<float>(need)));
  wave_lds_sync();
  const int rounds = static_cast<int>((total + 63u) >> 6);
  // A joining entry of rank r goes to slot r of its query's join list (the
  // query's first 64 words, free once the slots are flattened) and, with
  // indices, sets its bit in the query's selection mask.
  for (int h = 0; h < rounds; ++h) {
    const unsigned e = static_cast<unsigned>(lane + 64 * h);
    if (e < total) {
      const uint2 me = *flat(e);
      const unsigned q = (me.y >> 16) & 15u;
      const unsigned info = wscr[q];
      const unsigned qs = info & 1023u, qc = (info >> 10) & 1023u, qn = info >> 20;
      const uint64_t mk = (static_cast<uint64_t>(me.x) << 32) | me.y;
      unsigned rank = 0u;
      for (unsigned i = 0; i < qcmax; ++i) {
        const uint2 o = *flat(min(qs + i, 511u));
        const uint64_t ok = (static_cast<uint64_t>(o.x) << 32) | o.y;
        rank += (i < qc && ok < mk) ? 1u : 0u;
      }
      if (rank < qn) {
        const unsigned j = me.y & 0xffffu;
        reinterpret_cast<uint2*>(wreg + q * kHistQWords)[rank] = make_uint2(me.x, j);
        if constexpr (WITH_IDX)
          atomicOr(wreg + q * kHistQWords + kHistBins + (j >> 5), 1u << (j & 31u));
      }
    }
  }
  wave_lds_sync();

  // ---- the joining keys' value rows (from the transposed copy in LDS) ------
  // each query's four lanes walk its join list: weights from the query's own
  // maximum
  const uint2* jl = reinterpret_cast<const uint2*>(qscr);
  for (unsigned i = 0; i < needmax; ++i) {
    if (i < need) {
      const uint2 o = jl[i];
      const uint32_t m = static_cast<uint32_t>(static_cast<int>(o.x) >> 31);
      const float pw = expw(__uint_as_float(m ? o.x : (~o.x & 0x7fffffffu)));  // the score back
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[h][r] = fmaf(pw, Vt[(16 * h + 4 * grp + r) * LDV + o.y], acc[h][r]);
      lsum += grp == 0 ? pw : 0.f;
    }
  }

  // ---- normalise and store ------------------------------------------------
  const float l = rows_sum(lsum);
  const float il = 1.f / l;
  if (live) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = acc[h][r] * il;
      st_row<T, 4>(O + boff + static_cast<size_t>(qi) * D + 16 * h + 4 * grp, o);
    }
  }
  if constexpr (!WITH_IDX) return;
  // ---- retained indices, ascending -----------------------------------------
  // selection word w (keys 32 w .. 32 w + 31) = the kept flags of tiles 2 w
  // and 2 w + 1 (lane row g holds bits 4 g .. 4 g + 3 of each 16-key half;
  // the rows' disjoint bits meet in a sum) plus the joining keys' marks
  constexpr int NW = NP / 32;
  uint32_t wv[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const uint32_t n0 = (kept[(8 * w) >> 5] >> ((8 * w) & 31)) & 0xfu;
    const uint32_t n1 = (kept[(8 * w + 4) >> 5] >> ((8 * w + 4) & 31)) & 0xfu;
    wv[w] = rows_sum((n0 << (4 * grp)) | (n1 << (16 + 4 * grp))) | selw[w];
  }
  const int nq = min(16, N - q0);
  int32_t* dst = Idx + (static_cast<size_t>(b) * N + q0) * topk;
  if (topk <= kHistQWords) {
    // the wave's 16 x topk indices are one contiguous block: staged in the
    // wave's words (free once the bitmasks are read), then stored with
    // consecutive lanes on consecutive addresses
    wave_lds_sync();
    // lane row g expands words g, g + 4, ... of its query, all lanes at once,
    // two keys per step
    unsigned pre[NW];  // selected keys in the words before word i
    {
      unsigned run = 0u;
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        pre[i] = run;
        run += __builtin_popcount(wv[i]);
      }
    }
    unsigned* orow = wreg + col * topk;
#pragma unroll
    for (int k = 0; k < (NW + 3) / 4; ++k) {
      uint32_t bits = 0u;
      unsigned pos = 0u;
#pragma unroll
      for (int i = 4 * k; i < 4 * k + 4 && i < NW; ++i)
        if ((i & 3) == grp) {
          bits = wv[i];
          pos = pre[i];
        }
      if (!live) bits = 0u;
      const unsigned wbase = 32u * static_cast<unsigned>(grp + 4 * k);
      while (bits) {
        const unsigned b1 = static_cast<unsigned>(__builtin_ctz(bits));
        bits &= bits - 1u;
        orow[pos] = wbase + b1;
        if (bits) {
          orow[pos + 1] = wbase + static_cast<unsigned>(__builtin_ctz(bits));
          bits &= bits - 1u;
          pos += 2u;
        } else {
          pos += 1u;
        }
      }
    }
    wave_lds_sync();
    const int count = nq * topk;
    if ((reinterpret_cast<uintptr_t>(dst) & 15u) == 0u && (count & 3) == 0) {
      const uint4* src4 = reinterpret_cast<const uint4*>(wreg);
      uint4* dst4 = reinterpret_cast<uint4*>(dst);
      for (int e = lane; e < (count >> 2); e += 64) dst4[e] = src4[e];
    } else {
      for (int e = lane; e < count; e += 64) dst[e] = static_cast<int32_t>(wreg[e]);
    }
    return;
  }
  if (!live) return;
  unsigned base = 0u;
  int32_t* qdst = dst + col * topk;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    if ((i & 3) == grp) {
      uint32_t bits = wv[i];
      unsigned pos = base;
      while (bits) {
        if (pos < static_cast<unsigned>(topk)) qdst[pos] = 32 * i + __builtin_ctz(bits);
        ++pos;
        bits &= bits - 1u;
      }
    }
    base += __builtin_popcount(wv[i]);
  }
}

// Rows of up to 512 keys at d = 16 and 32, 256 at d = 64: the fp32 key rows
// and transposed value rows of a batch row then fit one workgroup's LDS.
static int hist_max_n(int d) { return d == 64 ? 256 : 512; }

bool topk_hist_supported(const TopkArgs& a) {
  return (a.dtype == kF32 || a.dtype == kBf16) && (a.d == 16 || a.d == 32 || a.d == 64) &&
         a.select == kSelTopk && a.topk > kTopkSmallMax && a.N <= hist_max_n(a.d);
}

template <int NT, typename T, int D>
static hipError_t launch_hist(const TopkArgs& a) {
  static_assert(hist_lds_bytes<NT, D>() <= 160 * 1024, "one workgroup's LDS");
  const int n_qblk = (a.N + 16 * kHistWaves - 1) / (16 * kHistWaves);
  const int nblocks = a.B * n_qblk;
  auto kern = a.idx != nullptr ? topk_hist_kernel<NT, true, T, D> : topk_hist_kernel<NT, false, T, D>;
  constexpr size_t lds = hist_lds_bytes<NT, D>();
  hipLaunchKernelGGL(kern, dim3(nblocks), dim3(64 * kHistWaves), lds,
                     static_cast<hipStream_t>(a.stream), static_cast<const T*>(a.q),
                     static_cast<const T*>(a.k), static_cast<const T*>(a.v),
                     static_cast<T*>(a.out), a.idx, a.N, n_qblk, a.topk, a.scale, nblocks);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t run_hist_t(const TopkArgs& a) {
  if (a.N <= 128) return launch_hist<8, T, D>(a);
  if (a.N <= 256) return launch_hist<16, T, D>(a);
  if constexpr (D <= 32) {
    if (a.N <= 384) return launch_hist<24, T, D>(a);
    return launch_hist<32, T, D>(a);
  }
  return hipErrorInvalidValue;
}

hipError_t run_topk_hist(const TopkArgs& a) {
  const bool bf = a.dtype == kBf16;
  switch (a.d) {
    case 16: return bf ? run_hist_t<bf16, 16>(a) : run_hist_t<float, 16>(a);
    case 32: return bf ? run_hist_t<bf16, 32>(a) : run_hist_t<float, 32>(a);
    case 64: return bf ? run_hist_t<bf16, 64>(a) : run_hist_t<float, 64>(a);
  }
  return hipErrorInvalidValue;
}

}  // namespace tarmac
