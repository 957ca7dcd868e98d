// Exact-selection helpers shared by the top-k kernels that select on packed
// values and then prove (or repair) the result: canonical fp32 rescoring of
// candidates, key staging with row norms (the error bound of bf16 scores),
// and the exact per-query fallback pass.
#pragma once

#include "frag.hpp"
#include "select.hpp"

namespace tarmac {

// Canonical fp32 score of one (query row, key row) pair: the fmaf chain with
// element kk*(D/4)+t at step t, slot kk (the order v_mfma_f32_16x16x4_f32
// rounds in), then scaled (the scale folded into q when it is a power of two).
// Inputs of type T are converted to fp32 first. Four steps at a time, so at
// most 32 elements are live instead of both whole rows.
template <typename T, int D, bool POW2>
__device__ __forceinline__ float canon_pair(const T* qrow, const T* krow, float scale) {
  constexpr int QD = D / 4;
  constexpr int TS = QD < 4 ? QD : 4;
  float acc = 0.f;
#pragma unroll
  for (int t0 = 0; t0 < QD; t0 += TS) {
    float q[4][TS], k[4][TS];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      ld_row<T, TS>(q[kk], qrow + kk * QD + t0);
      ld_row<T, TS>(k[kk], krow + kk * QD + t0);
    }
#pragma unroll
    for (int t = 0; t < TS; ++t)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc = fmaf(POW2 ? q[kk][t] * scale : q[kk][t], k[kk][t], acc);
  }
  return POW2 ? acc : acc * scale;
}

// ---------------------------------------------------------------------------
// cross-lane moves between the four 16-lane rows of a wave (gfx950
// v_permlane16_swap / v_permlane32_swap: VALU, no LDS round trip)
// ---------------------------------------------------------------------------

// x of the lane in row (r & ~1) (.a) and in row (r | 1) (.b), for a lane in
// row r at the same position: each lane gets its own and its xor-16 partner's.
struct LanePair {
  uint32_t a, b;
};
__device__ __forceinline__ LanePair swap_rows16(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  return {r[0], r[1]};
}
// x of the lane in row (r & 1) (.a) and in row (r & 1) + 2 (.b): own and
// xor-32 partner's.
__device__ __forceinline__ LanePair swap_rows32(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return {r[0], r[1]};
}

// x as held by the lanes of rows 0..3 at this lane's position, in every lane:
// three swaps.
__device__ __forceinline__ void gather_rows(uint32_t x, uint32_t (&v)[4]) {
  const LanePair p = swap_rows16(x);    // rows (r & ~1), (r | 1)
  const LanePair e = swap_rows32(p.a);  // rows 0, 2
  const LanePair o = swap_rows32(p.b);  // rows 1, 3
  v[0] = e.a;
  v[1] = o.a;
  v[2] = e.b;
  v[3] = o.b;
}

// Maximum of x over the wave, in every lane: four DPP row rotations and two
// row swaps (no LDS round trip). x NaN-free.
__device__ __forceinline__ float wave_max_rows(float x) {
  x = row16_reduce(x, [](float a, float b) { return max_plain(a, b); });
  const LanePair p = swap_rows16(__float_as_uint(x));
  x = max_plain(__uint_as_float(p.a), __uint_as_float(p.b));
  const LanePair q = swap_rows32(__float_as_uint(x));
  return max_plain(__uint_as_float(q.a), __uint_as_float(q.b));
}

// ---------------------------------------------------------------------------
// canonical rescoring from a query fragment
// ---------------------------------------------------------------------------

// The canonical chain reads query element kk * (D/4) + t at step t, slot kk.
// Every lane of a query holds a quarter of its row in the MFMA fragment
// (lane row g); FragWord names the fragment word and half-word that holds
// element kk * (D/4) + t, and the row that holds it.
template <typename T, int D>
struct FragWord;
template <int D>
struct FragWord<float, D> {  // Frag<float, D>: row g holds g*E + t in word t
  static constexpr int word(int kk, int t) { return t; }
  static constexpr int row(int kk, int t) { return kk; }
  static constexpr int half(int, int) { return -1; }
};
template <int D>
struct FragWord<bf16, D> {
  // d = 16: row g holds 4g .. 4g+3 as two packed words; d >= 32: word
  // 4h + w of row g holds elements 32h + 8g + 2w, +1 (element c = kk*(d/4)
  // + t sits in word 4 (c / 32) + (c % 8) / 2 of row (c % 32) / 8)
  static constexpr int elem(int kk, int t) { return kk * (D / 4) + t; }
  static constexpr int word(int kk, int t) {
    return D == 16 ? t >> 1 : 4 * (elem(kk, t) >> 5) + ((elem(kk, t) & 7) >> 1);
  }
  static constexpr int row(int kk, int t) { return D == 16 ? kk : (elem(kk, t) & 31) >> 3; }
  static constexpr int half(int kk, int t) { return elem(kk, t) & 1; }
};

template <int D>
__device__ __forceinline__ uint32_t frag_word(const Frag<float, D>& f, int j) {
  return __float_as_uint(f.q[j]);
}
__device__ __forceinline__ uint32_t frag_word(const Frag<bf16, 16>& f, int j) {
  const uint2 w = __builtin_bit_cast(uint2, f.q);
  return j ? w.y : w.x;
}
template <int D>
__device__ __forceinline__ uint32_t frag_word(const FragBf16Wide<D>& f, int j) {
  const uint4 w = __builtin_bit_cast(uint4, f.q[j >> 2]);
  const uint32_t a[4] = {w.x, w.y, w.z, w.w};
  return a[j & 3];
}

// Canonical fp32 score of this lane's query (its fragment f; fp32 fragments
// carry a power-of-two scale already) against one key row krow (LDS or
// global, type T), in the canonical order. Every lane of the wave must call
// it (the query's row is gathered across lane rows).
template <typename T, int D, bool POW2>
__device__ __forceinline__ float canon_from_frag(const Frag<T, D>& f, const T* krow, float scale) {
  using W = FragWord<T, D>;
  constexpr int QD = D / 4;
  constexpr int TS = QD < 4 ? QD : 4;
  float acc = 0.f;
#pragma unroll
  for (int t0 = 0; t0 < QD; t0 += TS) {
    float k[4][TS];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) ld_row<T, TS>(k[kk], krow + kk * QD + t0);
#pragma unroll
    for (int t = t0; t < t0 + TS; ++t)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        uint32_t v[4];
        gather_rows(frag_word(f, W::word(kk, t)), v);
        const uint32_t w = v[W::row(kk, t)];
        float qv;
        if constexpr (sizeof(T) == 4) {
          qv = __uint_as_float(w);  // POW2: already scaled
        } else {
          qv = __uint_as_float(W::half(kk, t) ? (w & 0xffff0000u) : (w << 16));
          if constexpr (POW2) qv *= scale;
        }
        acc = fmaf(qv, k[kk][t - t0], acc);
      }
  }
  return POW2 ? acc : acc * scale;
}

// Largest value whose truncation (bits `mask` cleared) equals trunc(t).
__device__ __forceinline__ float trunc_ceiling(float t, uint32_t mask) {
  const uint32_t b = __float_as_uint(t) & ~mask;
  return __uint_as_float((b & 0x80000000u) ? b : (b | mask));
}

// Smallest value whose truncation (bits `mask` cleared) equals trunc(t).
__device__ __forceinline__ float trunc_floor(float t, uint32_t mask) {
  const uint32_t b = __float_as_uint(t) & ~mask;
  return __uint_as_float((b & 0x80000000u) ? (b | mask) : b);
}

// t with the bits `mask` cleared (rounds toward zero: a monotone map).
__device__ __forceinline__ float trunc_bits(float t, uint32_t mask) {
  return __uint_as_float(__float_as_uint(t) & ~mask);
}

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
      const float n2 = group_sum<VPR>(sumsq_bf16x8(w));
      mx = fmaxf(mx, n2);
    }
  }
  return mx;
}

// |q|^2 of the query row whose bf16 fragment this lane holds: each of the
// four lane groups holds D/4 of its elements (Frag<bf16, D>), so the partial
// sums meet with two xor shuffles.
template <int D>
__device__ __forceinline__ float bf16_frag_norm2(const Frag<bf16, D>& f) {
  float n2 = 0.f;
  if constexpr (D == 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = __uint_as_float(static_cast<uint32_t>(static_cast<uint16_t>(f.q[i])) << 16);
      n2 = fmaf(x, x, n2);
    }
  } else {
#pragma unroll
    for (int h = 0; h < Frag<bf16, D>::NI; ++h) {
      const auto w = __builtin_bit_cast(uint4, f.q[h]);
      const uint32_t a[4] = {w.x, w.y, w.z, w.w};
      n2 += sumsq_bf16x8(a);
    }
  }
  return add_xor32(add_xor16(n2));
}

// ---------------------------------------------------------------------------
// exact top K of one query on the VALU, one key row per lane
// ---------------------------------------------------------------------------

// One key row held raw in registers (D elements of T as 32-bit words).
template <typename T, int D>
struct RawRow {
  static constexpr int W = D * static_cast<int>(sizeof(T)) / 4;
  static_assert((D * sizeof(T)) % 16 == 0, "rows are read as 16-byte vectors");
  uint32_t w[W];
  // src: 16-byte aligned row (global memory or LDS)
  __device__ __forceinline__ void load(const T* src) {
#pragma unroll
    for (int v = 0; v < W / 4; ++v) {
      const uint4 x = reinterpret_cast<const uint4*>(src)[v];
      w[4 * v] = x.x; w[4 * v + 1] = x.y; w[4 * v + 2] = x.z; w[4 * v + 3] = x.w;
    }
  }
  // element c as fp32 (bf16 widens exactly)
  __device__ __forceinline__ float at(int c) const {
    if constexpr (sizeof(T) == 4) return __uint_as_float(w[c]);
    else return __uint_as_float((c & 1) ? (w[c >> 1] & 0xffff0000u) : (w[c >> 1] << 16));
  }
};

// Rows per lane per round for kernels whose register count bounds their
// occupancy: one. Kernels that run at most two waves per SIMD (one query tile
// per wave, small batches) take exact_wide_rows: 64 VGPRs of raw key data in
// flight, so one round trip brings 64 G rows (fp32 d = 16: 256 keys; bf16
// d = 64: 128 keys).
template <typename T, int D>
constexpr int exact_wide_rows() {
  constexpr int words = D * static_cast<int>(sizeof(T)) / 4;
  return words >= 64 ? 1 : 64 / words;
}

// The exact top K of one query's canonical fp32 scores (score desc, index
// asc), by the whole wavefront on the VALU: lane l scores keys l, l + 64,
// l + 128, ... each with the canonical fmaf chain itself (element
// kk * (D/4) + t at step t, slot kk, from +0; the scale folded into the query
// when it is a power of two), so the scores are the oracle's bit for bit.
// Every product is one the answer needs -- an MFMA pass for a single query
// would use a sixteenth of its products -- and each round trip fetches G whole
// rows per lane (G = 1, or exact_wide_rows where registers are free). Each lane keeps a list of K over its keys, which arrive in
// ascending order (strict '>' keeps the lower index on ties); the 64 lists
// merge in six xor steps, after which every lane holds the result. The query
// row is read in chunks of 16 elements from qrow (global memory, uniform)
// inside each round, so at most 16 of its elements are live at a time.
// row_at(j): pointer to key row j (global memory or an LDS copy; 16-byte
// aligned).
template <typename T, int D, int K, int G, typename RowAt>
__device__ __forceinline__ void exact_query_topk_lanes(const T* __restrict__ qrow, RowAt row_at,
                                                       int N, int qi, float scale, int lane,
                                                       float (&val)[K], int (&ix)[K]) {
  constexpr bool POW2 = pow2_scale<D>();
  constexpr int QD = D / 4;
  constexpr int TS = QD < 4 ? QD : 4;  // chain steps per query chunk
#pragma unroll
  for (int m = 0; m < K; ++m) { val[m] = -INFINITY; ix[m] = kIdxSentinel; }
#pragma unroll 1
  for (int j0 = 0; j0 < N; j0 += 64 * G) {
    // re-read the query chunks every round (an opaque copy of the pointer
    // keeps the loads from being hoisted out of the loop with all D elements
    // held live across it)
    const T* qr = qrow;
    asm volatile("" : "+s"(qr));
    RawRow<T, D> kr[G];
#pragma unroll
    for (int g = 0; g < G; ++g) kr[g].load(row_at(min(j0 + 64 * g + lane, N - 1)));
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.f;
#pragma unroll
    for (int t0 = 0; t0 < QD; t0 += TS) {
      float qc[4][TS];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        ld_row<T, TS>(qc[kk], qr + kk * QD + t0);
        if constexpr (POW2) {
#pragma unroll
          for (int t = 0; t < TS; ++t) qc[kk][t] *= scale;
        }
      }
#pragma unroll
      for (int t = 0; t < TS; ++t)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int g = 0; g < G; ++g) acc[g] = fmaf(qc[kk][t], kr[g].at(kk * QD + t0 + t), acc[g]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int j = j0 + 64 * g + lane;
      float s = POW2 ? acc[g] : acc[g] * scale;
      if (j >= N || j == qi) s = -INFINITY;
      topk_insert<K>(val, ix, s, j);
    }
  }
#pragma unroll
  for (int step = 1; step < 64; step <<= 1) {
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

}  // namespace tarmac
