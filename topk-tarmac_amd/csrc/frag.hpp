// Register / LDS fragments for the score contraction S^T = K_tile * Q_tile^T.
//
// The query tile (MFMA B operand) lives in registers for a wave's whole pass
// over the keys; the key tile (A operand) is read from an LDS copy of K whose
// rows are padded to break bank conflicts.
//
// fp32: d/4 chained v_mfma_f32_16x16x4_f32. Contraction slot kk (= lane/16) of
// instruction t carries element c = kk*(d/4) + t, so each lane reads d/4
// contiguous elements of its row. The resulting rounding is the "canonical"
// score order restated in oracle/tarmac_oracle.c.
// bf16: v_mfma_f32_16x16x16_bf16 (d = 16) or v_mfma_f32_16x16x32_bf16
// (d = 32, 64, 128), fp32 accumulation.
#pragma once

#include "common.hpp"

namespace tarmac {

template <int E>
__device__ __forceinline__ void ld_f32(float (&dst)[E], const float* src) {
  if constexpr (E % 4 == 0) {
#pragma unroll
    for (int i = 0; i < E / 4; ++i) {
      f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * i);
      dst[4 * i] = v[0]; dst[4 * i + 1] = v[1]; dst[4 * i + 2] = v[2]; dst[4 * i + 3] = v[3];
    }
  } else if constexpr (E == 2) {
    f32x2 v = *reinterpret_cast<const f32x2*>(src);
    dst[0] = v[0]; dst[1] = v[1];
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) dst[i] = src[i];
  }
}

template <int E>
__device__ __forceinline__ void st_f32(float* dst, const float (&src)[E]) {
  if constexpr (E % 4 == 0) {
#pragma unroll
    for (int i = 0; i < E / 4; ++i) {
      f32x4 v = {src[4 * i], src[4 * i + 1], src[4 * i + 2], src[4 * i + 3]};
      *reinterpret_cast<f32x4*>(dst + 4 * i) = v;
    }
  } else if constexpr (E == 2) {
    f32x2 v = {src[0], src[1]};
    *reinterpret_cast<f32x2*>(dst) = v;
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) dst[i] = src[i];
  }
}

// E bf16 elements (E a multiple of 4) -> fp32.
template <int E>
__device__ __forceinline__ void ld_bf16(float (&dst)[E], const bf16* src) {
  static_assert(E % 4 == 0, "bf16 vector width");
#pragma unroll
  for (int i = 0; i < E / 4; ++i) {
    uint2 v = *reinterpret_cast<const uint2*>(src + 4 * i);
    dst[4 * i + 0] = __uint_as_float(v.x << 16);
    dst[4 * i + 1] = __uint_as_float(v.x & 0xffff0000u);
    dst[4 * i + 2] = __uint_as_float(v.y << 16);
    dst[4 * i + 3] = __uint_as_float(v.y & 0xffff0000u);
  }
}

template <int E>
__device__ __forceinline__ void st_bf16(bf16* dst, const float (&src)[E]) {
  static_assert(E % 4 == 0, "bf16 vector width");
  // hardware round to nearest even (v_cvt_pk_bf16_f32, two values per
  // instruction), the rounding of Tensor.to(torch.bfloat16)
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int i = 0; i < E / 4; ++i) {
    const bf16x2_t lo = {static_cast<__bf16>(src[4 * i]), static_cast<__bf16>(src[4 * i + 1])};
    const bf16x2_t hi = {static_cast<__bf16>(src[4 * i + 2]), static_cast<__bf16>(src[4 * i + 3])};
    *reinterpret_cast<uint2*>(dst + 4 * i) =
        make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
  }
}

template <typename T, int E>
__device__ __forceinline__ void ld_row(float (&dst)[E], const T* src) {
  if constexpr (sizeof(T) == 4) ld_f32<E>(dst, reinterpret_cast<const float*>(src));
  else ld_bf16<E>(dst, reinterpret_cast<const bf16*>(src));
}

template <typename T, int E>
__device__ __forceinline__ void st_row(T* dst, const float (&src)[E]) {
  if constexpr (sizeof(T) == 4) st_f32<E>(reinterpret_cast<float*>(dst), src);
  else st_bf16<E>(reinterpret_cast<bf16*>(dst), src);
}

template <typename T, int D>
struct Frag;

// ---- fp32 -----------------------------------------------------------------
template <int D>
struct Frag<float, D> {
  static_assert(D % 4 == 0 && D >= 8 && D <= 128, "fp32 head dim must be 8..128, multiple of 4");
  static constexpr int E = D / 4;       // elements per lane = MFMAs per tile
  static constexpr int LDK = D + 4;     // padded LDS row stride, in elements
  float q[E];

  // qrow: start of this lane's query row. pre: 1 or the power-of-two scale.
  __device__ __forceinline__ void load_q(const float* qrow, int grp, float pre) {
    ld_f32<E>(q, qrow + grp * E);
#pragma unroll
    for (int t = 0; t < E; ++t) q[t] *= pre;
  }
  static constexpr int NI = E;          // MFMA steps per 16x16 score tile
  struct KF { float v[E]; };
  // krow: LDS row of key (tile base + lane % 16).
  __device__ __forceinline__ static KF load_k(const float* krow, int grp) {
    KF f;
    ld_f32<E>(f.v, krow + grp * E);
    return f;
  }
  // Step i of the tile's MFMA chain (steps must run in order 0..NI-1).
  __device__ __forceinline__ f32x4 step(const KF& kf, int i, f32x4 acc) const {
    return mfma_f32_16x16x4(kf.v[i], q[i], acc);
  }
  __device__ __forceinline__ f32x4 score(const float* krow, int grp) const {
    const KF kf = load_k(krow, grp);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NI; ++t) acc = step(kf, t, acc);
    return acc;
  }
  // sum of squares of this lane's quarter of the (pre-scaled) query row
  __device__ __forceinline__ float sumsq() const {
    float a = 0.f;
#pragma unroll
    for (int t = 0; t < E; ++t) a = fmaf(q[t], q[t], a);
    return a;
  }
};

// ---- bf16 -----------------------------------------------------------------
__device__ __forceinline__ bf16 scale_bf16(bf16 x, float pre) {
  return f32_to_bf16(bf16_to_f32(x) * pre);  // exact for a power-of-two pre
}

template <>
struct Frag<bf16, 16> {
  static constexpr int LDK = 16 + 8;
  i16x4 q;
  // pre == 1 (a constant at every caller that passes it) takes the row as is
  __device__ __forceinline__ void load_q(const bf16* qrow, int grp, float pre) {
    uint2 v = *reinterpret_cast<const uint2*>(qrow + 4 * grp);
    if (pre == 1.f) {
      q = __builtin_bit_cast(i16x4, v);
      return;
    }
    bf16 e[4] = {static_cast<bf16>(v.x), static_cast<bf16>(v.x >> 16),
                 static_cast<bf16>(v.y), static_cast<bf16>(v.y >> 16)};
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = static_cast<short>(scale_bf16(e[i], pre));
  }
  static constexpr int NI = 1;
  struct KF { i16x4 v; };
  __device__ __forceinline__ static KF load_k(const bf16* krow, int grp) {
    return KF{*reinterpret_cast<const i16x4*>(krow + 4 * grp)};
  }
  __device__ __forceinline__ f32x4 step(const KF& kf, int, f32x4 acc) const {
    return mfma_bf16_16x16x16(kf.v, q, acc);
  }
  __device__ __forceinline__ f32x4 score(const bf16* krow, int grp) const {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    return step(load_k(krow, grp), 0, acc);
  }
  __device__ __forceinline__ float sumsq() const {
    const uint2 w = __builtin_bit_cast(uint2, q);
    return dot2_bf16(w.y, w.y, dot2_bf16(w.x, w.x, 0.f));
  }
};

template <int D>
struct FragBf16Wide {
  static_assert(D == 32 || D == 64 || D == 128, "bf16 wide fragment");
  static constexpr int NI = D / 32;     // 16x16x32 instructions per tile
  static constexpr int LDK = D + 8;
  bf16x8 q[NI];
  // One 16-byte load per half; the power-of-two rescale is exact, so the
  // packed round-to-nearest conversion back to bf16 returns x * pre exactly.
  __device__ __forceinline__ void load_q(const bf16* qrow, int grp, float pre) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int h = 0; h < NI; ++h) {
      const uint4 raw = *reinterpret_cast<const uint4*>(qrow + 32 * h + 8 * grp);
      if (pre == 1.f) {  // a constant at every caller that passes it
        q[h] = __builtin_bit_cast(bf16x8, raw);
        continue;
      }
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bf16x2_t y = {static_cast<__bf16>(__uint_as_float(w[e] << 16) * pre),
                            static_cast<__bf16>(__uint_as_float(w[e] & 0xffff0000u) * pre)};
        o[e] = __builtin_bit_cast(uint32_t, y);
      }
      q[h] = __builtin_bit_cast(bf16x8, o);
    }
  }
  struct KF { bf16x8 v[NI]; };
  __device__ __forceinline__ static KF load_k(const bf16* krow, int grp) {
    KF f;
#pragma unroll
    for (int h = 0; h < NI; ++h) f.v[h] = *reinterpret_cast<const bf16x8*>(krow + 32 * h + 8 * grp);
    return f;
  }
  __device__ __forceinline__ f32x4 step(const KF& kf, int i, f32x4 acc) const {
    return mfma_bf16_16x16x32(kf.v[i], q[i], acc);
  }
  __device__ __forceinline__ f32x4 score(const bf16* krow, int grp) const {
    const KF kf = load_k(krow, grp);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < NI; ++h) acc = step(kf, h, acc);
    return acc;
  }
  __device__ __forceinline__ float sumsq() const {
    float a = 0.f;
#pragma unroll
    for (int h = 0; h < NI; ++h) {
      const uint4 w = __builtin_bit_cast(uint4, q[h]);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) a = dot2_bf16(ww[e], ww[e], a);
    }
    return a;
  }
};

template <>
struct Frag<bf16, 32> : FragBf16Wide<32> {};
template <>
struct Frag<bf16, 64> : FragBf16Wide<64> {};
template <>
struct Frag<bf16, 128> : FragBf16Wide<128> {};

// 1/sqrt(d) is a power of two (d = 4^m): it can be folded into q exactly.
template <int D>
constexpr bool pow2_scale() {
  return D == 4 || D == 16 || D == 64 || D == 256;
}

// Scores of QT query tiles against BT consecutive 16-key tiles starting at
// LDS row `kb` (row stride LDK). The QT*BT MFMA chains are independent and
// issued round-robin; each chain still runs its steps in order 0..NI-1, so
// the rounding is that of a single tile.
template <typename F, int QT, int BT, typename T>
__device__ __forceinline__ void block_scores(const F (&frag)[QT], const T* Ks, int kb, int ldk,
                                             int lane, f32x4 (&s)[QT][BT]) {
  const int col = lane & 15, grp = lane >> 4;
  typename F::KF kf[BT];
#pragma unroll
  for (int t = 0; t < BT; ++t) kf[t] = F::load_k(Ks + (kb + 16 * t + col) * ldk, grp);
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int t = 0; t < BT; ++t) s[qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < F::NI; ++i)
#pragma unroll
    for (int t = 0; t < BT; ++t)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) s[qt][t] = frag[qt].step(kf[t], i, s[qt][t]);
}

// The same product split in two halves, so a caller can issue the LDS reads
// of the next block early and its MFMAs next to unrelated VALU work.
template <typename F, int BT, typename T>
__device__ __forceinline__ void load_block_k(const T* Ks, int kb, int ldk, int lane,
                                             typename F::KF (&kf)[BT]) {
  const int col = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int t = 0; t < BT; ++t) kf[t] = F::load_k(Ks + (kb + 16 * t + col) * ldk, grp);
}

template <typename F, int QT, int BT>
__device__ __forceinline__ void mma_block(const F (&frag)[QT], const typename F::KF (&kf)[BT],
                                          f32x4 (&s)[QT][BT]) {
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int t = 0; t < BT; ++t) s[qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < F::NI; ++i)
#pragma unroll
    for (int t = 0; t < BT; ++t)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) s[qt][t] = frag[qt].step(kf[t], i, s[qt][t]);
}

// Cooperative copy of `rows` rows of a [*, D] matrix into LDS with row stride
// LDK, zero-filling rows [rows, rows_pad). 16-byte vectors; every thread of
// the workgroup participates.
// Loads in flight per thread while staging: a chunk costs one memory round
// trip per kStageBatch * blockDim vectors instead of one per vector.
constexpr int kStageBatch = 4;

template <typename T, int D, int LDK>
__device__ __forceinline__ void stage_rows(T* lds, const T* src, int rows, int rows_pad) {
  constexpr int VE = 16 / sizeof(T);
  constexpr int VPR = D / VE;
  constexpr int U = kStageBatch;
  static_assert(D % VE == 0 && (LDK * sizeof(T)) % 16 == 0, "16-byte staging");
  // the rows are contiguous in global memory: vector v sits at byte 16 v of
  // the chunk (a 32-bit offset from the uniform base)
  const char* base = reinterpret_cast<const char*>(src);
  const int total = rows_pad * VPR;
  const int avail = rows * VPR;  // vectors backed by source rows
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
      if (v < total) *reinterpret_cast<uint4*>(lds + row * LDK + cv * VE) = x[u];
    }
  }
}

// stage_rows of K and the transposed V of the same rows together: every pass
// issues its K and V loads before any LDS write, so a chunk costs one memory
// round trip per pass rather than one for K and then one for V. fp32 V is
// written one element per store (stage_vt); bf16 V four rows per thread
// (stage_vt_quads), whose quad loop has the same trip count as the K loop
// with kStageBatch = 4 vectors per thread. rows_pad is a multiple of 4.
template <typename T, int D, int LDK, int CP>
__device__ __forceinline__ void stage_kv(T* Ks, T* Vt, int ldv, const T* ksrc, const T* vsrc,
                                         int rows, int rows_pad) {
  constexpr int VE = 16 / sizeof(T);
  constexpr int VPR = D / VE;
  constexpr int U = kStageBatch;
  constexpr bool QUADS = sizeof(T) == 2;
  static_assert(D % VE == 0 && (LDK * sizeof(T)) % 16 == 0 && U == 4, "16-byte staging");
  const char* kbase = reinterpret_cast<const char*>(ksrc);
  const char* vbase = reinterpret_cast<const char*>(vsrc);
  const int total = rows_pad * VPR;
  const int avail = rows * VPR;
  const int bd = blockDim.x;
  for (int it = 0; it * U * bd < total; ++it) {
    const int v0 = threadIdx.x + it * U * bd;
    uint4 xk[U], xv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * bd;
      xk[u] = make_uint4(0u, 0u, 0u, 0u);
      if (v < avail) xk[u] = *reinterpret_cast<const uint4*>(kbase + static_cast<uint32_t>(v) * 16u);
    }
    // V: QUADS, quad t = threadIdx.x + it * bd covers rows 4 (t / VPR) .. +3 at
    // vector column t % VPR; otherwise the same vectors as K
    const int t = threadIdx.x + it * bd;
    const int quad = t / VPR, cq = t - quad * VPR, row0 = 4 * quad;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xv[u] = make_uint4(0u, 0u, 0u, 0u);
      if constexpr (QUADS) {
        if (t < total / 4 && row0 + u < rows)
          xv[u] = *reinterpret_cast<const uint4*>(
              vbase + static_cast<uint32_t>((row0 + u) * VPR + cq) * 16u);
      } else {
        const int v = v0 + u * bd;
        if (v < avail) xv[u] = *reinterpret_cast<const uint4*>(vbase + static_cast<uint32_t>(v) * 16u);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * bd, row = v / VPR, cv = v - row * VPR;
      if (v < total) *reinterpret_cast<uint4*>(Ks + row * LDK + cv * VE) = xk[u];
    }
    if constexpr (QUADS) {
      if (t < total / 4) {
        const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&xv[0]);
        const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&xv[1]);
        const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&xv[2]);
        const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&xv[3]);
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          // element e is the low (e even) or high (e odd) half of word e / 2
          const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
          *reinterpret_cast<uint2*>(Vt + (cq * VE + e) * ldv + row0) =
              make_uint2(__builtin_amdgcn_perm(w1[e / 2], w0[e / 2], sel),
                         __builtin_amdgcn_perm(w3[e / 2], w2[e / 2], sel));
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int v = v0 + u * bd, row = v / VPR, cv = v - row * VPR;
        if (v >= total) break;
        T x[VE];
        __builtin_memcpy(x, &xv[u], 16);
#pragma unroll
        for (int e = 0; e < VE; ++e) Vt[(cv * VE + e) * ldv + row] = x[e];
      }
    }
  }
  if constexpr (CP > D) {
    const int pad = (CP - D) * rows_pad;
    for (int v = threadIdx.x; v < pad; v += bd) {
      const int c = D + v / rows_pad, row = v % rows_pad;
      Vt[c * ldv + row] = T(0);
    }
  }
}

// Stage V[rows, D] transposed into Vt[c][key] (row stride ldv), zero-filling
// keys [rows, rows_pad) and channels [D, CP).
template <typename T, int D, int CP>
__device__ __forceinline__ void stage_vt(T* Vt, int ldv, const T* src, int rows, int rows_pad) {
  constexpr int VE = 16 / sizeof(T);
  constexpr int VPR = D / VE;
  constexpr int U = kStageBatch;
  const int total = rows_pad * VPR;
  for (int v0 = threadIdx.x; v0 < total; v0 += U * blockDim.x) {
    uint4 raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * blockDim.x, row = v / VPR, cv = v - row * VPR;
      raw[u] = make_uint4(0u, 0u, 0u, 0u);
      if (v < total && row < rows)
        raw[u] = *reinterpret_cast<const uint4*>(src + static_cast<size_t>(row) * D + cv * VE);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int v = v0 + u * blockDim.x, row = v / VPR, cv = v - row * VPR;
      if (v >= total) break;
      T x[VE];
      __builtin_memcpy(x, &raw[u], 16);
#pragma unroll
      for (int e = 0; e < VE; ++e) Vt[(cv * VE + e) * ldv + row] = x[e];
    }
  }
  if constexpr (CP > D) {
    const int pad = (CP - D) * rows_pad;
    for (int v = threadIdx.x; v < pad; v += blockDim.x) {
      const int c = D + v / rows_pad, row = v % rows_pad;
      Vt[c * ldv + row] = T(0);
    }
  }
}

// As stage_vt, four rows per thread: each thread loads one 16-byte vector
// from each of four consecutive rows and writes, per channel, the four rows'
// elements as one 4-element store (8 bytes for bf16, 16 for fp32) -- a
// quarter of the LDS write instructions of one store per element. rows_pad
// is a multiple of 4; ldv * sizeof(T) a multiple of 4 * sizeof(T).
template <typename T, int D, int CP>
__device__ __forceinline__ void stage_vt_quads(T* Vt, int ldv, const T* src, int rows,
                                               int rows_pad) {
  constexpr int VE = 16 / sizeof(T);
  constexpr int VPR = D / VE;
  static_assert(D % VE == 0, "16-byte staging");
  const char* base = reinterpret_cast<const char*>(src);  // rows contiguous, 16 VPR bytes each
  const int total = (rows_pad / 4) * VPR;
  for (int v = threadIdx.x; v < total; v += blockDim.x) {
    const int quad = v / VPR, cv = v - quad * VPR, row0 = 4 * quad;
    uint4 x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = make_uint4(0u, 0u, 0u, 0u);
      if (row0 + j < rows)
        x[j] = *reinterpret_cast<const uint4*>(
            base + static_cast<uint32_t>((row0 + j) * VPR + cv) * 16u);
    }
    const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&x[0]);
    const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&x[1]);
    const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&x[2]);
    const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&x[3]);
#pragma unroll
    for (int e = 0; e < VE; ++e) {
      T* dst = Vt + (cv * VE + e) * ldv + row0;
      if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(w0[e], w1[e], w2[e], w3[e]);
      } else {
        // element e is the low (e even) or high (e odd) half of word e / 2:
        // one byte permute per pair of rows
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        *reinterpret_cast<uint2*>(dst) =
            make_uint2(__builtin_amdgcn_perm(w1[e / 2], w0[e / 2], sel),
                       __builtin_amdgcn_perm(w3[e / 2], w2[e / 2], sel));
      }
    }
  }
  if constexpr (CP > D) {
    const int pad = (CP - D) * rows_pad;
    for (int v = threadIdx.x; v < pad; v += blockDim.x) {
      const int c = D + v / rows_pad, row = v % rows_pad;
      Vt[c * ldv + row] = T(0);
    }
  }
}

}  // namespace tarmac
