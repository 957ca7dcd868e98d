// Exact score-then-select top-k attention (k <= 4) for fp32 and bf16 inputs
// at d = 16, on 32-key x 32-query score tiles.
//
// Reference behaviour: src/kernels/fused_topk_attention.py:211-333
// (fused_topk_attention_tiled) and src/kernels/streaming_topk_attention.py:
// 66-258 (streaming_topk_attention, incl. the retained-index output), with the
// tie rule score desc / index asc (:37-44).
//
// The algorithm is topk_packed_kernel's split-bf16 path: scores from bf16
// MFMA on three-way split operands (x = hi + mid + lo), the key in the low
// mantissa bits of each score, a value-only list of K + 2 entries per lane,
// a merge, a proof against the split error bound after canonical rescoring of
// the K + 1 candidates, and the per-query exact pass for what the proof
// leaves open. The tile is v_mfma_f32_32x32x16_bf16's: lane l owns query
// l % 32 and, of each 32-key tile, keys 8 (i / 4) + 4 (l / 32) + i % 4
// (i = 0..15). A query's keys are spread over two lanes instead of four, so
// the merge is one row swap, and each lane proves, rescores and finishes one
// query where a lane of the 16 x 16 kernel handles two (one per query tile);
// the scan itself costs the same MFMA cycles and list operations per score.
// Memory round trips per wave: the query row is read while the key row is
// staged (one trip, not two), and the value rows of all K + 1 candidates are
// read with the rows their rescoring needs (one trip at the end, not two).
//
// Fields: a score's low fb bits (fb = packed width of the row, at most 10:
// N <= 1024) hold its key's index in the row with bit 2 (the lane half) left
// zero; the merge sets bit 2, so a merged entry's field IS its key.
#include <type_traits>

#include "exact.hpp"
#include "frag.hpp"
#include "select.hpp"
#include "split.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// D += A(32x16) * B(16x32), bf16 inputs (gfx950). Lane l supplies
// A[l%32][8*(l/32)+e] and B[8*(l/32)+e][l%32], e = 0..7; element i of the
// result is D[8*(i/4) + 4*(l/32) + i%4][l%32].
__device__ __forceinline__ f32x16 mfma_bf16_32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

namespace {

constexpr int kS32Waves = 4;     // waves per workgroup (128 queries)
constexpr int kS32Tiles = 2;     // 32-key tiles per scan block (64 keys = kBlockKeys)
constexpr int kS32LDK = SplitFrag<16>::LDK;  // split row: lo[16] hi[16] mid[16] pad[8]
constexpr int kB32LDK = 16 + 8;              // bf16 row: x[16] pad[8]

// Split key fragment of one 32-key tile: row kb + l % 32, elements
// 8 (l / 32) .. +7 of each part.
struct KSplit32 {
  bf16x8 h, m, l;
};
__device__ __forceinline__ KSplit32 load_ksplit32(const bf16* Ks, int row, int half) {
  const bf16* r = Ks + row * kS32LDK + 8 * half;
  KSplit32 f;
  f.h = *reinterpret_cast<const bf16x8*>(r + SplitFrag<16>::OFF_H);
  f.m = *reinterpret_cast<const bf16x8*>(r + SplitFrag<16>::OFF_M);
  f.l = *reinterpret_cast<const bf16x8*>(r + SplitFrag<16>::OFF_L);
  return f;
}

// The six products of magnitude >= 2^-16 of q.k (split.hpp): kh.qh, km.qh,
// kh.qm, km.qm, kl.qh, kh.ql.
__device__ __forceinline__ f32x16 split32_score(const KSplit32& k, bf16x8 qh, bf16x8 qm,
                                                bf16x8 ql) {
  f32x16 acc = {};
  acc = mfma_bf16_32x32x16(k.h, qh, acc);
  acc = mfma_bf16_32x32x16(k.m, qh, acc);
  acc = mfma_bf16_32x32x16(k.h, qm, acc);
  acc = mfma_bf16_32x32x16(k.m, qm, acc);
  acc = mfma_bf16_32x32x16(k.l, qh, acc);
  acc = mfma_bf16_32x32x16(k.h, ql, acc);
  return acc;
}

// Canonical fp32 score (split.hpp / exact.hpp order: element kk*4 + t at step
// t, slot kk) of the query row qs (scaled by the power-of-two 1/4 already)
// against key row krow (fp32, or bf16 widened exactly).
template <typename T>
__device__ __forceinline__ float canon16(const float (&qs)[16], const T* krow) {
  float k[16];
  ld_row<T, 16>(k, krow);
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = fmaf(qs[4 * kk + t], k[4 * kk + t], acc);
  return acc;
}

}  // namespace

// One wave: 32 queries q0 .. q0 + 31 of batch row b; the workgroup's waves
// share one staged copy of the key row. kc: keys per LDS chunk (kc >= N:
// resident row). fm: the field mask of the row (2^fb - 1). T = float: the
// split-bf16 scores above; T = bf16: the inputs are bf16 already, so a score
// is one 32x32x16 product of the rows as they are (exact products, fp32
// accumulation) and the same packing, proof (the bf16 accumulation bound)
// and canonical rescoring of the inputs widened to fp32 follow.
template <int K, typename T>
__global__ void __launch_bounds__(64 * kS32Waves)
topk_split32_kernel(const T* __restrict__ Q, const T* __restrict__ Kx,
                    const T* __restrict__ V, T* __restrict__ O, int32_t* __restrict__ Idx,
                    int N, int n_qblk, int kc, float scale, int nblocks, uint32_t fm_arg) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int D = 16;
  constexpr int C = K + 1;   // candidates rescored
  constexpr int L = K + 2;   // lane and merged lists: the candidates and the (K+2)-th
  constexpr int BT = kS32Tiles;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  unsigned* kmax_slot = reinterpret_cast<unsigned*>(smem_raw);
  bf16* Ks = reinterpret_cast<bf16*>(smem_raw + 16);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qblk = blk - b * n_qblk;
  const int q0 = (qblk * kS32Waves + wave) * 32;  // uniform
  const int qc = lane & 31, half = lane >> 5;
  const int qi = q0 + qc;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const T* Qb = Q + boff;
  const T* Kb = Kx + boff;
  const uint32_t FM = fm_arg;

  // query fragment: elements 8 half .. +7 of row qi, read now and split after
  // the first chunk's keys are staged (their loads overlap)
  float qx[8];
  ld_row<T, 8>(qx, Qb + static_cast<size_t>(min(qi, N - 1)) * D + 8 * half);
  bf16x8 qh, qm, ql;
  float qn2 = 0.f;
  auto split_query = [&]() {
    const float(&x)[8] = qx;
    if constexpr (BF) {
      // bf16 values widened exactly: the fragment is the row as it is
      uint32_t h4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        h4[e] = (__float_as_uint(x[2 * e]) >> 16) | (__float_as_uint(x[2 * e + 1]) & 0xffff0000u);
      qh = __builtin_bit_cast(bf16x8, h4);
    } else {
      uint32_t h4[4], m4[4], l4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split3_pair(x[2 * e], x[2 * e + 1], h4[e], m4[e], l4[e]);
      qh = __builtin_bit_cast(bf16x8, h4);
      qm = __builtin_bit_cast(bf16x8, m4);
      ql = __builtin_bit_cast(bf16x8, l4);
    }
    float n2 = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) n2 = fmaf(x[e], x[e], n2);
    const LanePair p = swap_rows32(__float_as_uint(n2));
    qn2 = __uint_as_float(p.a) + __uint_as_float(p.b);  // same order in both lanes
  };

  float pv[L];
#pragma unroll
  for (int m = 0; m < L; ++m) pv[m] = kMasked;
  float kmax2 = 0.f;
  uint32_t nfmask;  // the field mask's complement in a VGPR (pack_field_u)
  asm volatile("v_mov_b32 %0, %1" : "=v"(nfmask) : "s"(~fm_arg));

  // one key chunk: stage it (split rows and the chunk's max |k|^2), then scan
  // it. The first chunk is peeled so the query's split can wait on the
  // staged keys without the query registers living across the loop.
  auto chunk = [&](int c0, auto first) {
    const int cn = min(kc, N - c0);
    const int cnb = (cn + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
    __syncthreads();
    if (threadIdx.x == 0) *kmax_slot = 0u;
    float mine;
    if constexpr (BF) {
      mine = stage_bf16_norm<D, kB32LDK>(Ks, Kb + static_cast<size_t>(c0) * D, cn, cnb);
    } else {
      bool exact_split = true;  // unused: rescoring reads the global rows
      mine = stage_split<D>(Ks, Kb + static_cast<size_t>(c0) * D, cn, cnb, exact_split);
    }
    const float wmax = wave_max_rows(mine);
    if constexpr (decltype(first)::value) {
      // tie the query's split to the staged keys, so the compiler cannot
      // wait on the query row before the key loads are issued
      asm volatile("" : "+v"(qx[0]), "+v"(qx[1]), "+v"(qx[2]), "+v"(qx[3]), "+v"(qx[4]),
                   "+v"(qx[5]), "+v"(qx[6]), "+v"(qx[7]) : "v"(mine));
      split_query();
    }
    __syncthreads();
    if (lane == 0) atomicMax(kmax_slot, __float_as_uint(wmax));
    if (q0 < N) {
      const int kend = c0 + cn;
      for (int kb0 = 0; kb0 < cnb; kb0 += 32 * BT) {
        const int kabs = c0 + kb0;
        f32x16 s[BT];
#pragma unroll
        for (int t = 0; t < BT; ++t) {
          if constexpr (BF) {
            const bf16x8 kf =
                *reinterpret_cast<const bf16x8*>(Ks + (kb0 + 32 * t + qc) * kB32LDK + 8 * half);
            s[t] = mfma_bf16_32x32x16(kf, qh, f32x16{});
          } else {
            const KSplit32 kf = load_ksplit32(Ks, kb0 + 32 * t + qc, half);
            s[t] = split32_score(kf, qh, qm, ql);
          }
        }
        // element i of tile t: key kabs + 32 t + 8 (i / 4) + 4 half + i % 4;
        // the field leaves bit 2 (half) for the merge
#pragma unroll
        for (int t = 0; t < BT; ++t)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            s[t][i] = pack_field_u(
                s[t][i], static_cast<uint32_t>(kabs + 32 * t + 8 * (i >> 2) + (i & 3)), nfmask);
        // the self pair (in the tiles that overlap the wave's queries: one
        // when the chunk starts at a multiple of 32 keys, two otherwise) and
        // keys past the chunk end
#pragma unroll
        for (int t = 0; t < BT; ++t) {
          const int kt = kabs + 32 * t;
          if (kt < q0 + 32 && q0 < kt + 32) {  // wave-uniform
            const int dq = qi - kt - 4 * half;
#pragma unroll
            for (int i = 0; i < 16; ++i)
              if (8 * (i >> 2) + (i & 3) == dq) s[t][i] = kMasked;
          }
        }
        if (kabs + 32 * BT > kend) {
#pragma unroll
          for (int t = 0; t < BT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i)
              if (kabs + 32 * t + 8 * (i >> 2) + 4 * half + (i & 3) >= kend) s[t][i] = kMasked;
        }
#pragma unroll
        for (int t = 0; t < BT; ++t)
#pragma unroll
          for (int i = 0; i < 16; ++i) vinsert<L>(pv, s[t][i]);
      }
    }
    __syncthreads();
    kmax2 = fmaxf(kmax2, __uint_as_float(*kmax_slot));
  };
  chunk(0, std::true_type{});
  for (int c0 = kc; c0 < N; c0 += kc) chunk(c0, std::false_type{});
  if (q0 >= N) return;

  // ---- merge the two lane lists of each query: one row swap -------------
  // Both lanes insert the upper half's entries into the lower half's list,
  // in the same order, so they end with identical lists.
  float pl[L];
  {
    float a[L], o[L];
#pragma unroll
    for (int m = 0; m < L; ++m) {
      const LanePair p =
          swap_rows32(__float_as_uint(pv[m]) | (static_cast<uint32_t>(half) << 2));
      a[m] = __uint_as_float(p.a);
      o[m] = __uint_as_float(p.b);
    }
#pragma unroll
    for (int m = 0; m < L; ++m) vinsert<L>(a, o[m]);
#pragma unroll
    for (int m = 0; m < L; ++m) pl[m] = a[m];
  }
  int cand[C];
#pragma unroll
  for (int m = 0; m < C; ++m)
    cand[m] = pl[m] < kMaskedBelow ? -1 : static_cast<int>(__float_as_uint(pl[m]) & FM);

  // ---- rescore the K + 1 candidates canonically, prove --------------------
  // Lane half h rescores candidates h, h + 2, ...; a row swap shares them.
  // The value rows (this lane's 8 channels) of every candidate are read with
  // the query and key rows, so the aggregation waits on no further trip.
  const T* Vb = V + boff + 8 * half;
  float vpre[C][8];
#pragma unroll
  for (int m = 0; m < C; ++m)
    ld_row<T, 8>(vpre[m], Vb + static_cast<size_t>(min(max(cand[m], 0), N - 1)) * D);
  float val[K];
  int ix[K];
  bool ok;
  {
    float qs[16];
    ld_row<T, 16>(qs, Qb + static_cast<size_t>(min(qi, N - 1)) * D);
#pragma unroll
    for (int e = 0; e < 16; ++e) qs[e] *= scale;  // 1/4: exact
    float cv[C];
#pragma unroll
    for (int u = 0; u < (C + 1) / 2; ++u) {
      const int m = 2 * u + half;
      int c = -1;
#pragma unroll
      for (int mm = 0; mm < C; ++mm)
        if (mm == m) c = cand[mm];
      const float e = canon16(qs, Kb + static_cast<size_t>(min(max(c, 0), N - 1)) * D);
      const LanePair p = swap_rows32(__float_as_uint(c < 0 ? -INFINITY : e));
      cv[2 * u] = __uint_as_float(p.a);
      if (2 * u + 1 < C) cv[2 * u + 1] = __uint_as_float(p.b);
    }
    int ci[C];
#pragma unroll
    for (int m = 0; m < C; ++m) ci[m] = cand[m];
    sort_lex<C>(cv, ci);
    // every key outside the candidates scores at most the (K+2)-th entry's
    // ceiling plus the split (or bf16 accumulation) error
    const float nprod = proof_norm(qn2, kmax2);
    const float bound = (trunc_ceiling(pl[K + 1], FM) + packed_eps<D>() * nprod) * scale;
    ok = qi >= N || (nprod < kPackedNormLimit && bound < cv[K - 1]);
#pragma unroll
    for (int m = 0; m < K; ++m) {
      val[m] = cv[m];
      ix[m] = ci[m];
    }
  }

  // ---- the exact pass for unproven queries (rare), then finish ------------
  if (!__all(ok)) {
    unsigned long long todo = __ballot(half == 0 && !ok);
    while (todo != 0ull) {
      const int c = __builtin_ctzll(todo);
      todo &= todo - 1ull;
      float ev[K];
      int ei[K];
      const int qx = q0 + c;
      exact_query_topk_lanes<T, D, K, 1>(
          Qb + static_cast<size_t>(qx) * D,
          [&](int j) { return Kb + static_cast<size_t>(j) * D; }, N, qx, scale, lane, ev, ei);
      if (qc == c) {
#pragma unroll
        for (int m = 0; m < K; ++m) { val[m] = ev[m]; ix[m] = ei[m]; }
      }
    }
  }
  if (qi >= N) return;
  // k-softmax over the K retained scores (score desc) and the gathered
  // aggregation: lane half h writes channels 8 h .. 8 h + 7
  const float mx = val[0];
  float acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = 0.f;
  float den = 0.f;
#pragma unroll
  for (int m = 0; m < K; ++m) {
    const float w = fast_exp2((val[m] - mx) * kLog2eF);
    den += w;
    // the row among the prefetched candidates' (the exact pass may retain
    // another key: read it then)
    float vr[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vr[e] = vpre[0][e];
    bool found = ix[m] == cand[0];
#pragma unroll
    for (int c = 1; c < C; ++c) {
      const bool hit = ix[m] == cand[c] && !found;
#pragma unroll
      for (int e = 0; e < 8; ++e) vr[e] = hit ? vpre[c][e] : vr[e];
      found = found || hit;
    }
    if (!found) ld_row<T, 8>(vr, Vb + static_cast<size_t>(min(max(ix[m], 0), N - 1)) * D);
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = fmaf(w, vr[c], acc[c]);
  }
  const float inv = 1.f / den;
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] *= inv;
  st_row<T, 8>(O + boff + static_cast<size_t>(qi) * D + 8 * half, acc);
  if (Idx != nullptr && half == 0) {
    int32_t* dst = Idx + (static_cast<size_t>(b) * N + qi) * K;
#pragma unroll
    for (int m = 0; m < K; ++m) dst[m] = ix[m];
  }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------

size_t split32_lds_bytes(int dtype, int kc) {
  const int kcb = (kc + kBlockKeys - 1) / kBlockKeys * kBlockKeys;
  return 16 + static_cast<size_t>(kcb) * (dtype == kBf16 ? kB32LDK : kS32LDK) * 2;
}

// Rows of up to 256 keys: a longer row's split copy (112 bytes a key) would
// leave a CU fewer than four four-wave workgroups (N = 512: two), where the
// 16 x 16 kernel's eight-wave workgroups keep sixteen waves per CU.
bool split32_supported(const TopkArgs& a) {
  // bf16 rows take 48 bytes a key: a resident row of up to 1024 keys (the
  // most the packed fields name) leaves three workgroups per CU
  const int max_n = a.dtype == kBf16 ? 1024 : 256;
  return (a.dtype == kF32 || a.dtype == kBf16) && a.d == 16 && a.topk <= 4 && a.N <= max_n &&
         a.select == kSelTopk;
}

template <int K, typename T>
static void launch_split32_t(const TopkArgs& a, int nblocks, int n_qblk, uint32_t fm) {
  hipLaunchKernelGGL((topk_split32_kernel<K, T>), dim3(nblocks), dim3(64 * kS32Waves),
                     split32_lds_bytes(a.dtype, a.key_chunk), static_cast<hipStream_t>(a.stream),
                     static_cast<const T*>(a.q), static_cast<const T*>(a.k),
                     static_cast<const T*>(a.v), static_cast<T*>(a.out), a.idx, a.N, n_qblk,
                     a.key_chunk, a.scale, nblocks, fm);
}

template <int K>
static void launch_split32_k(const TopkArgs& a, int nblocks, int n_qblk, uint32_t fm) {
  if (a.dtype == kBf16) launch_split32_t<K, bf16>(a, nblocks, n_qblk, fm);
  else launch_split32_t<K, float>(a, nblocks, n_qblk, fm);
}

hipError_t run_topk_split32(const TopkArgs& a) {
  if (!split32_supported(a)) return hipErrorInvalidValue;
  const int qb = 32 * kS32Waves;
  const int n_qblk = (a.N + qb - 1) / qb;
  const int nblocks = a.B * n_qblk;
  // the fewest bits that name every key of the row's whole 32-key tiles
  const int n32 = (a.N + 31) / 32 * 32;
  int fb = 5;
  while ((1 << fb) < n32) ++fb;
  const uint32_t fm = (1u << fb) - 1u;
  switch (a.topk) {
    case 1: launch_split32_k<1>(a, nblocks, n_qblk, fm); break;
    case 2: launch_split32_k<2>(a, nblocks, n_qblk, fm); break;
    case 3: launch_split32_k<3>(a, nblocks, n_qblk, fm); break;
    default: launch_split32_k<4>(a, nblocks, n_qblk, fm); break;
  }
  return hipGetLastError();
}

}  // namespace tarmac
