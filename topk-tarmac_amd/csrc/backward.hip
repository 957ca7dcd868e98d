// Backward passes of the attention core (fp32): gradients of the dense core
// and of attention over a fixed peer set -- the latter serves top-k (the set
// the forward retained), the Z-order selector's set and prescore attention.
//
// The reference's Triton kernels are forward-only
// (scripts/bench_attention_core.py:172-176); in training the reference
// differentiates its PyTorch composition with autograd
// (src/agents/mappo.py:192-231 gather path, :361-372 dense path; the step is
// src/training/train_mappo.py:366 and the module benchmark's
// scripts/microbenchmark_comm.py:401). These kernels compute the same
// gradients. The selection itself is piecewise constant in the scores, so,
// as for torch.topk's gather, gradients flow only through the retained
// scores and value rows.
//
// Fixed set, query i with peers j in S_i (scale c = 1/sqrt(d)):
//   s_j = c q_i.k_j, w = softmax(s over S_i), dw_j = dO_i.v_j,
//   D_i = sum_j w_j dw_j, ds_j = w_j (dw_j - D_i),
//   dq_i = c sum_j ds_j k_j,  dk_j += c ds_j q_i,  dv_j += w_j dO_i.
// dk and dv collect contributions from every query that retained j. The
// mask kernel (one workgroup per batch row, while the row's N x N bitmask
// fits LDS) sums them per key in ascending query order, with no float
// atomics; beyond that, or for sets that repeat a peer, they are summed with
// fp32 atomic adds in no fixed order: per-entry lists in LDS (gather form),
// accumulators in LDS, or global memory, whichever fits.
//
// In the mask kernel each query's pass is a single sweep over its set (dq
// from the rescaled sums of e_j dw_j k_j and e_j k_j, see
// fixedset_bwd_row_mask); the per-key pass recomputes each entry from the
// query's statistics.
//
// Dense, self pair excluded: P = softmax(c Q K^T), D_i = dO_i.O_i,
//   dS = P o (dO V^T - D 1^T),  dQ = c dS K,  dK = c dS^T Q,  dV = P^T dO.
// Pass 1 (per query, quad of lanes) forms the row statistics, dQ, and stores
// (logsumexp_i, D_i); pass 2 (per key) forms dK and dV from them. The other
// side's rows stream through LDS in chunks.
#include <algorithm>
#include <type_traits>

#include "frag.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

namespace {

// quad dot: lane (l % 4) holds E of the d channels; the sum lands in all four
template <int E>
__device__ __forceinline__ float quad_dot(const float (&a)[E], const float (&b)[E]) {
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < E; ++c) s = fmaf(a[c], b[c], s);
  return quad_sum(s);
}

// dot over a group of G lanes (2 or 4, aligned): lane (l % G) holds E of the
// d channels; the sum lands in all G lanes
template <int G, int E>
__device__ __forceinline__ float group_dot(const float (&a)[E], const float (&b)[E]) {
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < E; ++c) s = fmaf(a[c], b[c], s);
  if constexpr (G == 2) return s + dpp_mov<kDppQuadXor1>(s);
  else return quad_sum(s);
}

template <int E>
__device__ __forceinline__ void atomic_add_row(float* dst, const float (&x)[E], float w) {
#pragma unroll
  for (int c = 0; c < E; ++c) atomicAdd(dst + c, w * x[c]);
}

}  // namespace

// ---------------------------------------------------------------------------
// fixed peer set
// ---------------------------------------------------------------------------

// A query's softmax statistics over its set: the max m of its exp2-domain
// scores, 1 / sum 2^(s - m), and D = sum_j w_j dw_j.
struct RowStats {
  float m, inv_l, dsum;
};

// One query (a quad of lanes): dq is written and the statistics returned.
// Peers are taken U at a time with their index, K and V loads in flight
// together; when the set fits one batch (kk <= U) the second pass reuses the
// rows from registers. Kb / Vb are the batch row's keys and values, in LDS or
// global memory. For each valid peer, sink(j, p, q, g, ds, w) receives the
// query's contribution to dk_p (scale * ds * q) and dv_p (w * g); every lane
// of the quad calls it.
template <int D, typename I, typename Sink>
__device__ __forceinline__ RowStats fixedset_bwd_row(const float* __restrict__ qrow,
                                                 const float* __restrict__ grow,
                                                 const float* Kb, const float* Vb,
                                                 const I* __restrict__ ir, float* __restrict__ dqrow,
                                                 int N, int kk, float scale, int sub, Sink sink) {
  constexpr int E = D / 4;
  constexpr int U = E <= 4 ? 8 : (E <= 8 ? 4 : 1);  // within 128 VGPRs at 1024 threads
  const float c2 = scale * kLog2eF;  // scores in the exp2 domain
  float q[E], g[E];
  ld_f32<E>(q, qrow + sub * E);
  ld_f32<E>(g, grow + sub * E);
  int p[U];
  float kr[U][E], vr[U][E], sc[U], dw[U];
  auto load_batch = [&](int j0) {
#pragma unroll
    for (int u = 0; u < U; ++u) p[u] = j0 + u < kk ? static_cast<int>(ir[j0 + u]) : 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int pc = min(max(p[u], 0), N - 1);
      ld_f32<E>(kr[u], Kb + static_cast<size_t>(pc) * D + sub * E);
      ld_f32<E>(vr[u], Vb + static_cast<size_t>(pc) * D + sub * E);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      sc[u] = j0 + u < kk ? quad_dot<E>(q, kr[u]) * c2 : -INFINITY;
      dw[u] = quad_dot<E>(g, vr[u]);
    }
  };

  // pass 1: softmax statistics and D = sum_j w_j dw_j (online, per batch)
  float m = -INFINITY, l = 0.f, a = 0.f;
  bool bad = false;
  for (int j0 = 0; j0 < kk; j0 += U) {
    load_batch(j0);
    float mb = m;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      bad |= j0 + u < kk && ((p[u] < 0) | (p[u] >= N));
      mb = fmaxf(mb, sc[u]);
    }
    const float alpha = m == -INFINITY ? 0.f : fast_exp2(m - mb);
    l *= alpha;
    a *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float e = fast_exp2(sc[u] - mb);  // 0 for the -inf padding
      l += e;
      a = fmaf(e, dw[u], a);
    }
    m = mb;
  }
  const float inv_l = 1.f / l;
  const float Dq = a * inv_l;

  // pass 2: ds_j, dq_i, and the scatter into dk, dv
  float dq[E];
#pragma unroll
  for (int c = 0; c < E; ++c) dq[c] = 0.f;
  for (int j0 = 0; j0 < kk; j0 += U) {
    if (kk > U) load_batch(j0);  // else the single batch is still in registers
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j0 + u >= kk) continue;
      const float w = fast_exp2(sc[u] - m) * inv_l;
      const float ds = w * (dw[u] - Dq);
#pragma unroll
      for (int c = 0; c < E; ++c) dq[c] = fmaf(ds, kr[u][c], dq[c]);
      if (p[u] >= 0 && p[u] < N) sink(j0 + u, p[u], q, g, ds, w);
    }
  }
#pragma unroll
  for (int c = 0; c < E; ++c) dq[c] = bad ? __int_as_float(0x7fc00000) : dq[c] * scale;
  st_f32<E>(dqrow + sub * E, dq);
  return RowStats{m, inv_l, Dq};
}

// The scatter of a peer's contribution with fp32 atomic adds (global memory
// or LDS); lane (l % 4) adds its E channels.
template <int D>
struct AtomicSink {
  float* dK;
  float* dV;
  int sub;
  float scale;
  template <int E>
  __device__ __forceinline__ void operator()(int, int p, const float (&q)[E], const float (&g)[E],
                                             float ds, float w) const {
    atomic_add_row<E>(dK + static_cast<size_t>(p) * D + sub * E, q, ds * scale);
    atomic_add_row<E>(dV + static_cast<size_t>(p) * D + sub * E, g, w);
  }
};

// Global accumulation: one quad per query over the whole grid; dK, dV are
// zeroed by zero_fill_kernel first.
template <int D, typename I>
__global__ void __launch_bounds__(256)
fixedset_bwd_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                    const float* __restrict__ V, const float* __restrict__ dO,
                    const I* __restrict__ Idx, float* __restrict__ dQ, float* __restrict__ dK,
                    float* __restrict__ dV, int B, int N, int kk, float scale) {
  const int blk = xcd_logical_block(blockIdx.x, gridDim.x);  // a batch row's blocks share an XCD
  const long row = (static_cast<long>(blk) * blockDim.x + threadIdx.x) >> 2;
  if (row >= static_cast<long>(B) * N) return;  // whole quads exit together
  const int b = static_cast<int>(row / N);
  const size_t boff = static_cast<size_t>(b) * N * D;
  const int sub = threadIdx.x & 3;
  fixedset_bwd_row<D, I>(Q + static_cast<size_t>(row) * D, dO + static_cast<size_t>(row) * D,
                         Kx + boff, V + boff, Idx + static_cast<size_t>(row) * kk,
                         dQ + static_cast<size_t>(row) * D, N, kk, scale, sub,
                         AtomicSink<D>{dK + boff, dV + boff, sub, scale});
}

__global__ void __launch_bounds__(256) zero_fill_kernel(float4* __restrict__ a, float4* __restrict__ b,
                                                        long n4) {
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  for (long t = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; t < n4;
       t += static_cast<long>(gridDim.x) * blockDim.x) {
    a[t] = z;
    b[t] = z;
  }
}

// LDS accumulation: one workgroup (256 query quads) per batch row sums dK
// and dV for its N keys in LDS and writes them once. With STAGE, the row's K
// and V are staged in LDS too, so the peer gathers are LDS reads.
template <int D, typename I, bool STAGE>
__global__ void __launch_bounds__(1024)
fixedset_bwd_lds_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                        const float* __restrict__ V, const float* __restrict__ dO,
                        const I* __restrict__ Idx, float* __restrict__ dQ,
                        float* __restrict__ dK, float* __restrict__ dV, int N, int kk,
                        float scale) {
  extern __shared__ __align__(16) float acc[];  // dK, dV rows (then K, V rows), N * D each
  const int b = blockIdx.x;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const int nd = N * D;
  float* dKs = acc;
  float* dVs = acc + nd;
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int t = threadIdx.x; t < nd / 2; t += blockDim.x) reinterpret_cast<float4*>(acc)[t] = z;
  const float* Kb = Kx + boff;
  const float* Vb = V + boff;
  if constexpr (STAGE) {
    float* Ks = acc + 2 * nd;
    float* Vs = Ks + nd;
    for (int t = threadIdx.x; t < nd / 4; t += blockDim.x) {
      reinterpret_cast<float4*>(Ks)[t] = reinterpret_cast<const float4*>(Kb)[t];
      reinterpret_cast<float4*>(Vs)[t] = reinterpret_cast<const float4*>(Vb)[t];
    }
    Kb = Ks;
    Vb = Vs;
  }
  __syncthreads();
  const int quads = blockDim.x >> 2;
  for (int i0 = 0; i0 < N; i0 += quads) {
    const int i = i0 + (threadIdx.x >> 2);
    if (i < N) {  // whole quads agree
      const size_t row = static_cast<size_t>(b) * N + i;
      const int sub = threadIdx.x & 3;
      fixedset_bwd_row<D, I>(Q + row * D, dO + row * D, Kb, Vb, Idx + row * kk, dQ + row * D, N,
                             kk, scale, sub, AtomicSink<D>{dKs, dVs, sub, scale});
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < nd / 4; t += blockDim.x) {
    reinterpret_cast<float4*>(dK + boff)[t] = reinterpret_cast<const float4*>(dKs)[t];
    reinterpret_cast<float4*>(dV + boff)[t] = reinterpret_cast<const float4*>(dVs)[t];
  }
}

// Gather form (no float atomics), one workgroup per batch row:
//   1. K, V rows in LDS; each query (a quad) computes dq and, per peer slot
//      e = i*kk + j, ds and w into LDS, counting its peers per key;
//   2. an exclusive scan of the counts gives each key's list start; every
//      entry takes a place in its key's list (an integer atomic);
//   3. Q, dO rows replace K, V in LDS; each key (a quad) sums its list:
//      dk = scale * sum ds q_i, dv = sum w g_i, written once.
// Entry order within a key's list follows the atomics, so dk, dv are summed
// in no fixed order, like the atomic forms.
template <int D>
struct GatherSink {
  float* e_ds;
  float* e_w;
  int* cnt;
  int row0;  // i * kk
  int sub;
  template <int E>
  __device__ __forceinline__ void operator()(int j, int p, const float (&)[E], const float (&)[E],
                                             float ds, float w) const {
    if (sub == 0) {
      e_ds[row0 + j] = ds;
      e_w[row0 + j] = w;
      atomicAdd(cnt + p, 1);
    }
  }
};

size_t fixedset_gather_lds_bytes(int N, int D, int kk) {
  return (static_cast<size_t>(2) * N * D + 3 * static_cast<size_t>(N) * kk +
          3 * static_cast<size_t>(N) + 1) * 4;
}

template <int D, typename I>
__global__ void __launch_bounds__(1024)
fixedset_bwd_gather_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                           const float* __restrict__ V, const float* __restrict__ dO,
                           const I* __restrict__ Idx, float* __restrict__ dQ,
                           float* __restrict__ dK, float* __restrict__ dV, int N, int kk,
                           float scale) {
  constexpr int E = D / 4;
  extern __shared__ __align__(16) float smem[];
  const int nd = N * D, nk = N * kk;
  float* rows = smem;                 // [2 * N * D]: K, V, then Q, dO
  float* e_ds = rows + 2 * nd;        // [N * kk]
  float* e_w = e_ds + nk;             // [N * kk]
  int* perm = reinterpret_cast<int*>(e_w + nk);  // [N * kk]: entries in key order
  int* cnt = perm + nk;               // [N]
  int* start = cnt + N;               // [N + 1]
  int* cursor = start + N + 1;        // [N]
  const int b = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
  const size_t boff = static_cast<size_t>(b) * nd;
  const int sub = tid & 3, quads = nt >> 2;

  for (int t = tid; t < N; t += nt) { cnt[t] = 0; cursor[t] = 0; }
  for (int t = tid; t < nd / 4; t += nt) {
    reinterpret_cast<float4*>(rows)[t] = reinterpret_cast<const float4*>(Kx + boff)[t];
    reinterpret_cast<float4*>(rows + nd)[t] = reinterpret_cast<const float4*>(V + boff)[t];
  }
  __syncthreads();
  // 1. per query
  for (int i0 = 0; i0 < N; i0 += quads) {
    const int i = i0 + (tid >> 2);
    if (i < N) {  // whole quads agree
      const size_t row = static_cast<size_t>(b) * N + i;
      fixedset_bwd_row<D, I>(Q + row * D, dO + row * D, rows, rows + nd, Idx + row * kk,
                             dQ + row * D, N, kk, scale, sub,
                             GatherSink<D>{e_ds, e_w, cnt, i * kk, sub});
    }
  }
  __syncthreads();
  // 2. list starts (one wavefront scans), then places
  if (tid < 64) {
    int carry = 0;
    for (int c0 = 0; c0 < N; c0 += 64) {
      const int c = c0 + tid < N ? cnt[c0 + tid] : 0;
      int x = c;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (tid >= o) x += y;
      }
      if (c0 + tid < N) start[c0 + tid] = carry + x - c;
      carry += __shfl(x, 63);
    }
    if (tid == 0) start[N] = carry;
  }
  __syncthreads();
  for (int e = tid; e < nk; e += nt) {
    const int i = e / kk;
    const int p = static_cast<int>(Idx[(static_cast<size_t>(b) * N + i) * kk + (e - i * kk)]);
    if (p >= 0 && p < N) perm[start[p] + atomicAdd(cursor + p, 1)] = e;
  }
  for (int t = tid; t < nd / 4; t += nt) {  // K, V are no longer read
    reinterpret_cast<float4*>(rows)[t] = reinterpret_cast<const float4*>(Q + boff)[t];
    reinterpret_cast<float4*>(rows + nd)[t] = reinterpret_cast<const float4*>(dO + boff)[t];
  }
  __syncthreads();
  // 3. per key
  for (int j0 = 0; j0 < N; j0 += quads) {
    const int j = j0 + (tid >> 2);
    if (j >= N) continue;
    float dk[E], dv[E];
#pragma unroll
    for (int c = 0; c < E; ++c) dk[c] = dv[c] = 0.f;
    const int s1 = start[j + 1];
    for (int s = start[j]; s < s1; ++s) {
      const int e = perm[s];
      const int i = e / kk;
      const float ds = e_ds[e], w = e_w[e];
      float q[E], g[E];
      ld_f32<E>(q, rows + i * D + sub * E);
      ld_f32<E>(g, rows + nd + i * D + sub * E);
#pragma unroll
      for (int c = 0; c < E; ++c) {
        dk[c] = fmaf(ds, q[c], dk[c]);
        dv[c] = fmaf(w, g[c], dv[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < E; ++c) dk[c] *= scale;
    st_f32<E>(dK + boff + static_cast<size_t>(j) * D + sub * E, dk);
    st_f32<E>(dV + boff + static_cast<size_t>(j) * D + sub * E, dv);
  }
}

// Mask form (no float atomics, sums in ascending query order), one workgroup
// per batch row:
//   1. each query (a quad) writes dq, keeps its statistics in LDS and sets
//      bit i of row p of an N x N bitmask for every peer p (integer LDS
//      atomics; an OR lands the same whatever the order);
//   2. each key p (a quad) walks the set bits of its row in ascending query
//      order and, for every query i that retains it, recomputes s, w, dw and
//      ds from the saved statistics (the same operations on the same lanes
//      as step 1) and sums dk = scale * sum ds q_i, dv = sum w g_i, written
//      once. LDS holds N statistics and N^2 bits, plus (STAGE) the row's K
//      and V, then Q and dO.
// A set that names one peer twice does not fit a bitmask: a batch row where
// step 1 finds a repeated peer is summed with global fp32 atomics instead
// (its dK, dV rows zeroed first), in no fixed order.
struct MaskSink {
  unsigned* mask;
  int* repeated;
  int words;  // per mask row
  int i;
  int sub;
  template <int E>
  __device__ __forceinline__ void operator()(int, int p, const float (&)[E], const float (&)[E],
                                             float, float) const {
    if (sub == 0) {
      const unsigned bit = 1u << (i & 31);
      if (atomicOr(mask + static_cast<size_t>(p) * words + (i >> 5), bit) & bit) *repeated = 1;
    }
  }
};

// One query (a group of G lanes) in one pass over its set, for the mask form:
// with e_j = 2^(s_j - m) under a running maximum m,
//   dq = sum_j w_j (dw_j - D) k_j = (sum_j e_j dw_j k_j - D sum_j e_j k_j) / l,
// l = sum_j e_j, D = sum_j e_j dw_j / l, all four sums rescaled as m grows;
// each valid peer sets its bit in the mask (sink). Returns the statistics the
// per-key pass recomputes the entries from.
template <int D, int G, typename I>
__device__ __forceinline__ RowStats fixedset_bwd_row_mask(const float* __restrict__ qrow,
                                                      const float* __restrict__ grow,
                                                      const float* Kb, const float* Vb,
                                                      const I* __restrict__ ir,
                                                      float* __restrict__ dqrow, int N, int kk,
                                                      float scale, int sub, MaskSink sink) {
  constexpr int E = D / G;
  constexpr int U = E <= 4 ? 8 : (E <= 8 ? 4 : 1);
  const float c2 = scale * kLog2eF;  // scores in the exp2 domain
  float q[E], g[E];
  ld_f32<E>(q, qrow + sub * E);
  ld_f32<E>(g, grow + sub * E);
  float m = -INFINITY, l = 0.f, a = 0.f, ak[E], bk[E];
#pragma unroll
  for (int c = 0; c < E; ++c) ak[c] = bk[c] = 0.f;
  bool bad = false;
  for (int j0 = 0; j0 < kk; j0 += U) {
    int p[U];
    float kr[U][E], vr[U][E], sc[U], dw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) p[u] = j0 + u < kk ? static_cast<int>(ir[j0 + u]) : 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int pc = min(max(p[u], 0), N - 1);
      ld_f32<E>(kr[u], Kb + static_cast<size_t>(pc) * D + sub * E);
      ld_f32<E>(vr[u], Vb + static_cast<size_t>(pc) * D + sub * E);
    }
    float mb = m;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      sc[u] = j0 + u < kk ? group_dot<G, E>(q, kr[u]) * c2 : -INFINITY;
      dw[u] = group_dot<G, E>(g, vr[u]);
      bad |= j0 + u < kk && ((p[u] < 0) | (p[u] >= N));
      mb = fmaxf(mb, sc[u]);
    }
    const float alpha = m == -INFINITY ? 0.f : fast_exp2(m - mb);
    l *= alpha;
    a *= alpha;
#pragma unroll
    for (int c = 0; c < E; ++c) {
      ak[c] *= alpha;
      bk[c] *= alpha;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float e = fast_exp2(sc[u] - mb);  // 0 for the -inf padding
      const float ed = e * dw[u];
      l += e;
      a += ed;
#pragma unroll
      for (int c = 0; c < E; ++c) {
        ak[c] = fmaf(ed, kr[u][c], ak[c]);
        bk[c] = fmaf(e, kr[u][c], bk[c]);
      }
      if (j0 + u < kk && p[u] >= 0 && p[u] < N) sink(j0 + u, p[u], q, g, 0.f, 0.f);
    }
    m = mb;
  }
  const float inv_l = 1.f / l;
  const float Dq = a * inv_l;
  float dq[E];
#pragma unroll
  for (int c = 0; c < E; ++c)
    dq[c] = bad ? __int_as_float(0x7fc00000) : fmaf(-Dq, bk[c], ak[c]) * inv_l * scale;
  st_f32<E>(dqrow + sub * E, dq);
  return RowStats{m, inv_l, Dq};
}

size_t fixedset_mask_lds_bytes(int N, int D, bool stage) {
  const size_t words = (static_cast<size_t>(N) + 31) / 32;
  return (stage ? 8 * static_cast<size_t>(N) * D : 0) + 16 * static_cast<size_t>(N) +
         4 * static_cast<size_t>(N) * words + 16;
}

template <int D, int G, typename I, bool STAGE>
__global__ void __launch_bounds__(1024)
fixedset_bwd_mask_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                         const float* __restrict__ V, const float* __restrict__ dO,
                         const I* __restrict__ Idx, float* __restrict__ dQ,
                         float* __restrict__ dK, float* __restrict__ dV, int N, int kk,
                         float scale) {
  constexpr int E = D / G;  // channels per lane
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int nd = N * D, words = (N + 31) >> 5;
  float* rows = reinterpret_cast<float*>(smem_raw);  // STAGE: K, V, then Q, dO
  float4* stats = reinterpret_cast<float4*>(smem_raw + (STAGE ? 8 * static_cast<size_t>(nd) : 0));
  unsigned* mask = reinterpret_cast<unsigned*>(stats + N);  // [N keys][words]
  int* repeated = reinterpret_cast<int*>(mask + static_cast<size_t>(N) * words);
  const int b = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
  const size_t boff = static_cast<size_t>(b) * nd;
  const int sub = tid & (G - 1), groups = nt / G;

  for (int t = tid; t < N * words; t += nt) mask[t] = 0u;
  if (tid == 0) *repeated = 0;
  const float* Kb = Kx + boff;
  const float* Vb = V + boff;
  if constexpr (STAGE) {
    for (int t = tid; t < nd / 4; t += nt) {
      reinterpret_cast<float4*>(rows)[t] = reinterpret_cast<const float4*>(Kb)[t];
      reinterpret_cast<float4*>(rows + nd)[t] = reinterpret_cast<const float4*>(Vb)[t];
    }
    Kb = rows;
    Vb = rows + nd;
  }
  __syncthreads();
  // 1. per query (a group of G lanes)
  for (int i0 = 0; i0 < N; i0 += groups) {
    const int i = i0 + tid / G;
    if (i < N) {  // whole groups agree
      const size_t row = static_cast<size_t>(b) * N + i;
      const RowStats r = fixedset_bwd_row_mask<D, G, I>(Q + row * D, dO + row * D, Kb, Vb,
                                                     Idx + row * kk, dQ + row * D, N, kk, scale,
                                                     sub, MaskSink{mask, repeated, words, i, sub});
      if (sub == 0) stats[i] = make_float4(r.m, r.inv_l, r.dsum, 0.f);
    }
  }
  __syncthreads();
  if (*repeated) {  // uniform over the workgroup
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int t = tid; t < nd / 4; t += nt) {
      reinterpret_cast<float4*>(dK + boff)[t] = z;
      reinterpret_cast<float4*>(dV + boff)[t] = z;
    }
    __syncthreads();
    const int sub4 = tid & 3, quads = nt >> 2;
    for (int i0 = 0; i0 < N; i0 += quads) {
      const int i = i0 + (tid >> 2);
      if (i < N) {
        const size_t row = static_cast<size_t>(b) * N + i;
        fixedset_bwd_row<D, I>(Q + row * D, dO + row * D, Kb, Vb, Idx + row * kk, dQ + row * D, N,
                               kk, scale, sub4, AtomicSink<D>{dK + boff, dV + boff, sub4, scale});
      }
    }
    return;
  }
  const float* Qb = Q + boff;
  const float* Gb = dO + boff;
  if constexpr (STAGE) {  // K, V are read from global memory below
    for (int t = tid; t < nd / 4; t += nt) {
      reinterpret_cast<float4*>(rows)[t] = reinterpret_cast<const float4*>(Qb)[t];
      reinterpret_cast<float4*>(rows + nd)[t] = reinterpret_cast<const float4*>(Gb)[t];
    }
    Qb = rows;
    Gb = rows + nd;
    __syncthreads();
  }
  // 2. per key (a group of G lanes)
  const float c2 = scale * kLog2eF;
  for (int p0 = 0; p0 < N; p0 += groups) {
    const int p = p0 + tid / G;
    if (p >= N) break;  // whole groups agree; no barrier follows
    float kr[E], vr[E], dk[E], dv[E];
    ld_f32<E>(kr, Kx + boff + static_cast<size_t>(p) * D + sub * E);
    ld_f32<E>(vr, V + boff + static_cast<size_t>(p) * D + sub * E);
#pragma unroll
    for (int c = 0; c < E; ++c) dk[c] = dv[c] = 0.f;
    const unsigned* mrow = mask + static_cast<size_t>(p) * words;
    for (int w = 0; w < words; ++w) {
      unsigned bits = mrow[w];
      while (bits) {  // the same bits on the group's lanes
        const int i = (w << 5) + __builtin_ctz(bits);
        bits &= bits - 1u;
        float q[E], g[E];
        ld_f32<E>(q, Qb + static_cast<size_t>(i) * D + sub * E);
        ld_f32<E>(g, Gb + static_cast<size_t>(i) * D + sub * E);
        const float4 st = stats[i];
        const float sc = group_dot<G, E>(q, kr) * c2;
        const float dw = group_dot<G, E>(g, vr);
        const float wgt = fast_exp2(sc - st.x) * st.y;
        const float ds = wgt * (dw - st.z);
#pragma unroll
        for (int c = 0; c < E; ++c) {
          dk[c] = fmaf(ds, q[c], dk[c]);
          dv[c] = fmaf(wgt, g[c], dv[c]);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < E; ++c) dk[c] *= scale;
    st_f32<E>(dK + boff + static_cast<size_t>(p) * D + sub * E, dk);
    st_f32<E>(dV + boff + static_cast<size_t>(p) * D + sub * E, dv);
  }
}

// ---------------------------------------------------------------------------
// dense
// ---------------------------------------------------------------------------
//
// P = softmax(scale * Q K^T) (self pair excluded), dP = dO V^T,
// dS = P * (dP - rowsum(dO * O)), dQ = scale * dS K, dK = scale * dS^T Q,
// dV = P^T dO, on fp32 MFMA in two passes:
//   pass 1 (per query tile, keys streamed): S^T tiles as in the forward kernel
//     (lane l: query l%16, keys 4*(l/16)+r), a first sweep for the row's
//     log2-domain logsumexp, a second for dQ^T += K^T dS^T, whose B operand
//     is each lane's own dS (contraction slot j of step u = key 4j+u);
//   pass 2 (per key tile, queries streamed): S tiles (lane l: key l%16,
//     queries 4*(l/16)+r), so dV^T += dO^T P and dK^T += Q^T dS take P and
//     dS as B operands from the lane's own registers in the same way.
// Pass 1 writes the per-query statistics pass 2 needs into the workspace:
// stats[b][0][i] = log2-domain logsumexp of the scaled scores,
// stats[b][1][i] = dO_i . O_i.

template <int D>
constexpr int bwd_block_tiles() { return D <= 32 ? 4 : 2; }

// A^T-operand product: acc[h] (16 output channels x 16 columns) +=
// Xt[16h + col][c0 + 4*grp + u] * w[u] over u, Xt transposed in LDS.
template <int NX, int NH>
__device__ __forceinline__ void mma_t(f32x4 (&acc)[NX][NH], const float* Xt, int ldt, int c0,
                                      int lane, const float (&w)[NX][4]) {
  const int col = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const f32x4 xv = *reinterpret_cast<const f32x4*>(Xt + (16 * h + col) * ldt + c0 + 4 * grp);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int x = 0; x < NX; ++x) acc[x][h] = mfma_f32_16x16x4(xv[u], w[x][u], acc[x][h]);
  }
}

template <int D, int QT>
__global__ void __launch_bounds__(256)
dense_bwd_dq_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                    const float* __restrict__ V, const float* __restrict__ O,
                    const float* __restrict__ dO, float* __restrict__ dQ,
                    float* __restrict__ stats, int have_lse, int N, int n_qblk, int kc,
                    float scale, int nblocks) {
  using F = Frag<float, D>;
  constexpr int E = D / 4, LDK = F::LDK, NH = (D + 15) / 16, CP = 16 * NH;
  constexpr int BT = bwd_block_tiles<D>(), BK = 16 * BT;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int kcp = (kc + BK - 1) / BK * BK, ldt = kcp + 4;
  float* Ks = reinterpret_cast<float*>(smem_raw);
  float* Vs = Ks + static_cast<size_t>(kcp) * LDK;
  float* Kt = Vs + static_cast<size_t>(kcp) * LDK;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qblk = blk - b * n_qblk;
  const int q0 = (qblk * nw + wave) * 16 * QT;
  const int col = lane & 15, grp = lane >> 4;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const float c2 = scale * kLog2eF;

  F fq[QT], fg[QT];
  float Di[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const size_t row = boff + static_cast<size_t>(min(q0 + 16 * qt + col, N - 1)) * D;
    fq[qt].load_q(Q + row, grp, c2);
    fg[qt].load_q(dO + row, grp, 1.f);
    float o[E];
    ld_f32<E>(o, O + row + grp * E);
    float dd = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) dd = fmaf(fg[qt].q[e], o[e], dd);
    dd += __shfl_xor(dd, 16);
    dd += __shfl_xor(dd, 32);
    Di[qt] = dd;
  }

  // sweep 1 (unless the forward saved it): per-lane running max / sum of
  // 2^s, then combined per query into the log2-domain logsumexp
  const bool single = N <= kc && !have_lse;  // sweep 1 stages everything once
  float lse[QT];
  if (have_lse) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
      lse[qt] = stats[static_cast<size_t>(b) * 2 * N + min(q0 + 16 * qt + col, N - 1)];
  } else {
    float m[QT], l[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) { m[qt] = -INFINITY; l[qt] = 0.f; }
    for (int c0 = 0; c0 < N; c0 += kc) {
      const int cn = min(kc, N - c0), cnp = (cn + BK - 1) / BK * BK;
      __syncthreads();
      stage_rows<float, D, LDK>(Ks, Kx + boff + static_cast<size_t>(c0) * D, cn, cnp);
      if (single) {
        stage_rows<float, D, LDK>(Vs, V + boff + static_cast<size_t>(c0) * D, cn, cnp);
        stage_vt<float, D, CP>(Kt, ldt, Kx + boff + static_cast<size_t>(c0) * D, cn, cnp);
      }
      __syncthreads();
      if (q0 >= N) continue;
      for (int kb0 = 0; kb0 < cnp; kb0 += BK) {
        f32x4 st[QT][BT];
        block_scores<F, QT, BT>(fq, Ks, kb0, LDK, lane, st);
        const int kabs = c0 + kb0;
        const bool edge = (q0 < kabs + BK && kabs < q0 + 16 * QT) || kabs + BK > c0 + cn;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          float s[BT][4];
          float mloc = -INFINITY;
#pragma unroll
          for (int t = 0; t < BT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int key = kabs + 16 * t + 4 * grp + r;
              s[t][r] = (edge && (key >= c0 + cn || key == q0 + 16 * qt + col)) ? -INFINITY
                                                                                  : st[qt][t][r];
              mloc = fmaxf(mloc, s[t][r]);
            }
          const float m_new = fmaxf(m[qt], mloc);
          if (m_new != -INFINITY) {
            float acc = l[qt] * fast_exp2(m[qt] - m_new);
#pragma unroll
            for (int t = 0; t < BT; ++t)
#pragma unroll
              for (int r = 0; r < 4; ++r) acc += fast_exp2(s[t][r] - m_new);
            l[qt] = acc;
            m[qt] = m_new;
          }
        }
      }
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float mm = fmaxf(m[qt], __shfl_xor(m[qt], 16));
      mm = fmaxf(mm, __shfl_xor(mm, 32));
      float ll = (m[qt] == -INFINITY) ? 0.f : l[qt] * fast_exp2(m[qt] - mm);
      ll += __shfl_xor(ll, 16);
      ll += __shfl_xor(ll, 32);
      lse[qt] = mm + log2f(ll);
    }
  }

  // sweep 2: dQ^T += K^T dS^T
  f32x4 acc[QT][NH];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int h = 0; h < NH; ++h) acc[qt][h] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < N; c0 += kc) {
    const int cn = min(kc, N - c0), cnp = (cn + BK - 1) / BK * BK;
    if (!single) {
      __syncthreads();
      stage_rows<float, D, LDK>(Ks, Kx + boff + static_cast<size_t>(c0) * D, cn, cnp);
      stage_rows<float, D, LDK>(Vs, V + boff + static_cast<size_t>(c0) * D, cn, cnp);
      stage_vt<float, D, CP>(Kt, ldt, Kx + boff + static_cast<size_t>(c0) * D, cn, cnp);
      __syncthreads();
    }
    if (q0 >= N) continue;
    for (int kb0 = 0; kb0 < cnp; kb0 += BK) {
      f32x4 st[QT][BT], dp[QT][BT];
      block_scores<F, QT, BT>(fq, Ks, kb0, LDK, lane, st);
      block_scores<F, QT, BT>(fg, Vs, kb0, LDK, lane, dp);
      const int kabs = c0 + kb0;
      const bool edge = (q0 < kabs + BK && kabs < q0 + 16 * QT) || kabs + BK > c0 + cn;
#pragma unroll
      for (int t = 0; t < BT; ++t) {
        float ds[QT][4];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = kabs + 16 * t + 4 * grp + r;
            float p = fast_exp2(st[qt][t][r] - lse[qt]);
            if (edge && (key >= c0 + cn || key == q0 + 16 * qt + col)) p = 0.f;
            ds[qt][r] = p * (dp[qt][t][r] - Di[qt]);
          }
        mma_t<QT, NH>(acc, Kt, ldt, kb0 + 16 * t, lane, ds);
      }
    }
  }
  if (q0 >= N) return;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = q0 + 16 * qt + col;
    if (qi >= N) continue;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const int cbase = 16 * h + 4 * grp;
      if (cbase < D) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = acc[qt][h][r] * scale;
        st_f32<4>(dQ + boff + static_cast<size_t>(qi) * D + cbase, o);
      }
    }
    if (grp == 0) {
      if (!have_lse) stats[static_cast<size_t>(b) * 2 * N + qi] = lse[qt];
      stats[static_cast<size_t>(b) * 2 * N + N + qi] = Di[qt];
    }
  }
}

template <int D, int KT>
__global__ void __launch_bounds__(256)
dense_bwd_dkv_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                     const float* __restrict__ V, const float* __restrict__ dO,
                     const float* __restrict__ stats, float* __restrict__ dK,
                     float* __restrict__ dV, int N, int n_kblk, int qc, float scale,
                     int nblocks) {
  using F = Frag<float, D>;
  constexpr int LDK = F::LDK, NH = (D + 15) / 16, CP = 16 * NH;
  constexpr int BT = bwd_block_tiles<D>(), BQ = 16 * BT;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int qcp = (qc + BQ - 1) / BQ * BQ, ldt = qcp + 4;
  float* Qs = reinterpret_cast<float*>(smem_raw);
  float* Gs = Qs + static_cast<size_t>(qcp) * LDK;
  float* Qt = Gs + static_cast<size_t>(qcp) * LDK;
  float* Gt = Qt + static_cast<size_t>(CP) * ldt;
  float* Ls = Gt + static_cast<size_t>(CP) * ldt;
  float* Ds = Ls + qcp;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_kblk, kblk = blk - b * n_kblk;
  const int k0 = (kblk * nw + wave) * 16 * KT;
  const int col = lane & 15, grp = lane >> 4;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const float* st_b = stats + static_cast<size_t>(b) * 2 * N;

  F fk[KT], fv[KT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    const size_t row = boff + static_cast<size_t>(min(k0 + 16 * kt + col, N - 1)) * D;
    fk[kt].load_q(Kx + row, grp, scale * kLog2eF);
    fv[kt].load_q(V + row, grp, 1.f);
  }
  f32x4 dk[KT][NH], dv[KT][NH];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int h = 0; h < NH; ++h) dk[kt][h] = dv[kt][h] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int c0 = 0; c0 < N; c0 += qc) {
    const int cn = min(qc, N - c0), cnp = (cn + BQ - 1) / BQ * BQ;
    __syncthreads();
    stage_rows<float, D, LDK>(Qs, Q + boff + static_cast<size_t>(c0) * D, cn, cnp);
    stage_rows<float, D, LDK>(Gs, dO + boff + static_cast<size_t>(c0) * D, cn, cnp);
    stage_vt<float, D, CP>(Qt, ldt, Q + boff + static_cast<size_t>(c0) * D, cn, cnp);
    stage_vt<float, D, CP>(Gt, ldt, dO + boff + static_cast<size_t>(c0) * D, cn, cnp);
    for (int t = threadIdx.x; t < cnp; t += blockDim.x) {
      Ls[t] = t < cn ? st_b[c0 + t] : INFINITY;  // padded queries: p = 0
      Ds[t] = t < cn ? st_b[N + c0 + t] : 0.f;
    }
    __syncthreads();
    if (k0 >= N) continue;
    for (int qb0 = 0; qb0 < cnp; qb0 += BQ) {
      f32x4 s[KT][BT], dp[KT][BT];
      block_scores<F, KT, BT>(fk, Qs, qb0, LDK, lane, s);   // S: query 4*grp+r, key col
      block_scores<F, KT, BT>(fv, Gs, qb0, LDK, lane, dp);
      const int qabs = c0 + qb0;
      const bool diag = k0 < qabs + BQ && qabs < k0 + 16 * KT;  // wave-uniform
#pragma unroll
      for (int t = 0; t < BT; ++t) {
        const int qrow = qb0 + 16 * t + 4 * grp;
        const f32x4 lse = *reinterpret_cast<const f32x4*>(Ls + qrow);
        const f32x4 dd = *reinterpret_cast<const f32x4*>(Ds + qrow);
        float p[KT][4], ds[KT][4];
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[kt][r] = fast_exp2(s[kt][t][r] - lse[r]);
            if (diag && c0 + qrow + r == k0 + 16 * kt + col) p[kt][r] = 0.f;
            ds[kt][r] = p[kt][r] * (dp[kt][t][r] - dd[r]);
          }
        mma_t<KT, NH>(dv, Gt, ldt, qb0 + 16 * t, lane, p);
        mma_t<KT, NH>(dk, Qt, ldt, qb0 + 16 * t, lane, ds);
      }
    }
  }
  if (k0 >= N) return;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    const int kj = k0 + 16 * kt + col;
    if (kj >= N) continue;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const int cbase = 16 * h + 4 * grp;
      if (cbase < D) {
        float a[4], v4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          a[r] = dk[kt][h][r] * scale;
          v4[r] = dv[kt][h][r];
        }
        st_f32<4>(dK + boff + static_cast<size_t>(kj) * D + cbase, a);
        st_f32<4>(dV + boff + static_cast<size_t>(kj) * D + cbase, v4);
      }
    }
  }
}

// LDS bytes of the two passes for a chunk of `c` rows.
template <int D>
constexpr size_t dq_lds_bytes(int c) {
  constexpr int CP = 16 * ((D + 15) / 16);
  return (static_cast<size_t>(c) * 2 * (D + 4) + static_cast<size_t>(CP) * (c + 4)) * 4;
}
template <int D>
constexpr size_t dkv_lds_bytes(int c) {
  constexpr int CP = 16 * ((D + 15) / 16);
  return (static_cast<size_t>(c) * 2 * (D + 4) + static_cast<size_t>(2) * CP * (c + 4) +
          static_cast<size_t>(2) * c) * 4;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

constexpr size_t kBwdLdsBudget = 65536;
// the mask kernel runs one 1024-thread workgroup per CU whatever its LDS
constexpr size_t kMaskLdsBudget = 160 * 1024;

template <int D, typename I>
static hipError_t launch_fixedset_bwd_t(const FixedsetBwdArgs& a) {
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  const I* idx = static_cast<const I*>(a.idx);
  const size_t row_bytes = static_cast<size_t>(a.N) * D * sizeof(float);
  const size_t mask_stage = fixedset_mask_lds_bytes(a.N, D, true);
  const size_t mask_plain = fixedset_mask_lds_bytes(a.N, D, false);
  // lanes per query / key: pairs where quads would take a second, partly
  // idle round and 512 pairs cover the row in one (256 < N <= 512), while a
  // lane's share (D / 2 channels) stays within the register budget
  // (B=256 N=384 k=95: 97 -> 90 us)
  auto launch_mask = [&](auto g, auto stage, size_t lds) {
    hipLaunchKernelGGL((fixedset_bwd_mask_kernel<D, decltype(g)::value, I, decltype(stage)::value>),
                       dim3(a.B), dim3(1024), lds, st, a.q, a.k, a.v, a.dout, idx, a.dq, a.dk, a.dv,
                       a.N, a.kk, a.scale);
    return hipGetLastError();
  };
  using G2 = std::integral_constant<int, 2>;
  using G4 = std::integral_constant<int, 4>;
  const bool pairs = D <= 16 && a.N > 256 && a.N <= 512;
  // d = 128: a lane's share of a row exceeds the 128 VGPRs of a 1024-thread
  // workgroup, so those rows take the per-query kernel below
  if constexpr (D <= 64) {
    if (mask_stage <= kMaskLdsBudget) {  // statistics, bitmask and the row's K, V fit LDS
      if constexpr (D <= 16)
        if (pairs) return launch_mask(G2{}, std::true_type{}, mask_stage);
      return launch_mask(G4{}, std::true_type{}, mask_stage);
    }
    if (mask_plain <= kMaskLdsBudget) {  // statistics and bitmask fit LDS
      if constexpr (D <= 16)
        if (pairs) return launch_mask(G2{}, std::false_type{}, mask_plain);
      return launch_mask(G4{}, std::false_type{}, mask_plain);
    }
    const size_t gather_lds = fixedset_gather_lds_bytes(a.N, D, a.kk);
    if (gather_lds <= kBwdLdsBudget) {  // rows and per-entry lists fit LDS
      hipLaunchKernelGGL((fixedset_bwd_gather_kernel<D, I>), dim3(a.B), dim3(1024), gather_lds, st,
                         a.q, a.k, a.v, a.dout, idx, a.dq, a.dk, a.dv, a.N, a.kk, a.scale);
      return hipGetLastError();
    }
    if (4 * row_bytes <= kBwdLdsBudget) {  // dK, dV and the staged K, V fit LDS
      hipLaunchKernelGGL((fixedset_bwd_lds_kernel<D, I, true>), dim3(a.B), dim3(1024), 4 * row_bytes,
                         st, a.q, a.k, a.v, a.dout, idx, a.dq, a.dk, a.dv, a.N, a.kk, a.scale);
      return hipGetLastError();
    }
    if (2 * row_bytes <= kBwdLdsBudget) {  // the batch row's dK, dV fit LDS
      hipLaunchKernelGGL((fixedset_bwd_lds_kernel<D, I, false>), dim3(a.B), dim3(1024), 2 * row_bytes,
                         st, a.q, a.k, a.v, a.dout, idx, a.dq, a.dk, a.dv, a.N, a.kk, a.scale);
      return hipGetLastError();
    }
  }
  const long n4 = static_cast<long>(a.B) * a.N * D / 4;
  const int zgrid = static_cast<int>(std::min<long>((n4 + 255) / 256, 4096));
  hipLaunchKernelGGL(zero_fill_kernel, dim3(zgrid), dim3(256), 0, st,
                     reinterpret_cast<float4*>(a.dk), reinterpret_cast<float4*>(a.dv), n4);
  const long rows = static_cast<long>(a.B) * a.N;
  const int grid = static_cast<int>((rows * 4 + 255) / 256);
  hipLaunchKernelGGL((fixedset_bwd_kernel<D, I>), dim3(grid), dim3(256), 0, st, a.q, a.k, a.v,
                     a.dout, idx, a.dq, a.dk, a.dv, a.B, a.N, a.kk, a.scale);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_fixedset_bwd(const FixedsetBwdArgs& a) {
  return a.idx_is_i64 ? launch_fixedset_bwd_t<D, int64_t>(a) : launch_fixedset_bwd_t<D, int32_t>(a);
}

hipError_t run_fixedset_bwd(const FixedsetBwdArgs& a) {
  switch (a.d) {
    case 8: return launch_fixedset_bwd<8>(a);
    case 16: return launch_fixedset_bwd<16>(a);
    case 32: return launch_fixedset_bwd<32>(a);
    case 64: return launch_fixedset_bwd<64>(a);
    case 128: return launch_fixedset_bwd<128>(a);
  }
  return hipErrorInvalidValue;
}

template <int D>
static hipError_t launch_dense_bwd(const DenseBwdArgs& a) {
  constexpr int T = 2;                              // 16-row tiles per wavefront
  constexpr int BQ = 16 * bwd_block_tiles<D>();
  const int waves = (a.N + 16 * T - 1) / (16 * T);
  const int nw = waves >= 4 ? 4 : waves;
  const int per = 16 * T * nw;
  const int nblk = (a.N + per - 1) / per;
  const int nblocks = a.B * nblk;
  // largest chunk (multiple of the block) within the LDS budget, capped at N
  const int npad = (a.N + BQ - 1) / BQ * BQ;
  // d = 128: one 32-row block of the dK/dV pass needs 71 KB, so those rows
  // take up to 80 KB (two workgroups per CU)
  constexpr size_t budget = D > 64 ? 80 * 1024 : kBwdLdsBudget;
  static_assert(dq_lds_bytes<D>(BQ) <= budget && dkv_lds_bytes<D>(BQ) <= budget,
                "one block of each backward pass fits LDS");
  int kc = BQ, qc = BQ;
  while (kc + BQ <= npad && dq_lds_bytes<D>(kc + BQ) <= budget) kc += BQ;
  while (qc + BQ <= npad && dkv_lds_bytes<D>(qc + BQ) <= budget) qc += BQ;
  if (kc >= a.N) kc = a.N;
  if (qc >= a.N) qc = a.N;
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  const size_t lds_q = dq_lds_bytes<D>((kc + BQ - 1) / BQ * BQ);
  const size_t lds_kv = dkv_lds_bytes<D>((qc + BQ - 1) / BQ * BQ);
  hipLaunchKernelGGL((dense_bwd_dq_kernel<D, T>), dim3(nblocks), dim3(64 * nw), lds_q, st, a.q,
                     a.k, a.v, a.out, a.dout, a.dq, a.stats, a.stats_ready, a.N, nblk, kc, a.scale,
                     nblocks);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((dense_bwd_dkv_kernel<D, T>), dim3(nblocks), dim3(64 * nw), lds_kv, st, a.q,
                     a.k, a.v, a.dout, a.stats, a.dk, a.dv, a.N, nblk, qc, a.scale, nblocks);
  return hipGetLastError();
}

hipError_t run_dense_bwd(const DenseBwdArgs& a) {
  switch (a.d) {
    case 8: return launch_dense_bwd<8>(a);
    case 16: return launch_dense_bwd<16>(a);
    case 32: return launch_dense_bwd<32>(a);
    case 64: return launch_dense_bwd<64>(a);
    case 128: return launch_dense_bwd<128>(a);
  }
  return hipErrorInvalidValue;
}

}  // namespace tarmac
