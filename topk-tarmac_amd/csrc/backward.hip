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
// dk and dv collect contributions from every query that retained j, with
// fp32 atomic adds (accumulation order is not fixed): in LDS, one workgroup
// per batch row, when the row's dK and dV fit 64 KiB; else in global memory.
//
// Dense, self pair excluded: P = softmax(c Q K^T), D_i = dO_i.O_i,
//   dS = P o (dO V^T - D 1^T),  dQ = c dS K,  dK = c dS^T Q,  dV = P^T dO.
// Pass 1 (per query, quad of lanes) forms the row statistics, dQ, and stores
// (logsumexp_i, D_i); pass 2 (per key) forms dK and dV from them. The other
// side's rows stream through LDS in chunks.
#include "frag.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

namespace {

// quad dot: lane (l % 4) holds E of the d channels; the sum lands in all four
__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 1);
  return x + __shfl_xor(x, 2);
}

template <int E>
__device__ __forceinline__ float quad_dot(const float (&a)[E], const float (&b)[E]) {
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < E; ++c) s = fmaf(a[c], b[c], s);
  return quad_sum(s);
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

// One query (a quad of lanes): dq is written; the dk / dv rows of its peers
// receive atomic adds (global memory or LDS). Peers are taken U at a time
// with all their index, K and V loads in flight together; when the set fits
// one batch (kk <= U) the second pass reuses the rows from registers.
template <int D, typename I>
__device__ __forceinline__ void fixedset_bwd_row(const float* __restrict__ qrow,
                                                 const float* __restrict__ grow,
                                                 const float* __restrict__ Kb,
                                                 const float* __restrict__ Vb,
                                                 const I* __restrict__ ir, float* __restrict__ dqrow,
                                                 float* dK, float* dV, int N, int kk, float scale,
                                                 int sub) {
  constexpr int E = D / 4;
  constexpr int U = E <= 4 ? 8 : (E <= 8 ? 4 : 2);
  float q[E], g[E];
  ld_f32<E>(q, qrow + sub * E);
  ld_f32<E>(g, grow + sub * E);
  int p[U];
  float kr[U][E], vr[U][E], sc[U], dw[U];
  auto load_batch = [&](int j0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = j0 + u < kk;
      p[u] = live ? static_cast<int>(ir[j0 + u]) : 0;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int pc = min(max(p[u], 0), N - 1);
      ld_f32<E>(kr[u], Kb + static_cast<size_t>(pc) * D + sub * E);
      ld_f32<E>(vr[u], Vb + static_cast<size_t>(pc) * D + sub * E);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      sc[u] = j0 + u < kk ? quad_dot<E>(q, kr[u]) * scale : -INFINITY;
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
    const float alpha = m == -INFINITY ? 0.f : expf(m - mb);
    l *= alpha;
    a *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float e = sc[u] == -INFINITY ? 0.f : expf(sc[u] - mb);
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
      const float w = expf(sc[u] - m) * inv_l;
      const float ds = w * (dw[u] - Dq);
#pragma unroll
      for (int c = 0; c < E; ++c) dq[c] = fmaf(ds, kr[u][c], dq[c]);
      if (p[u] >= 0 && p[u] < N) {
        atomic_add_row<E>(dK + static_cast<size_t>(p[u]) * D + sub * E, q, ds * scale);
        atomic_add_row<E>(dV + static_cast<size_t>(p[u]) * D + sub * E, g, w);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < E; ++c) dq[c] = bad ? __int_as_float(0x7fc00000) : dq[c] * scale;
  st_f32<E>(dqrow + sub * E, dq);
}

// Global accumulation: one quad per query over the whole grid; dK, dV must
// be zero on entry.
template <int D, typename I>
__global__ void __launch_bounds__(256)
fixedset_bwd_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                    const float* __restrict__ V, const float* __restrict__ dO,
                    const I* __restrict__ Idx, float* __restrict__ dQ, float* __restrict__ dK,
                    float* __restrict__ dV, int B, int N, int kk, float scale) {
  const long row = (static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x) >> 2;
  if (row >= static_cast<long>(B) * N) return;  // whole quads exit together
  const int b = static_cast<int>(row / N);
  const size_t boff = static_cast<size_t>(b) * N * D;
  fixedset_bwd_row<D, I>(Q + static_cast<size_t>(row) * D, dO + static_cast<size_t>(row) * D,
                         Kx + boff, V + boff, Idx + static_cast<size_t>(row) * kk,
                         dQ + static_cast<size_t>(row) * D, dK + boff, dV + boff, N, kk, scale,
                         threadIdx.x & 3);
}

// LDS accumulation: one workgroup (256 query quads) per batch row sums dK and dV for its N keys
// in LDS (fast atomics, no zeroing pass), then adds them to dK, dV once.
template <int D, typename I>
__global__ void __launch_bounds__(1024)
fixedset_bwd_lds_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                        const float* __restrict__ V, const float* __restrict__ dO,
                        const I* __restrict__ Idx, float* __restrict__ dQ,
                        float* __restrict__ dK, float* __restrict__ dV, int N, int kk,
                        float scale) {
  extern __shared__ __align__(16) float acc[];  // dK rows then dV rows, N * D each
  const int b = blockIdx.x;
  const size_t boff = static_cast<size_t>(b) * N * D;
  float* dKs = acc;
  float* dVs = acc + static_cast<size_t>(N) * D;
  for (int t = threadIdx.x; t < 2 * N * D; t += blockDim.x) acc[t] = 0.f;
  __syncthreads();
  const int quads = blockDim.x >> 2;
  for (int i0 = 0; i0 < N; i0 += quads) {
    const int i = i0 + (threadIdx.x >> 2);
    if (i < N) {  // whole quads agree
      const size_t row = static_cast<size_t>(b) * N + i;
      fixedset_bwd_row<D, I>(Q + row * D, dO + row * D, Kx + boff, V + boff, Idx + row * kk,
                             dQ + row * D, dKs, dVs, N, kk, scale, threadIdx.x & 3);
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < N * D; t += blockDim.x) {
    dK[boff + t] += dKs[t];
    dV[boff + t] += dVs[t];
  }
}

// ---------------------------------------------------------------------------
// dense
// ---------------------------------------------------------------------------

// rows of the other side staged per LDS pass (two padded row arrays <= 48 KiB)
template <int D>
constexpr int bwd_chunk() { return D <= 16 ? 256 : (D <= 32 ? 128 : 64); }

// Pass 1: one quad per query; K and V of the batch row stream through LDS.
template <int D>
__global__ void __launch_bounds__(256)
dense_bwd_q_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                   const float* __restrict__ V, const float* __restrict__ O,
                   const float* __restrict__ dO, float* __restrict__ dQ,
                   float* __restrict__ stats, int N, int n_qblk, float scale) {
  constexpr int E = D / 4;
  constexpr int LD = D + 4;  // padded LDS row (floats)
  constexpr int kBwdChunk = bwd_chunk<D>();
  __shared__ __align__(16) float Ks[kBwdChunk * LD];
  __shared__ __align__(16) float Vs[kBwdChunk * LD];
  const int b = blockIdx.x / n_qblk, qb = blockIdx.x - b * n_qblk;
  const int sub = threadIdx.x & 3;
  const int i_raw = qb * (blockDim.x >> 2) + (threadIdx.x >> 2);
  const bool live = i_raw < N;
  const int i = live ? i_raw : N - 1;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const size_t roff = boff + static_cast<size_t>(i) * D + sub * E;
  float q[E], g[E], o[E];
  ld_f32<E>(q, Q + roff);
  ld_f32<E>(g, dO + roff);
  ld_f32<E>(o, O + roff);
  const float Dq = quad_dot<E>(g, o);

  float m = -INFINITY, l = 0.f;
  float dq[E];
#pragma unroll
  for (int c = 0; c < E; ++c) dq[c] = 0.f;
  // two sweeps over the key chunks: statistics, then gradients
  for (int sweep = 0; sweep < 2; ++sweep) {
    for (int c0 = 0; c0 < N; c0 += kBwdChunk) {
      const int cn = min(kBwdChunk, N - c0);
      __syncthreads();
      stage_rows<float, D, LD>(Ks, Kx + boff + static_cast<size_t>(c0) * D, cn, cn);
      if (sweep == 1) stage_rows<float, D, LD>(Vs, V + boff + static_cast<size_t>(c0) * D, cn, cn);
      __syncthreads();
      for (int jj = 0; jj < cn; ++jj) {
        const int j = c0 + jj;
        float kr[E];
        ld_f32<E>(kr, Ks + jj * LD + sub * E);
        const float s = quad_dot<E>(q, kr) * scale;
        if (sweep == 0) {
          if (j != i) {
            const float m_new = fmaxf(m, s);
            l = l * (m == -INFINITY ? 0.f : expf(m - m_new)) + expf(s - m_new);
            m = m_new;
          }
        } else {
          float vr[E];
          ld_f32<E>(vr, Vs + jj * LD + sub * E);
          const float p = j == i ? 0.f : expf(s - m) / l;
          const float ds = p * (quad_dot<E>(g, vr) - Dq);
#pragma unroll
          for (int c = 0; c < E; ++c) dq[c] = fmaf(ds, kr[c], dq[c]);
        }
      }
    }
  }
  if (!live) return;
#pragma unroll
  for (int c = 0; c < E; ++c) dq[c] *= scale;
  st_f32<E>(dQ + roff, dq);
  if (sub == 0) {
    float* st = stats + (static_cast<size_t>(b) * N + i) * 2;
    st[0] = m + logf(l);
    st[1] = Dq;
  }
}

// Pass 2: one quad per key; Q, dO and the query statistics stream through LDS.
template <int D>
__global__ void __launch_bounds__(256)
dense_bwd_kv_kernel(const float* __restrict__ Q, const float* __restrict__ Kx,
                    const float* __restrict__ V, const float* __restrict__ dO,
                    const float* __restrict__ stats, float* __restrict__ dK,
                    float* __restrict__ dV, int N, int n_kblk, float scale) {
  constexpr int E = D / 4;
  constexpr int LD = D + 4;
  constexpr int kBwdChunk = bwd_chunk<D>();
  __shared__ __align__(16) float Qs[kBwdChunk * LD];
  __shared__ __align__(16) float Gs[kBwdChunk * LD];
  __shared__ __align__(16) float Ss[kBwdChunk * 2];
  const int b = blockIdx.x / n_kblk, kb = blockIdx.x - b * n_kblk;
  const int sub = threadIdx.x & 3;
  const int j_raw = kb * (blockDim.x >> 2) + (threadIdx.x >> 2);
  const bool live = j_raw < N;
  const int j = live ? j_raw : N - 1;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const size_t roff = boff + static_cast<size_t>(j) * D + sub * E;
  float kr[E], vr[E];
  ld_f32<E>(kr, Kx + roff);
  ld_f32<E>(vr, V + roff);
  float dk[E], dv[E];
#pragma unroll
  for (int c = 0; c < E; ++c) dk[c] = dv[c] = 0.f;
  for (int c0 = 0; c0 < N; c0 += kBwdChunk) {
    const int cn = min(kBwdChunk, N - c0);
    __syncthreads();
    stage_rows<float, D, LD>(Qs, Q + boff + static_cast<size_t>(c0) * D, cn, cn);
    stage_rows<float, D, LD>(Gs, dO + boff + static_cast<size_t>(c0) * D, cn, cn);
    for (int t = threadIdx.x; t < 2 * cn; t += blockDim.x)
      Ss[t] = stats[(static_cast<size_t>(b) * N + c0) * 2 + t];
    __syncthreads();
    for (int ii = 0; ii < cn; ++ii) {
      const int i = c0 + ii;
      float q[E], g[E];
      ld_f32<E>(q, Qs + ii * LD + sub * E);
      ld_f32<E>(g, Gs + ii * LD + sub * E);
      const float s = quad_dot<E>(q, kr) * scale;
      const float p = i == j ? 0.f : expf(s - Ss[2 * ii]);
      const float ds = p * (quad_dot<E>(g, vr) - Ss[2 * ii + 1]);
#pragma unroll
      for (int c = 0; c < E; ++c) {
        dv[c] = fmaf(p, g[c], dv[c]);
        dk[c] = fmaf(ds, q[c], dk[c]);
      }
    }
  }
  if (!live) return;
#pragma unroll
  for (int c = 0; c < E; ++c) dk[c] *= scale;
  st_f32<E>(dK + roff, dk);
  st_f32<E>(dV + roff, dv);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

constexpr size_t kBwdLdsBudget = 65536;

template <int D>
static hipError_t launch_fixedset_bwd(const FixedsetBwdArgs& a) {
  const long rows = static_cast<long>(a.B) * a.N;
  const int grid = static_cast<int>((rows * 4 + 255) / 256);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  const size_t lds = static_cast<size_t>(2) * a.N * D * sizeof(float);
  if (lds <= kBwdLdsBudget) {  // the batch row's dK, dV fit LDS
    if (a.idx_is_i64)
      hipLaunchKernelGGL((fixedset_bwd_lds_kernel<D, int64_t>), dim3(a.B), dim3(1024), lds, st,
                         a.q, a.k, a.v, a.dout, static_cast<const int64_t*>(a.idx), a.dq, a.dk,
                         a.dv, a.N, a.kk, a.scale);
    else
      hipLaunchKernelGGL((fixedset_bwd_lds_kernel<D, int32_t>), dim3(a.B), dim3(1024), lds, st,
                         a.q, a.k, a.v, a.dout, static_cast<const int32_t*>(a.idx), a.dq, a.dk,
                         a.dv, a.N, a.kk, a.scale);
    return hipGetLastError();
  }
  if (a.idx_is_i64)
    hipLaunchKernelGGL((fixedset_bwd_kernel<D, int64_t>), dim3(grid), dim3(256), 0, st, a.q, a.k,
                       a.v, a.dout, static_cast<const int64_t*>(a.idx), a.dq, a.dk, a.dv, a.B, a.N,
                       a.kk, a.scale);
  else
    hipLaunchKernelGGL((fixedset_bwd_kernel<D, int32_t>), dim3(grid), dim3(256), 0, st, a.q, a.k,
                       a.v, a.dout, static_cast<const int32_t*>(a.idx), a.dq, a.dk, a.dv, a.B, a.N,
                       a.kk, a.scale);
  return hipGetLastError();
}

hipError_t run_fixedset_bwd(const FixedsetBwdArgs& a) {
  switch (a.d) {
    case 8: return launch_fixedset_bwd<8>(a);
    case 16: return launch_fixedset_bwd<16>(a);
    case 32: return launch_fixedset_bwd<32>(a);
    case 64: return launch_fixedset_bwd<64>(a);
  }
  return hipErrorInvalidValue;
}

template <int D>
static hipError_t launch_dense_bwd(const DenseBwdArgs& a) {
  const int per = 256 / 4;  // queries (keys) per workgroup
  const int nblk = (a.N + per - 1) / per;
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  hipLaunchKernelGGL((dense_bwd_q_kernel<D>), dim3(a.B * nblk), dim3(256), 0, st, a.q, a.k, a.v,
                     a.out, a.dout, a.dq, a.stats, a.N, nblk, a.scale);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((dense_bwd_kv_kernel<D>), dim3(a.B * nblk), dim3(256), 0, st, a.q, a.k, a.v,
                     a.dout, a.stats, a.dk, a.dv, a.N, nblk, a.scale);
  return hipGetLastError();
}

hipError_t run_dense_bwd(const DenseBwdArgs& a) {
  switch (a.d) {
    case 8: return launch_dense_bwd<8>(a);
    case 16: return launch_dense_bwd<16>(a);
    case 32: return launch_dense_bwd<32>(a);
    case 64: return launch_dense_bwd<64>(a);
  }
  return hipErrorInvalidValue;
}

}  // namespace tarmac
