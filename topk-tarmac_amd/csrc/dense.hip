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
// contiguous read. The running max is shared by the 4 lanes of a query
// (two xor shuffles per 64-key block); the running sum stays per lane and is
// combined once at the end.
#include "frag.hpp"
#include "tarmac_internal.hpp"

namespace tarmac {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kDenseBlockTiles = 4;  // 64 keys per online-softmax step

template <typename T, int D>
struct PvOperand;

// fp32: O^T block h (channels 16h..16h+15) += V^T(16 x 4 keys) * P^T(4 keys x 16 q)
template <int D>
struct PvOperand<float, D> {
  static constexpr int NH = (D + 15) / 16;  // output blocks of 16 channels
  static constexpr int CP = NH * 16;        // padded channel count in LDS
  static constexpr int LDV = 0;             // set by kernel (kc + 4)
  __device__ __forceinline__ static void pv_tile(f32x4 (&acc)[NH], const float* Vt, int ldv,
                                                 int kb, int lane, const float (&p)[4]) {
    const int col = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const f32x4 vv = *reinterpret_cast<const f32x4*>(Vt + (16 * h + col) * ldv + kb + 4 * grp);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[h] = mfma_f32_16x16x4(vv[u], p[u], acc[h]);
    }
  }
};

// bf16: O^T block h += V^T(16 x 16 keys) * P^T(16 keys x 16 q), one MFMA
template <int D>
struct PvOperand<bf16, D> {
  static constexpr int NH = D / 16;
  static constexpr int CP = NH * 16;
  __device__ __forceinline__ static void pv_tile(f32x4 (&acc)[NH], const bf16* Vt, int ldv, int kb,
                                                 int lane, const float (&p)[4]) {
    const int col = lane & 15, grp = lane >> 4;
    i16x4 pb;
#pragma unroll
    for (int u = 0; u < 4; ++u) pb[u] = static_cast<short>(f32_to_bf16(p[u]));
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const i16x4 vv = *reinterpret_cast<const i16x4*>(Vt + (16 * h + col) * ldv + kb + 4 * grp);
      acc[h] = mfma_bf16_16x16x16(vv, pb, acc[h]);
    }
  }
};

// Stage V[rows, D] transposed into Vt[c][key] (row stride ldv), zero-filling
// keys [rows, rows_pad) and channels [D, CP).
template <typename T, int D, int CP>
__device__ __forceinline__ void stage_vt(T* Vt, int ldv, const T* src, int rows, int rows_pad) {
  constexpr int VE = 16 / sizeof(T);
  constexpr int VPR = D / VE;
  const int total = rows_pad * VPR;
  for (int v = threadIdx.x; v < total; v += blockDim.x) {
    const int row = v / VPR, cv = v - row * VPR;
    T x[VE];
    if (row < rows) {
      const uint4 raw = *reinterpret_cast<const uint4*>(src + static_cast<size_t>(row) * D + cv * VE);
      __builtin_memcpy(x, &raw, 16);
    } else {
#pragma unroll
      for (int e = 0; e < VE; ++e) x[e] = T(0);
    }
#pragma unroll
    for (int e = 0; e < VE; ++e) Vt[(cv * VE + e) * ldv + row] = x[e];
  }
  if constexpr (CP > D) {
    const int pad = (CP - D) * rows_pad;
    for (int v = threadIdx.x; v < pad; v += blockDim.x) {
      const int c = D + v / rows_pad, row = v % rows_pad;
      Vt[c * ldv + row] = T(0);
    }
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(256)
dense_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
             T* __restrict__ O, int N, int n_qblk, int kc, float scale, int nblocks) {
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

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int blk = xcd_logical_block(blockIdx.x, nblocks);
  const int b = blk / n_qblk, qblk = blk - b * n_qblk;
  const int q0 = qblk * (16 * nw) + wave * 16;
  const int col = lane & 15, grp = lane >> 4;
  const int qi = q0 + col;
  const size_t boff = static_cast<size_t>(b) * N * D;

  // Scores come out pre-multiplied by scale*log2(e), ready for exp2.
  F frag;
  {
    const float pre = scale * kLog2e;
    if constexpr (sizeof(T) == 4) {
      frag.load_q(Q + boff + static_cast<size_t>(min(qi, N - 1)) * D, grp, pre);
    } else {
      frag.load_q(Q + boff + static_cast<size_t>(min(qi, N - 1)) * D, grp, 1.f);
    }
  }
  const float post = (sizeof(T) == 4) ? 1.f : scale * kLog2e;

  f32x4 acc[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) acc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  for (int c0 = 0; c0 < N; c0 += kc) {
    const int cn = min(kc, N - c0);
    const int cnp = (cn + BK - 1) / BK * BK;
    __syncthreads();
    stage_rows<T, D, LDK>(Ks, Kx + boff + static_cast<size_t>(c0) * D, cn, cnp);
    stage_vt<T, D, PV::CP>(Vt, ldv, V + boff + static_cast<size_t>(c0) * D, cn, cnp);
    __syncthreads();
    if (q0 >= N) continue;
    for (int kb0 = 0; kb0 < cnp; kb0 += BK) {
      float s[kDenseBlockTiles][4];
#pragma unroll
      for (int t = 0; t < kDenseBlockTiles; ++t) {
        const f32x4 st = frag.score(Ks + (kb0 + 16 * t + col) * LDK, grp);
#pragma unroll
        for (int r = 0; r < 4; ++r) s[t][r] = st[r] * post;
      }
      const int kabs = c0 + kb0;
      const int kend = c0 + cn;  // rows past the chunk end are zero padding
      if (kabs + BK > kend || (q0 >= kabs && q0 < kabs + BK)) {  // wave-uniform
#pragma unroll
        for (int t = 0; t < kDenseBlockTiles; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = kabs + 16 * t + 4 * grp + r;
            if (key >= kend || key == qi) s[t][r] = -INFINITY;
          }
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int t = 0; t < kDenseBlockTiles; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, s[t][r]);
      mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
      const float m_new = fmaxf(m_run, mloc);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = exp2f(m_run - m_use);  // 0 while nothing has been seen
      l_run *= alpha;
#pragma unroll
      for (int h = 0; h < NH; ++h) acc[h] *= alpha;
      m_run = m_new;
#pragma unroll
      for (int t = 0; t < kDenseBlockTiles; ++t) {
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[r] = exp2f(s[t][r] - m_use);
          l_run += p[r];
        }
        PV::pv_tile(acc, Vt, ldv, kb0 + 16 * t, lane, p);
      }
    }
  }
  if (q0 >= N) return;
  float l_tot = l_run + __shfl_xor(l_run, 16);
  l_tot += __shfl_xor(l_tot, 32);
  if (qi >= N) return;
  // lane l holds O^T[c = 16h + 4*(l/16) + r][q = l%16]
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int cbase = 16 * h + 4 * grp;
    if (cbase < D) {
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = acc[h][r] / l_tot;
      st_row<T, 4>(O + boff + static_cast<size_t>(qi) * D + cbase, o);
    }
  }
}

template <typename T, int D>
static hipError_t launch_dense(const DenseArgs& a) {
  const int nw = a.N >= 64 ? 4 : (a.N + 15) / 16;
  const int qb = 16 * nw;
  const int n_qblk = (a.N + qb - 1) / qb;
  const int nblocks = a.B * n_qblk;
  const size_t lds = dense_lds_bytes(a.dtype, a.d, a.key_chunk);
  hipLaunchKernelGGL((dense_kernel<T, D>), dim3(nblocks), dim3(64 * nw), lds,
                     static_cast<hipStream_t>(a.stream), static_cast<const T*>(a.q),
                     static_cast<const T*>(a.k), static_cast<const T*>(a.v), static_cast<T*>(a.out),
                     a.N, n_qblk, a.key_chunk, a.scale, nblocks);
  return hipGetLastError();
}

size_t dense_lds_bytes(int dtype, int d, int kc) {
  const int bk = 16 * kDenseBlockTiles;
  const int kcp = (kc + bk - 1) / bk * bk;
  const int cp = (d + 15) / 16 * 16;
  const size_t es = dtype == kF32 ? 4 : 2;
  const int ldk = dtype == kF32 ? d + 4 : d + 8;
  return (static_cast<size_t>(kcp) * ldk + static_cast<size_t>(cp) * (kcp + 4)) * es;
}

hipError_t run_dense(const DenseArgs& a) {
  if (a.dtype == kF32) {
    switch (a.d) {
      case 8: return launch_dense<float, 8>(a);
      case 16: return launch_dense<float, 16>(a);
      case 32: return launch_dense<float, 32>(a);
      case 64: return launch_dense<float, 64>(a);
    }
  } else {
    switch (a.d) {
      case 16: return launch_dense<bf16, 16>(a);
      case 32: return launch_dense<bf16, 32>(a);
      case 64: return launch_dense<bf16, 64>(a);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace tarmac
