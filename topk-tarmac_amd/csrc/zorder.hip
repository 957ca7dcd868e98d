// Select-before-scoring: attention over a peer set fixed before any score
// exists, and the Z-order (Morton-window) selector that produces such sets.
//
// Reference behaviour:
//   src/kernels/fused_prescore_attention.py:27-114  fused_prescore_attention
//   src/kernels/prescore_selection.py:62-84         _morton_code, select_morton_window
//   src/kernels/prescore_selection.py:184-195       prescore_attention
//   src/agents/mappo.py:265-292                     zorder_k (selector + attend)
//
// Fixed-set attention: a quad of lanes owns one query; lane (l % 4) holds d/4
// channels. Peers are taken in batches whose index, K and V loads are all in
// flight together; the quad forms each dot with two xor shuffles and folds the
// batch into an online softmax (one rescale per batch) and its V slice.
//
// Morton window, one workgroup per batch row:
//   1. per-axis min/max over the agents (a wavefront reduction);
//   2. fp32 quantisation exactly as torch does it: (p - lo) / span * (2^bits-1),
//      truncated, clamped; x bits to even positions, y bits to odd;
//   3. a bitonic sort of the packed words (code << 32 | agent), so equal codes
//      come out in agent order: one wavefront, keys in registers, exchanges
//      between lanes by DPP / lane swaps / ds_bpermute, no LDS stage and no
//      barrier (rows past 2048 agents: the whole workgroup, with LDS stages
//      across wavefronts);
//   4. rank[order[r]] = r, and agent i's peers are order[(rank[i] + off) mod N]
//      for off = +1..+ceil(k/2), -1..-floor(k/2).
// The fused variant then runs the fixed-set attention for the batch row from
// the peer lists in LDS, in the same launch.
#include "frag.hpp"
#include "sort.hpp"
#include "tarmac_internal.hpp"

#pragma clang fp contract(off)

namespace tarmac {

// One workgroup per batch row for the selector.
constexpr int kZorderThreads = 256;
// Longest padded row (next_pow2(N)) the selector sorts: four wavefronts with
// runs of up to 1024 keys (16 per lane).
constexpr int kZorderMaxP = 4096;
static_assert(kZorderMaxP == (kZorderThreads / 64) * 64 * 16,
              "the selector's longest row: every wavefront sorts 16 keys per lane");
// Queries per quad per pass of the fused Z-order attention (peers from
// global memory / from LDS).
template <int D>
constexpr int zorder_rows() { return D <= 32 ? 2 : 1; }
template <int D>
constexpr int zorder_lds_rows() { return D <= 16 ? 8 : (D <= 32 ? 4 : 2); }

// Key slots of the selector: whole sorting runs, at least one run of 128
// (64 lanes x 2 keys) even for rows shorter than that.
__host__ __device__ inline int zorder_key_slots(int P) { return P < 128 ? 128 : P; }

// Selector LDS: keys [zorder_key_slots(P)] (8 B), order and rank [N] (4 B
// each), min / max scratch; the LDS-staged fused kernel's K and V rows
// follow, 16-byte aligned.
__host__ __device__ inline size_t zorder_selector_bytes(int N, int P) {
  return static_cast<size_t>(zorder_key_slots(P)) * 8 + static_cast<size_t>(N) * 8 +
         4 * 4 * (kZorderThreads / 64);
}
__host__ __device__ inline size_t zorder_kv_offset(int N, int P) {
  return (zorder_selector_bytes(N, P) + 15) / 16 * 16;
}

// ---------------------------------------------------------------------------
// fixed-set attention for one query (a quad of lanes)
// ---------------------------------------------------------------------------

// QR queries per quad at once (row r: query row qrow[r], peers peer(r, j));
// live[r] false skips row r's loads and store. All index, K and V loads of
// a batch of U peers of every row are in flight together.
template <typename T, int D, int QR, typename IdxFn>
__device__ __forceinline__ void quad_fixedset_rows(const T* const (&qrow)[QR],
                                                   const T* __restrict__ Kb,
                                                   const T* __restrict__ Vb,
                                                   T* const (&orow)[QR], const bool (&live)[QR],
                                                   int N, int kk, float scale, int sub,
                                                   IdxFn peer) {
  constexpr int E = D / 4;
  // peers per batch: fewer when several rows share the registers
  constexpr int U = QR == 1 ? (E <= 4 ? 4 : (E <= 8 ? 2 : 1)) : (E <= 4 ? 2 : 1);
  float q[QR][E], acc[QR][E], m_run[QR], l_run[QR];
  bool bad[QR];
#pragma unroll
  for (int r = 0; r < QR; ++r) {
    if (live[r]) ld_row<T, E>(q[r], qrow[r] + sub * E);
    else
#pragma unroll
      for (int c = 0; c < E; ++c) q[r][c] = 0.f;
#pragma unroll
    for (int c = 0; c < E; ++c) acc[r][c] = 0.f;
    m_run[r] = -INFINITY;
    l_run[r] = 0.f;
    bad[r] = false;
  }
  for (int j0 = 0; j0 < kk; j0 += U) {
    int p[QR][U];
#pragma unroll
    for (int r = 0; r < QR; ++r)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = live[r] && j0 + u < kk;
        p[r][u] = ok ? peer(r, j0 + u) : 0;
        bad[r] |= ok && ((p[r][u] < 0) | (p[r][u] >= N));
        p[r][u] = min(max(p[r][u], 0), N - 1);
      }
    float kr[QR][U][E], vr[QR][U][E];
#pragma unroll
    for (int r = 0; r < QR; ++r)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (live[r] && j0 + u < kk) {
          ld_row<T, E>(kr[r][u], Kb + static_cast<size_t>(p[r][u]) * D + sub * E);
          ld_row<T, E>(vr[r][u], Vb + static_cast<size_t>(p[r][u]) * D + sub * E);
        } else {
#pragma unroll
          for (int c = 0; c < E; ++c) kr[r][u][c] = vr[r][u][c] = 0.f;
        }
      }
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      // scores of the batch (log2 domain), then one rescale of the running sums
      float s[U];
      float m_b = m_run[r];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float t = 0.f;
#pragma unroll
        for (int c = 0; c < E; ++c) t = fmaf(q[r][c], kr[r][u][c], t);
        t = quad_sum(t);
        s[u] = j0 + u < kk ? t * scale * kLog2eF : -INFINITY;
        m_b = fmaxf(m_b, s[u]);
      }
      const float alpha = m_run[r] == -INFINITY ? 0.f : fast_exp2(m_run[r] - m_b);
      l_run[r] *= alpha;
#pragma unroll
      for (int c = 0; c < E; ++c) acc[r][c] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float w = s[u] == -INFINITY ? 0.f : fast_exp2(s[u] - m_b);
        l_run[r] += w;
#pragma unroll
        for (int c = 0; c < E; ++c) acc[r][c] = fmaf(w, vr[r][u][c], acc[r][c]);
      }
      m_run[r] = m_b;
    }
  }
#pragma unroll
  for (int r = 0; r < QR; ++r) {
    if (!live[r]) continue;
    const float inv = 1.f / l_run[r];
    float o[E];
#pragma unroll
    for (int c = 0; c < E; ++c) o[c] = bad[r] ? __int_as_float(0x7fc00000) : acc[r][c] * inv;
    if constexpr (E % 4 == 0) {
      st_row<T, E>(orow[r] + sub * E, o);
    } else {
#pragma unroll
      for (int c = 0; c < E; ++c) {
        if constexpr (sizeof(T) == 4) orow[r][sub * E + c] = o[c];
        else orow[r][sub * E + c] = f32_to_bf16(o[c]);
      }
    }
  }
}

template <typename T, int D, typename IdxFn>
__device__ __forceinline__ void quad_fixedset_row(const T* __restrict__ qrow,
                                                  const T* __restrict__ Kb,
                                                  const T* __restrict__ Vb, T* __restrict__ orow,
                                                  int N, int kk, float scale, int sub,
                                                  IdxFn peer) {
  const T* const qr[1] = {qrow};
  T* const orr[1] = {orow};
  const bool lv[1] = {true};
  quad_fixedset_rows<T, D, 1>(qr, Kb, Vb, orr, lv, N, kk, scale, sub,
                              [&](int, int j) { return peer(j); });
}

template <typename T, int D, typename I>
__global__ void __launch_bounds__(256)
fixedset_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
                const I* __restrict__ Idx, T* __restrict__ O, int B, int N, int kk, float scale) {
  const int lane = threadIdx.x & 63;
  // consecutive logical blocks (the queries of one batch row) share an XCD,
  // so the row's K and V rows are fetched into one L2
  const int blk = xcd_logical_block(blockIdx.x, gridDim.x);
  const long row = (static_cast<long>(blk) * blockDim.x + threadIdx.x) >> 2;
  if (row >= static_cast<long>(B) * N) return;  // whole quads exit together
  const int b = static_cast<int>(row / N);
  const size_t boff = static_cast<size_t>(b) * N * D;
  const I* ir = Idx + static_cast<size_t>(row) * kk;
  quad_fixedset_row<T, D>(Q + static_cast<size_t>(row) * D, Kx + boff, V + boff,
                          O + static_cast<size_t>(row) * D, N, kk, scale, lane & 3,
                          [&](int j) { return static_cast<int>(ir[j]); });
}

// ---------------------------------------------------------------------------
// Morton window selector
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t spread_bits16(uint32_t x) {
  // Standard shift-and-mask bit spread of a 16-bit value.
  x &= 0x0000ffffu;
  x = (x | (x << 8)) & 0x00ff00ffu;
  x = (x | (x << 4)) & 0x0f0f0f0fu;
  x = (x | (x << 2)) & 0x33333333u;
  x = (x | (x << 1)) & 0x55555555u;
  return x;
}

__device__ __forceinline__ int quantise(float p, float lo, float span, float top, int topi) {
  const float t = p - lo;
  const float u = t / span;   // correctly rounded fp32 division
  const float w = u * top;
  long g = static_cast<long>(w);  // truncation toward zero, as Tensor.long()
  g = g < 0 ? 0 : (g > topi ? topi : g);
  return static_cast<int>(g);
}

struct ZorderSmem {
  uint64_t* keys;   // [P] packed (code << 32 | agent)
  int* order;       // [N]
  int* rank;        // [N]
  float* red;       // [4 * waves] min / max scratch
};

// Number of keys in the sorted run [run, run + len) (len a power of two)
// strictly below k: a branch-free lower bound, log2(len) + 1 LDS reads.
__device__ __forceinline__ int count_below(const uint64_t* run, int len, uint64_t k) {
  int pos = 0;
  for (int step = len >> 1; step > 0; step >>= 1)
    if (run[pos + step - 1] < k) pos += step;
  return pos + (run[pos] < k ? 1 : 0);
}

// Codes, sort, order and rank for batch row `pos` ([N, 2]). The P = 64 RW *
// runs padded keys are split into `runs` (1, 2 or 4) runs of 64 RW, one per
// wavefront: each wavefront loads its agents' positions once, and after a
// workgroup min / max, quantises them and sorts its run of words
// (code << 32 | agent) in registers (wave_bitonic_sort: no LDS, no barrier;
// padding ~0 sorts last). A word's rank is its position in its own run plus
// the number of smaller words in each other run (a binary search in LDS);
// words are distinct (agent in the low bits), so equal codes rank in agent
// order. `after_load` runs on every wavefront, once its positions have been
// used: memory operations issued there queue behind nothing the sort needs
// (global-to-LDS loads issued there still complete before the sort's first
// barrier: the compiler waits for them there).
template <int RW, typename AfterLoad>
__device__ void morton_order_rank(const float* __restrict__ pos, int N, int P, int bits,
                                  const ZorderSmem& sm, AfterLoad after_load) {
  constexpr int RUN = 64 * RW;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int runs = P > RUN ? P / RUN : 1;
  const bool in_run = wave < runs;  // wave-uniform
  const int a0 = wave * RUN + lane * RW;
  float2 p[RW];
  float lo0 = INFINITY, lo1 = INFINITY, hi0 = -INFINITY, hi1 = -INFINITY;
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    p[r] = make_float2(0.f, 0.f);
    if (in_run && a0 + r < N) {
      p[r] = reinterpret_cast<const float2*>(pos)[a0 + r];
      lo0 = fminf(lo0, p[r].x); hi0 = fmaxf(hi0, p[r].x);
      lo1 = fminf(lo1, p[r].y); hi1 = fmaxf(hi1, p[r].y);
    }
  }
  after_load();
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lo0 = fminf(lo0, __shfl_xor(lo0, o)); hi0 = fmaxf(hi0, __shfl_xor(hi0, o));
    lo1 = fminf(lo1, __shfl_xor(lo1, o)); hi1 = fmaxf(hi1, __shfl_xor(hi1, o));
  }
  if (lane == 0) {
    sm.red[4 * wave + 0] = lo0; sm.red[4 * wave + 1] = hi0;
    sm.red[4 * wave + 2] = lo1; sm.red[4 * wave + 3] = hi1;
  }
  __syncthreads();
  lo0 = sm.red[0]; hi0 = sm.red[1]; lo1 = sm.red[2]; hi1 = sm.red[3];
  for (int w = 1; w < runs; ++w) {
    lo0 = fminf(lo0, sm.red[4 * w + 0]); hi0 = fmaxf(hi0, sm.red[4 * w + 1]);
    lo1 = fminf(lo1, sm.red[4 * w + 2]); hi1 = fmaxf(hi1, sm.red[4 * w + 3]);
  }
  uint64_t key[RW];
  if (in_run) {
    const float span0 = fmaxf(hi0 - lo0, 1e-6f), span1 = fmaxf(hi1 - lo1, 1e-6f);
    const int topi = (1 << bits) - 1;
    const float top = static_cast<float>(topi);
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      key[r] = ~0ull;
      if (a0 + r < N) {
        const uint32_t gx = quantise(p[r].x, lo0, span0, top, topi);
        const uint32_t gy = quantise(p[r].y, lo1, span1, top, topi);
        const uint32_t code = spread_bits16(gx) | (spread_bits16(gy) << 1);
        key[r] = (static_cast<uint64_t>(code) << 32) | static_cast<uint32_t>(a0 + r);
      }
    }
    wave_bitonic_sort<uint64_t, RW>(key, lane);
#pragma unroll
    for (int r = 0; r < RW; ++r) sm.keys[wave * RUN + lane * RW + r] = key[r];
  }
  __syncthreads();
  int rk[RW];
  if (in_run) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      rk[r] = lane * RW + r;
      if (key[r] == ~0ull) continue;  // padding
      for (int w = 0; w < runs; ++w)
        if (w != wave) rk[r] += count_below(sm.keys + w * RUN, RUN, key[r]);
      const int agent = static_cast<int>(key[r] & 0xffffffffu);
      sm.order[rk[r]] = agent;
      sm.rank[agent] = rk[r];
    }
  }
  __syncthreads();  // the runs have been searched: the words go to their ranks
  if (in_run) {
#pragma unroll
    for (int r = 0; r < RW; ++r)
      if (key[r] != ~0ull) sm.keys[rk[r]] = key[r];
  }
  __syncthreads();
}

// Keys per lane of each wavefront's run for a padded row length P (runs of
// 128 keys up to P = 512, then four runs of P / 4).
inline int zorder_sort_r(int P) { return P <= 512 ? 2 : P / 256; }

__device__ __forceinline__ int window_peer(const ZorderSmem& sm, int i, int j, int k, int N) {
  const int half = (k + 1) >> 1;
  const int off = (j < half) ? (j + 1) : -(j - half + 1);
  // |off| <= ceil(k / 2) < N (k <= N - 1): one conditional wrap
  int r = sm.rank[i] + off;
  r = r >= N ? r - N : (r < 0 ? r + N : r);
  return sm.order[r];
}

__device__ __forceinline__ ZorderSmem zorder_smem(unsigned char* raw, int N, int P) {
  ZorderSmem sm;
  sm.keys = reinterpret_cast<uint64_t*>(raw);
  sm.order = reinterpret_cast<int*>(sm.keys + zorder_key_slots(P));
  sm.rank = sm.order + N;
  sm.red = reinterpret_cast<float*>(sm.rank + N);
  return sm;
}

template <typename I, int RW>
__global__ void __launch_bounds__(kZorderThreads)
morton_window_kernel(const float* __restrict__ pos, I* __restrict__ idx, int64_t* __restrict__ codes,
                     int N, int P, int k, int bits) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const ZorderSmem sm = zorder_smem(smem_raw, N, P);
  const int b = blockIdx.x;
  morton_order_rank<RW>(pos + static_cast<size_t>(b) * N * 2, N, P, bits, sm, [] {});
  if (codes != nullptr) {
    // codes in agent order: the sorted word at rank[i] carries agent i's code
    for (int i = threadIdx.x; i < N; i += blockDim.x)
      codes[static_cast<size_t>(b) * N + i] = static_cast<int64_t>(sm.keys[sm.rank[i]] >> 32);
  }
  if (idx != nullptr) {
    const int total = N * k;
    for (int t = threadIdx.x; t < total; t += blockDim.x) {
      const int i = t / k, j = t - i * k;
      idx[static_cast<size_t>(b) * total + t] = static_cast<I>(window_peer(sm, i, j, k, N));
    }
  }
}

// Asynchronous copy of `bytes` (a multiple of 16) from global memory into LDS
// with global_load_lds_dwordx4 (lane i of a wave writes 16 bytes at base +
// 16 i): wave w moves the 1 KiB pieces w, w + nw, ... The data is in LDS once
// every issuing wave's vector memory count has drained.
__device__ __forceinline__ void copy_to_lds_async(void* dst, const void* src, int bytes) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int piece = wave; piece * 1024 < bytes; piece += nw) {
    const int off = piece * 1024 + lane * 16;
    if (off < bytes)
      __builtin_amdgcn_global_load_lds(static_cast<const char*>(src) + off,
                                       static_cast<char*>(dst) + piece * 1024, 16, 0, 0);
  }
}

// Attention over the window peers with the row's K and V in LDS. A quad of
// lanes owns QR queries per pass (their query loads are all in flight
// together); each peer's score is one quad_sum, folded into an online softmax.
template <typename T, int D, int QR>
__device__ __forceinline__ void zorder_lds_attention(const T* __restrict__ Qb, const T* Ks,
                                                     const T* Vs, T* __restrict__ Ob,
                                                     const ZorderSmem& sm, int N, int k,
                                                     float scale) {
  constexpr int E = D / 4;
  const int sub = threadIdx.x & 3, quad = threadIdx.x >> 2, quads = blockDim.x >> 2;
  const float c = scale * kLog2eF;
  for (int i0 = quad; i0 < N; i0 += QR * quads) {
    float q[QR][E];
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int i = i0 + r * quads;
      if (i < N) {
        ld_row<T, E>(q[r], Qb + static_cast<size_t>(i) * D + sub * E);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) q[r][e] = 0.f;
      }
    }
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int i = i0 + r * quads;
      if (i >= N) continue;  // uniform over the quad
      float acc[E], m = -INFINITY, l = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = 0.f;
      for (int j = 0; j < k; ++j) {
        const int pj = window_peer(sm, i, j, k, N);
        float kr[E], vr[E];
        ld_row<T, E>(kr, Ks + pj * D + sub * E);
        ld_row<T, E>(vr, Vs + pj * D + sub * E);
        float t = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) t = fmaf(q[r][e], kr[e], t);
        const float sc = quad_sum(t) * c;
        const float m_new = fmaxf(m, sc);
        const float alpha = fast_exp2(m - m_new);  // 0 for the first peer
        const float w = fast_exp2(sc - m_new);
        l = l * alpha + w;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] = fmaf(w, vr[e], acc[e] * alpha);
        m = m_new;
      }
      const float inv = 1.f / l;
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = acc[e] * inv;
      if constexpr (E % 4 == 0) {
        st_row<T, E>(Ob + static_cast<size_t>(i) * D + sub * E, o);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if constexpr (sizeof(T) == 4) Ob[static_cast<size_t>(i) * D + sub * E + e] = o[e];
          else Ob[static_cast<size_t>(i) * D + sub * E + e] = f32_to_bf16(o[e]);
        }
      }
    }
  }
}

// KV_LDS: the row's K and V are copied into LDS with global-to-LDS loads
// issued as soon as the positions are in, and the attention gathers peers
// from there (LDS, unlike L2, is private to the workgroup); otherwise peers
// are gathered from global memory. The compiler drains such loads at the next
// barrier (their LDS writes must land before it), so the copy overlaps the
// position reduction, not the sort; with two workgroups per CU one row's
// copy overlaps the other's sort. Holding K and V in registers through the
// sort instead (151 VGPRs) measured slower: 33.8 -> 36.2 us at N = 512 and
// 16.7 -> 21.0 us at N = 256, where it halves the workgroups per CU.
template <typename T, int D, bool KV_LDS, int RW>
__global__ void __launch_bounds__(kZorderThreads)
zorder_attn_kernel(const T* __restrict__ Q, const T* __restrict__ Kx, const T* __restrict__ V,
                   const float* __restrict__ pos, T* __restrict__ O, int32_t* __restrict__ idx_out,
                   int N, int P, int k, int bits, float scale) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const ZorderSmem sm = zorder_smem(smem_raw, N, P);
  const int b = blockIdx.x;
  const size_t boff = static_cast<size_t>(b) * N * D;
  const int lane = threadIdx.x & 63;
  if constexpr (KV_LDS) {
    T* Ks = reinterpret_cast<T*>(smem_raw + zorder_kv_offset(N, P));
    T* Vs = Ks + static_cast<size_t>(N) * D;
    const int rbytes = N * D * static_cast<int>(sizeof(T));
    morton_order_rank<RW>(pos + static_cast<size_t>(b) * N * 2, N, P, bits, sm, [&] {
      copy_to_lds_async(Ks, Kx + boff, rbytes);
      copy_to_lds_async(Vs, V + boff, rbytes);
    });
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies have landed
    __syncthreads();
    zorder_lds_attention<T, D, zorder_lds_rows<D>()>(Q + boff, Ks, Vs, O + boff, sm, N, k, scale);
  } else {
    morton_order_rank<RW>(pos + static_cast<size_t>(b) * N * 2, N, P, bits, sm, [] {});
    const int quads = blockDim.x >> 2;
    // several queries per quad per pass: their peer loads overlap
    constexpr int QR = zorder_rows<D>();
    for (int i0 = threadIdx.x >> 2; i0 < N; i0 += QR * quads) {
      const T* qr[QR];
      T* orr[QR];
      bool lv[QR];
#pragma unroll
      for (int r = 0; r < QR; ++r) {
        const int i = i0 + r * quads;
        lv[r] = i < N;
        const int ic = lv[r] ? i : 0;
        qr[r] = Q + boff + static_cast<size_t>(ic) * D;
        orr[r] = O + boff + static_cast<size_t>(ic) * D;
      }
      quad_fixedset_rows<T, D, QR>(qr, Kx + boff, V + boff, orr, lv, N, k, scale, lane & 3,
                                   [&](int r, int j) { return window_peer(sm, i0 + r * quads, j, k, N); });
    }
  }
  if (idx_out != nullptr) {
    const int total = N * k;
    for (int t = threadIdx.x; t < total; t += blockDim.x) {
      const int i = t / k, j = t - i * k;
      idx_out[static_cast<size_t>(b) * total + t] = window_peer(sm, i, j, k, N);
    }
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

size_t zorder_lds_bytes(int N) { return zorder_selector_bytes(N, next_pow2(N)); }

// Two such workgroups per CU (160 KiB of LDS) keep the sort of one row
// overlapping the attention of another.
constexpr size_t kZorderKvLds = 80 * 1024;

template <typename T, int D>
static hipError_t launch_fixedset(const FixedsetArgs& a) {
  const long rows = static_cast<long>(a.B) * a.N;
  const int grid = static_cast<int>((rows * 4 + 255) / 256);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  if (a.idx_is_i64) {
    hipLaunchKernelGGL((fixedset_kernel<T, D, int64_t>), dim3(grid), dim3(256), 0, st,
                       static_cast<const T*>(a.q), static_cast<const T*>(a.k),
                       static_cast<const T*>(a.v), static_cast<const int64_t*>(a.idx),
                       static_cast<T*>(a.out), a.B, a.N, a.kk, a.scale);
  } else {
    hipLaunchKernelGGL((fixedset_kernel<T, D, int32_t>), dim3(grid), dim3(256), 0, st,
                       static_cast<const T*>(a.q), static_cast<const T*>(a.k),
                       static_cast<const T*>(a.v), static_cast<const int32_t*>(a.idx),
                       static_cast<T*>(a.out), a.B, a.N, a.kk, a.scale);
  }
  return hipGetLastError();
}

hipError_t run_fixedset(const FixedsetArgs& a) {
  if (a.dtype == kF32) {
    switch (a.d) {
      case 8: return launch_fixedset<float, 8>(a);
      case 16: return launch_fixedset<float, 16>(a);
      case 32: return launch_fixedset<float, 32>(a);
      case 64: return launch_fixedset<float, 64>(a);
      case 128: return launch_fixedset<float, 128>(a);
    }
  } else {
    switch (a.d) {
      case 16: return launch_fixedset<bf16, 16>(a);
      case 32: return launch_fixedset<bf16, 32>(a);
      case 64: return launch_fixedset<bf16, 64>(a);
      case 128: return launch_fixedset<bf16, 128>(a);
    }
  }
  return hipErrorInvalidValue;
}

template <typename I, int RW>
static void launch_morton_sr(const MortonArgs& a, int P, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((morton_window_kernel<I, RW>), dim3(a.B), dim3(kZorderThreads), lds, st,
                     a.pos, static_cast<I*>(a.idx), a.codes, a.N, P, a.k, a.bits);
}

template <typename I>
static hipError_t launch_morton(const MortonArgs& a) {
  const int P = next_pow2(a.N);
  const size_t lds = zorder_lds_bytes(a.N);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  switch (zorder_sort_r(P)) {
    case 2: launch_morton_sr<I, 2>(a, P, lds, st); break;
    case 4: launch_morton_sr<I, 4>(a, P, lds, st); break;
    case 8: launch_morton_sr<I, 8>(a, P, lds, st); break;
    case 16: launch_morton_sr<I, 16>(a, P, lds, st); break;
    default: return hipErrorInvalidValue;  // P > kZorderMaxP
  }
  return hipGetLastError();
}

hipError_t run_morton_window(const MortonArgs& a) {
  return a.idx_is_i64 ? launch_morton<int64_t>(a) : launch_morton<int32_t>(a);
}

template <typename T, int D, int RW>
static void launch_zorder_sr(const ZorderArgs& a, int P) {
  const size_t kv = zorder_kv_offset(a.N, P) + 2 * static_cast<size_t>(a.N) * D * sizeof(T);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  if (kv <= kZorderKvLds) {
    hipLaunchKernelGGL((zorder_attn_kernel<T, D, true, RW>), dim3(a.B), dim3(kZorderThreads), kv,
                       st, static_cast<const T*>(a.q), static_cast<const T*>(a.k),
                       static_cast<const T*>(a.v), a.pos, static_cast<T*>(a.out), a.idx, a.N, P,
                       a.topk, a.bits, a.scale);
  } else {
    hipLaunchKernelGGL((zorder_attn_kernel<T, D, false, RW>), dim3(a.B), dim3(kZorderThreads),
                       zorder_lds_bytes(a.N), st, static_cast<const T*>(a.q),
                       static_cast<const T*>(a.k), static_cast<const T*>(a.v), a.pos,
                       static_cast<T*>(a.out), a.idx, a.N, P, a.topk, a.bits, a.scale);
  }
}

template <typename T, int D>
static hipError_t launch_zorder(const ZorderArgs& a) {
  const int P = next_pow2(a.N);
  switch (zorder_sort_r(P)) {
    case 2: launch_zorder_sr<T, D, 2>(a, P); break;
    case 4: launch_zorder_sr<T, D, 4>(a, P); break;
    case 8: launch_zorder_sr<T, D, 8>(a, P); break;
    case 16: launch_zorder_sr<T, D, 16>(a, P); break;
    default: return hipErrorInvalidValue;  // P > kZorderMaxP
  }
  return hipGetLastError();
}

hipError_t run_zorder(const ZorderArgs& a) {
  if (a.dtype == kF32) {
    switch (a.d) {
      case 8: return launch_zorder<float, 8>(a);
      case 16: return launch_zorder<float, 16>(a);
      case 32: return launch_zorder<float, 32>(a);
      case 64: return launch_zorder<float, 64>(a);
      case 128: return launch_zorder<float, 128>(a);
    }
  } else {
    switch (a.d) {
      case 16: return launch_zorder<bf16, 16>(a);
      case 32: return launch_zorder<bf16, 32>(a);
      case 64: return launch_zorder<bf16, 64>(a);
      case 128: return launch_zorder<bf16, 128>(a);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace tarmac
