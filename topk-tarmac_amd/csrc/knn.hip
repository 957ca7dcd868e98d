// k-nearest-neighbour pre-score selectors: positions -> retained peer sets,
// before any attention score exists.
//
// Reference behaviour:
//   src/kernels/prescore_selection.py:35-42    select_radius_knn (all pairs)
//   src/kernels/prescore_selection.py:87-101   grid_knn_shape
//   src/kernels/prescore_selection.py:107-164  select_grid_knn (3x3 grid cells)
//
// Distances are squared, in fp32: dx = xc - xq, dy = yc - yq, dx*dx + dy*dy,
// every operation rounded (no contraction), as torch evaluates
// (pc - pos).square().sum(-1). Squares are non-negative, so the bit pattern of
// a distance orders like its value as an unsigned integer.
//
// Selection is packed-key filter-and-verify. A candidate's key is the
// distance's bits with the low `cbits` bits replaced by its candidate number c
// (agent index for the radius selector, slot number for the grid), so one
// unsigned min / med3 per list entry keeps a sorted list of the smallest keys
// with no index bookkeeping. With the k+1 smallest keys Q[0..k] in hand: if
// the truncated distance of Q[k] is strictly above that of Q[k-1], every
// other candidate's true distance is at least trunc(Q[k]) > trunc(Q[k-1]) +
// (2^cbits - 1), which bounds the true distances of Q[0..k-1], so Q[0..k-1] is
// exactly the set of the k smallest (distance, c). Queries where the check
// fails (two of the nearest distances agree in their high bits, distances at
// +inf, fewer than k candidates) are redone by the exact wave-cooperative
// selection below, which follows the reference's rule: the k smallest by
// (distance, c), the self pair and missing slots at +inf.
//
// Radius: workgroup = 64 queries of one batch row, row positions in LDS; four
// lanes per query (lane l: query l % 16 of its wave, candidates
// j = 8u + 2(l/16) + {0,1}); the four lane lists merge with two xor shuffles.
// Grid: workgroup per batch row; cell ids, a bitonic sort of (cell, agent)
// words (equal cells in agent order; keys in registers, LDS only across
// wavefronts), cell starts, then one lane per query scans the three column
// runs of its 3x3 block.
//
// Output order within a row: the reference's topk(sorted=False) leaves it
// open; here the radius selector emits ascending agent index and the grid
// selector ascending slot (the order of the sorted cell runs).
#include <cmath>

#include "common.hpp"
#include "sort.hpp"
#include "tarmac_internal.hpp"

#pragma clang fp contract(off)

namespace tarmac {

constexpr uint32_t kInfBits = 0x7f800000u;
constexpr uint32_t kNoKey = 0xffffffffu;

__device__ __forceinline__ float pair_d2(float px, float py, float cx, float cy) {
  const float dx = cx - px;
  const float dy = cy - py;
  return dx * dx + dy * dy;
}

__device__ __forceinline__ uint32_t umed3(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm volatile("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Insert x into the ascending list l[0..n).
template <int n>
__device__ __forceinline__ void key_insert(uint32_t (&l)[n], uint32_t x) {
#pragma unroll
  for (int t = n - 1; t > 0; --t) l[t] = umed3(l[t - 1], l[t], x);
  l[0] = min(l[0], x);
}

__device__ __forceinline__ int lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

// Exact selection by one wavefront: the k smallest (key(c), c) over
// c = 0..nc-1, written as agent(c) in ascending c to out[0..k). Bisection on
// the 32-bit key finds the k-th smallest key t, starting from [lo, hi] (the
// bucket the filter pass narrowed it to; widened to the full range if the
// bounds do not hold); keys below t are taken, and keys equal to t in
// ascending c until k are taken. Counts are ballot popcounts. All lanes must
// call it with the same arguments.
template <typename Cand>
__device__ __forceinline__ int wave_count_le(const Cand& cand, int nc, uint32_t t) {
  const int lane = threadIdx.x & 63;
  int c = 0;
  for (int b = 0; b < nc; b += 64) {
    const int cc = b + lane;
    c += __popcll(__ballot(cc < nc && cand.key(cc) <= t));
  }
  return c;
}

template <typename Cand, typename I>
__device__ __forceinline__ void wave_select_exact(const Cand cand, int nc, int k, uint32_t lo,
                                                  uint32_t hi, I* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  if (wave_count_le(cand, nc, hi) < k) hi = 0xffffffffu;
  if (lo > 0u && wave_count_le(cand, nc, lo - 1u) >= k) lo = 0u;
  if (lo > hi) lo = hi;
  while (lo < hi) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    const int c = wave_count_le(cand, nc, mid);
    if (c >= k) {
      hi = mid;
      if (c == k) break;  // the keys <= mid are exactly k: t = mid
    } else {
      lo = mid + 1u;
    }
  }
  const uint32_t t = hi;
  const int ties = k - (t == 0u ? 0 : wave_count_le(cand, nc, t - 1u));
  int taken_ties = 0, written = 0;
  for (int b = 0; b < nc && written < k; b += 64) {
    const int cc = b + lane;
    const uint32_t key = cc < nc ? cand.key(cc) : kNoKey;
    const bool eq = cc < nc && key == t;
    const uint64_t meq = __ballot(eq);
    const bool sel = (cc < nc && key < t) || (eq && taken_ties + lanes_below(meq) < ties);
    const uint64_t msel = __ballot(sel);
    if (sel) out[written + lanes_below(msel)] = static_cast<I>(cand.agent(cc));
    taken_ties += __popcll(meq);
    written += __popcll(msel);
  }
}

// Bisection bounds for the exact pass from the filter list: with Q[0..k) the
// k smallest packed keys, the k-th smallest true distance lies in
// [trunc(Q[k-1]), trunc(Q[k-1]) + 2^cbits - 1]. A short list (fewer than k
// candidates) puts it at +inf (all finite candidates and the first +inf
// slots are taken).
__device__ __forceinline__ void exact_bounds(uint32_t qk1, uint32_t cmask, uint32_t& lo,
                                             uint32_t& hi) {
  if (qk1 == kNoKey) {
    lo = hi = kInfBits;
  } else if ((qk1 & ~cmask) < (kInfBits & ~cmask)) {
    lo = qk1 & ~cmask;
    hi = qk1 | cmask;
  } else {
    lo = 0u;
    hi = 0xffffffffu;
  }
}

// Ascending sort of c[0..n) (odd-even transposition).
template <int n>
__device__ __forceinline__ void sort_u32(uint32_t (&c)[n]) {
#pragma unroll
  for (int r = 0; r < n; ++r) {
#pragma unroll
    for (int t = r & 1; t + 1 < n; t += 2) {
      const uint32_t a = c[t], b = c[t + 1];
      c[t] = min(a, b);
      c[t + 1] = max(a, b);
    }
  }
}

// l[t] for a runtime t, as an or of masked entries (a select chain here is
// turned into an indexed scratch array by the compiler).
template <int n>
__device__ __forceinline__ uint32_t pick(const uint32_t (&l)[n], int t) {
  uint32_t r = 0u;
#pragma unroll
  for (int s = 0; s < n; ++s) r |= l[s] & (0u - static_cast<uint32_t>(t == s));
  return r;
}

// k+1 smallest keys Q[0..K] -> verified? and, if so, the k selected candidate
// numbers in ascending order in c[0..k).
template <int K>
__device__ __forceinline__ bool verify_and_order(const uint32_t (&Q)[K + 1], int k, uint32_t hmask,
                                                 uint32_t (&c)[K]) {
  const uint32_t a = pick(Q, k - 1) & hmask, b = pick(Q, k) & hmask;
  const bool ok = a < (kInfBits & hmask) && b > a;
#pragma unroll
  for (int t = 0; t < K; ++t) c[t] = (t < k) ? (Q[t] & ~hmask) : kNoKey;
  sort_u32(c);
  return ok;
}

// ---------------------------------------------------------------------------
// radius (all pairs)
// ---------------------------------------------------------------------------

struct RadiusCand {
  const float2* P;
  float px, py;
  int i;
  __device__ uint32_t key(int c) const {
    if (c == i) return kInfBits;  // the reference's +inf diagonal
    const float2 p = P[c];
    return __float_as_uint(pair_d2(px, py, p.x, p.y));
  }
  __device__ int agent(int c) const { return c; }
};

constexpr int kKnnRadiusThreads = 256;  // 64 queries: 4 waves x 16

// K = 0: every query takes the exact wave selection (k above the list sizes).
template <int K, typename I>
__global__ void __launch_bounds__(kKnnRadiusThreads)
knn_radius_kernel(const float* __restrict__ pos, I* __restrict__ idx, int N, int n_qblk, int k,
                  int cbits) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  float2* P = reinterpret_cast<float2*>(smem_raw);
  const int blk = xcd_logical_block(blockIdx.x, gridDim.x);  // a batch row's blocks share an XCD
  const int b = blk / n_qblk, qb = blk - b * n_qblk;
  const float2* prow = reinterpret_cast<const float2*>(pos) + static_cast<size_t>(b) * N;
  const int N8 = (N + 7) & ~7;
  for (int j = threadIdx.x; j < N8; j += blockDim.x)
    P[j] = j < N ? prow[j] : make_float2(INFINITY, INFINITY);
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s = lane >> 4;
  const int q0 = qb * 64 + wave * 16;
  const int i = q0 + (lane & 15);
  const bool live = i < N;
  const float2 me = P[live ? i : 0];
  I* const out_row = idx + (static_cast<size_t>(b) * N + i) * k;
  const uint32_t cmask = (1u << cbits) - 1u, hmask = ~cmask;

  uint64_t fail = 0;
  uint32_t qk1 = kNoKey;  // Q[k-1]: bounds for the exact pass
  if constexpr (K > 0) {
    uint32_t l[K + 2];
#pragma unroll
    for (int t = 0; t < K + 2; ++t) l[t] = kNoKey;
    const float4* P4 = reinterpret_cast<const float4*>(P);
    const int nu = N8 / 8;
    uint32_t j = 2 * s;
    int u = 0;
    for (; u + 1 < nu; u += 2, j += 16) {  // two LDS reads in flight
      const float4 c0 = P4[4 * u + s];
      const float4 c1 = P4[4 * u + 4 + s];
      key_insert(l, (__float_as_uint(pair_d2(me.x, me.y, c0.x, c0.y)) & hmask) | j);
      key_insert(l, (__float_as_uint(pair_d2(me.x, me.y, c0.z, c0.w)) & hmask) | (j + 1));
      key_insert(l, (__float_as_uint(pair_d2(me.x, me.y, c1.x, c1.y)) & hmask) | (j + 8));
      key_insert(l, (__float_as_uint(pair_d2(me.x, me.y, c1.z, c1.w)) & hmask) | (j + 9));
    }
    if (u < nu) {
      const float4 c = P4[4 * u + s];
      key_insert(l, (__float_as_uint(pair_d2(me.x, me.y, c.x, c.y)) & hmask) | j);
      key_insert(l, (__float_as_uint(pair_d2(me.x, me.y, c.z, c.w)) & hmask) | (j + 1));
    }
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
      uint32_t o[K + 2];
#pragma unroll
      for (int t = 0; t < K + 2; ++t) o[t] = __shfl_xor(l[t], sh);
#pragma unroll
      for (int t = 0; t < K + 2; ++t) key_insert(l, o[t]);
    }
    // drop the self pair (candidate number i) if it is in the list
    uint32_t Q[K + 1];
    bool f = false;
#pragma unroll
    for (int t = 0; t < K + 1; ++t) {
      f = f || ((l[t] & cmask) == static_cast<uint32_t>(i) && l[t] != kNoKey);
      Q[t] = f ? l[t + 1] : l[t];
    }
    uint32_t c[K];
    const bool ok = verify_and_order<K>(Q, k, hmask, c);
    if (live && ok) {
#pragma unroll
      for (int t = 0; t < K; ++t)
        if (t < k && (t & 3) == s) out_row[t] = static_cast<I>(c[t]);
    }
    qk1 = pick(Q, k - 1);
    fail = __ballot(live && !ok && s == 0);
  } else {
    fail = __ballot(live && s == 0);
  }
  while (fail) {
    const int f = __builtin_ctzll(fail);
    fail &= fail - 1;
    const int qi = q0 + f;
    const float2 p = P[qi];
    const RadiusCand cand{P, p.x, p.y, qi};
    uint32_t lo = 0u, hi = 0xffffffffu;
    if constexpr (K > 0) exact_bounds(__builtin_amdgcn_readlane(qk1, f), cmask, lo, hi);
    wave_select_exact(cand, N, k, lo, hi, idx + (static_cast<size_t>(b) * N + qi) * k);
  }
}

// ---------------------------------------------------------------------------
// grid (3x3 cells)
// ---------------------------------------------------------------------------

__device__ __forceinline__ int grid_coord(float p, float lo, float span, float g, int gmax) {
  const float t = p - lo;
  const float u = t / span;   // correctly rounded fp32 division
  const float w = u * g;
  long c = static_cast<long>(w);  // truncation toward zero, as Tensor.long()
  c = c < 0 ? 0 : (c > gmax ? gmax : c);
  return static_cast<int>(c);
}

// A query's three column runs: slots col*L + l, l < L. Accessors for a
// runtime column use masked ors (see pick).
struct GridRuns {
  int s_lo[3], s_hi[3];
  bool ok[3];
  __device__ static int sel3(const int (&v)[3], int col) {
    int r = 0;
#pragma unroll
    for (int s = 0; s < 3; ++s) r |= v[s] & -static_cast<int>(col == s);
    return r;
  }
  __device__ int lo(int col) const { return sel3(s_lo, col); }
  __device__ int hi(int col) const { return sel3(s_hi, col); }
  __device__ bool okc(int col) const {
    return ((ok[0] && col == 0) || (ok[1] && col == 1) || (ok[2] && col == 2));
  }
};

__device__ __forceinline__ GridRuns grid_runs(const int* __restrict__ start, int cx, int cy, int G,
                                              int L) {
  GridRuns r;
#pragma unroll
  for (int col = 0; col < 3; ++col) {
    const int x = cx + col - 1;
    r.ok[col] = x >= 0 && x < G;
    const int xc = x < 0 ? 0 : (x > G - 1 ? G - 1 : x);
    const int c_lo = xc * G + (cy - 1 > 0 ? cy - 1 : 0);
    const int c_hi = xc * G + (cy + 1 < G - 1 ? cy + 1 : G - 1) + 1;
    r.s_lo[col] = start[c_lo];
    r.s_hi[col] = min(start[c_hi], r.s_lo[col] + L);
  }
  return r;
}

struct GridCand {
  const float2* P;
  const int* order;
  GridRuns runs;
  float px, py;
  int i, L, N;
  __device__ int sorted_pos(int c) const {
    const int col = c / L;
    return min(runs.lo(col) + (c - col * L), N - 1);
  }
  __device__ uint32_t key(int c) const {
    const int col = c / L;
    const int r = runs.lo(col) + (c - col * L);
    const int a = order[min(r, N - 1)];
    if (!runs.okc(col) || r >= runs.hi(col) || a == i) return kInfBits;
    const float2 p = P[a];
    return __float_as_uint(pair_d2(px, py, p.x, p.y));
  }
  __device__ int agent(int c) const { return order[sorted_pos(c)]; }
};

struct GridSmem {
  float2* P;       // [N]
  uint32_t* keys;  // [Pn]: (cell << 16 | agent), then agents in cell order
  int* start;      // [G*G + 1]
  float* red;      // [4 * nwaves]
};

__device__ __forceinline__ GridSmem grid_smem(unsigned char* raw, int N, int Pn, int C) {
  GridSmem sm;
  sm.P = reinterpret_cast<float2*>(raw);
  sm.keys = reinterpret_cast<uint32_t*>(sm.P + N);
  sm.start = reinterpret_cast<int*>(sm.keys + Pn);
  sm.red = reinterpret_cast<float*>(sm.start + C + 1);
  return sm;
}

size_t knn_grid_lds_bytes(int N, int G, int threads) {
  const size_t Pn = static_cast<size_t>(next_pow2(N));
  return static_cast<size_t>(N) * 8 + Pn * 4 + static_cast<size_t>(G * G + 1) * 4 +
         16 * static_cast<size_t>(threads / 64);
}

struct GridQuant {
  float lo0, lo1, span0, span1, g;
  int G;
};

template <int R>
__device__ void grid_sort(const GridSmem& sm, int N, int Pn, const GridQuant& gq) {
  const int t = threadIdx.x;
  const bool active = t * R < Pn;
  uint32_t key[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int a = t * R + r;
    key[r] = kNoKey;
    if (active && a < N) {
      const float2 p = sm.P[a];
      const int cx = grid_coord(p.x, gq.lo0, gq.span0, gq.g, gq.G - 1);
      const int cy = grid_coord(p.y, gq.lo1, gq.span1, gq.g, gq.G - 1);
      key[r] = (static_cast<uint32_t>(cx * gq.G + cy) << 16) | static_cast<uint32_t>(a);
    }
  }
  block_bitonic_sort<uint32_t, R>(key, sm.keys, Pn, t, active);
  __syncthreads();  // the last LDS stage's reads are done before the keys land
  if (active) {
#pragma unroll
    for (int r = 0; r < R; ++r) sm.keys[t * R + r] = key[r];
  }
}

template <int K, typename I>
__global__ void __launch_bounds__(1024)
knn_grid_kernel(const float* __restrict__ pos, I* __restrict__ idx, int N, int Pn, int k, int G,
                int L, int cbits) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int C = G * G;
  const GridSmem sm = grid_smem(smem_raw, N, Pn, C);
  const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
  const int b = blockIdx.x;
  const float2* prow = reinterpret_cast<const float2*>(pos) + static_cast<size_t>(b) * N;

  // 1. positions and per-axis extent
  float lo0 = INFINITY, lo1 = INFINITY, hi0 = -INFINITY, hi1 = -INFINITY;
  for (int i = tid; i < N; i += nt) {
    const float2 p = prow[i];
    sm.P[i] = p;
    lo0 = fminf(lo0, p.x); hi0 = fmaxf(hi0, p.x);
    lo1 = fminf(lo1, p.y); hi1 = fmaxf(hi1, p.y);
  }
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
  for (int w = 1; w < nw; ++w) {
    lo0 = fminf(lo0, sm.red[4 * w + 0]); hi0 = fmaxf(hi0, sm.red[4 * w + 1]);
    lo1 = fminf(lo1, sm.red[4 * w + 2]); hi1 = fmaxf(hi1, sm.red[4 * w + 3]);
  }
  const float span0 = fmaxf(hi0 - lo0, 1e-6f), span1 = fmaxf(hi1 - lo1, 1e-6f);
  const float g = static_cast<float>(G);

  // 2. cell keys (cell << 16 | agent), sorted in registers / across lanes,
  //    through LDS only across wavefronts; padding sorts last
  {
    const int R = Pn / nt < 2 ? 2 : Pn / nt;
    const GridQuant gq{lo0, lo1, span0, span1, g, G};
    switch (R) {
      case 2: grid_sort<2>(sm, N, Pn, gq); break;
      case 4: grid_sort<4>(sm, N, Pn, gq); break;
      case 8: grid_sort<8>(sm, N, Pn, gq); break;
      default: grid_sort<16>(sm, N, Pn, gq); break;
    }
  }
  __syncthreads();
  // 3. start[c] = first sorted position whose cell is >= c
  for (int r = tid; r <= N; r += nt) {
    const int prev = r == 0 ? -1 : static_cast<int>(sm.keys[r - 1] >> 16);
    const int cur = r == N ? C : static_cast<int>(sm.keys[r] >> 16);
    for (int c = prev + 1; c <= cur; ++c) sm.start[c] = r;
  }
  __syncthreads();
  for (int r = tid; r < N; r += nt) sm.keys[r] &= 0xffffu;
  __syncthreads();
  const int* order = reinterpret_cast<const int*>(sm.keys);

  // 4. per query: scan the three column runs
  const uint32_t cmask = (1u << cbits) - 1u, hmask = ~cmask;
  for (int base = 0; base < N; base += nt) {
    const int i = base + tid;
    const bool live = i < N;
    const int ii = live ? i : 0;
    const float2 me = sm.P[ii];
    const int cx = grid_coord(me.x, lo0, span0, g, G - 1);
    const int cy = grid_coord(me.y, lo1, span1, g, G - 1);
    uint64_t fail;
    uint32_t qk1 = kNoKey;
    if constexpr (K > 0) {
      const GridRuns runs = grid_runs(sm.start, cx, cy, G, L);
      uint32_t Q[K + 1];
#pragma unroll
      for (int t = 0; t < K + 1; ++t) Q[t] = kNoKey;
#pragma unroll
      for (int col = 0; col < 3; ++col) {
        const int r0 = runs.s_lo[col];
        const int len = runs.ok[col] ? runs.s_hi[col] - r0 : 0;
        for (int l = 0; l < len; ++l) {
          const int a = order[r0 + l];
          const float2 p = sm.P[a];
          const uint32_t key = (__float_as_uint(pair_d2(me.x, me.y, p.x, p.y)) & hmask) |
                               static_cast<uint32_t>(col * L + l);
          key_insert(Q, a == ii ? kNoKey : key);
        }
      }
      uint32_t c[K];
      const bool ok = verify_and_order<K>(Q, k, hmask, c);
      if (live && ok) {
        I* out_row = idx + (static_cast<size_t>(b) * N + i) * k;
#pragma unroll
        for (int t = 0; t < K; ++t) {
          if (t < k) {
            const int col = static_cast<int>(c[t]) / L;
            out_row[t] = static_cast<I>(order[runs.lo(col) + static_cast<int>(c[t]) - col * L]);
          }
        }
      }
      qk1 = pick(Q, k - 1);
      fail = __ballot(live && !ok);
    } else {
      fail = __ballot(live);
    }
    while (fail) {
      const int f = __builtin_ctzll(fail);
      fail &= fail - 1;
      const int qi = base + wave * 64 + f;
      const float2 p = sm.P[qi];
      const int qx = grid_coord(p.x, lo0, span0, g, G - 1);
      const int qy = grid_coord(p.y, lo1, span1, g, G - 1);
      const GridCand cand{sm.P, order, grid_runs(sm.start, qx, qy, G, L), p.x, p.y, qi, L, N};
      uint32_t lo = 0u, hi = 0xffffffffu;
      if constexpr (K > 0) exact_bounds(__builtin_amdgcn_readlane(qk1, f), cmask, lo, hi);
      wave_select_exact(cand, 3 * L, k, lo, hi, idx + (static_cast<size_t>(b) * N + qi) * k);
    }
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

static int ceil_log2(int x) {
  int b = 0;
  while ((1 << b) < x) ++b;
  return b;
}

size_t knn_radius_lds_bytes(int N) { return static_cast<size_t>((N + 7) & ~7) * 8; }

template <typename I>
static hipError_t launch_radius(const KnnArgs& a, hipStream_t st) {
  const int n_qblk = (a.N + 63) / 64;
  const int N8 = (a.N + 7) & ~7;
  const int cbits = ceil_log2(N8);
  const dim3 grid(a.B * n_qblk), block(kKnnRadiusThreads);
  const size_t lds = knn_radius_lds_bytes(a.N);
  I* idx = static_cast<I*>(a.idx);
#define TARMAC_RADIUS(KK)                                                                 \
  hipLaunchKernelGGL((knn_radius_kernel<KK, I>), grid, block, lds, st, a.pos, idx, a.N, \
                     n_qblk, a.k, cbits)
  if (a.k <= 1) TARMAC_RADIUS(1);
  else if (a.k <= 2) TARMAC_RADIUS(2);
  else if (a.k <= 4) TARMAC_RADIUS(4);
  else if (a.k <= 8) TARMAC_RADIUS(8);
  else if (a.k <= 16) TARMAC_RADIUS(16);
  else TARMAC_RADIUS(0);
#undef TARMAC_RADIUS
  return hipGetLastError();
}

template <typename I>
static hipError_t launch_grid(const KnnArgs& a, hipStream_t st) {
  const int threads = knn_grid_threads(a.N);
  const int cbits = ceil_log2(3 * a.L);
  const size_t lds = knn_grid_lds_bytes(a.N, a.G, threads);
  I* idx = static_cast<I*>(a.idx);
#define TARMAC_GRID(KK)                                                                   \
  hipLaunchKernelGGL((knn_grid_kernel<KK, I>), dim3(a.B), dim3(threads), lds, st, a.pos, idx, \
                     a.N, next_pow2(a.N), a.k, a.G, a.L, cbits)
  if (a.k <= 1) TARMAC_GRID(1);
  else if (a.k <= 2) TARMAC_GRID(2);
  else if (a.k <= 4) TARMAC_GRID(4);
  else if (a.k <= 8) TARMAC_GRID(8);
  else if (a.k <= 16) TARMAC_GRID(16);
  else TARMAC_GRID(0);
#undef TARMAC_GRID
  return hipGetLastError();
}

// grid_knn_shape (src/kernels/prescore_selection.py:87-101), in the same
// double arithmetic: about max(2, k) agents per cell, capacity
// mean + 3 sqrt(mean) + 2.
void grid_knn_shape(int N, int k, int* G, int* M) {
  const int occ = k > 2 ? k : 2;
  int g = static_cast<int>(std::sqrt(static_cast<double>(N) / occ));
  if (g < 1) g = 1;
  const double mean = static_cast<double>(N) / (static_cast<double>(g) * g);
  *G = g;
  *M = static_cast<int>(mean + 3 * std::sqrt(mean) + 2);
}

int knn_grid_threads(int N) {
  const int t = (N + 63) / 64 * 64;
  return t < 256 ? 256 : (t > 1024 ? 1024 : t);
}

hipError_t run_knn(const KnnArgs& a) {
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  if (a.grid) return a.idx_is_i64 ? launch_grid<int64_t>(a, st) : launch_grid<int32_t>(a, st);
  return a.idx_is_i64 ? launch_radius<int64_t>(a, st) : launch_radius<int32_t>(a, st);
}

}  // namespace tarmac
