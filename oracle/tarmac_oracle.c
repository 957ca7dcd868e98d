/* Canonical-order CPU oracle for the TarMAC attention core.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never linked into
 * the product. Built with -ffp-contract=off so every rounding step is explicit.
 *
 * The fp32 score of query i against key j is defined as
 *
 *     dot  = fmaf chain over c in "slot order", starting from +0.0f
 *     s_ij = dot * fp32(1/sqrt(d))            (s_ii = -inf)
 *
 * where slot order visits c = kk*(d/4) + t for t = 0..d/4-1 (outer) and
 * kk = 0..3 (inner). That is the order in which a chain of
 * v_mfma_f32_16x16x4_f32 instructions accumulates when contraction slot kk of
 * instruction t carries element kk*(d/4)+t; each MFMA rounds like a sequential
 * fmaf chain over its four slots (measured on gfx950). When 1/sqrt(d) is a
 * power of two the kernels fold it into q beforehand, which gives the same bits.
 *
 * Selection: the topk largest s_ij, ties to the lower j (float comparison,
 * so -0 == +0). Reference: src/kernels/streaming_topk_attention.py:37-44 (tie
 * rule), src/kernels/fused_topk_attention.py:211-289 (scaled score, masked
 * diagonal, argmax rounds that keep the lower index).
 *
 * Morton codes: src/kernels/prescore_selection.py:62-84 in fp32 arithmetic,
 * equal codes ordered by agent index.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float inv_sqrt_d(int d) { return (float)(1.0 / sqrt((double)d)); }

static float canon_dot(const float* q, const float* k, int d) {
  float acc = 0.0f;
  int t4 = d / 4;
  for (int t = 0; t < t4; ++t)
    for (int kk = 0; kk < 4; ++kk) {
      int c = kk * t4 + t;
      acc = fmaf(q[c], k[c], acc);
    }
  return acc;
}

int or_canon_scores(const float* q, const float* k, int B, int N, int d, float* s) {
  if (d % 4 != 0) return 1;
  float sc = inv_sqrt_d(d);
  for (int b = 0; b < B; ++b)
    for (int i = 0; i < N; ++i)
      for (int j = 0; j < N; ++j) {
        float v = canon_dot(q + ((size_t)b * N + i) * d, k + ((size_t)b * N + j) * d, d) * sc;
        s[((size_t)b * N + i) * N + j] = (i == j) ? -INFINITY : v;
      }
  return 0;
}

/* Insert (x, j) into a list sorted by (value desc, index asc) of length n. */
static void insert_sorted(float* val, int* ix, int n, float x, int j) {
  int p = n;
  while (p > 0 && (x > val[p - 1] || (x == val[p - 1] && j < ix[p - 1]))) --p;
  if (p >= n) return;
  for (int m = n - 1; m > p; --m) { val[m] = val[m - 1]; ix[m] = ix[m - 1]; }
  val[p] = x; ix[p] = j;
}

int or_canon_topk(const float* q, const float* k, const float* v, int B, int N, int d, int topk,
                  double* out, int32_t* idx) {
  if (d % 4 != 0 || topk < 1 || topk > N - 1) return 1;
  float sc = inv_sqrt_d(d);
  float* val = (float*)malloc(sizeof(float) * topk);
  int* ix = (int*)malloc(sizeof(int) * topk);
  for (int b = 0; b < B; ++b)
    for (int i = 0; i < N; ++i) {
      const float* qi = q + ((size_t)b * N + i) * d;
      for (int m = 0; m < topk; ++m) { val[m] = -INFINITY; ix[m] = N; }
      for (int j = 0; j < N; ++j) {
        if (j == i) continue;
        float s = canon_dot(qi, k + ((size_t)b * N + j) * d, d) * sc;
        insert_sorted(val, ix, topk, s, j);
      }
      double mx = val[0], den = 0.0;
      double* o = out + ((size_t)b * N + i) * d;
      for (int c = 0; c < d; ++c) o[c] = 0.0;
      for (int m = 0; m < topk; ++m) {
        double w = exp((double)val[m] - mx);
        den += w;
        const float* vj = v + ((size_t)b * N + ix[m]) * d;
        for (int c = 0; c < d; ++c) o[c] += w * (double)vj[c];
        idx[((size_t)b * N + i) * topk + m] = ix[m];
      }
      for (int c = 0; c < d; ++c) o[c] /= den;
    }
  free(val);
  free(ix);
  return 0;
}

int or_dense(const float* q, const float* k, const float* v, int B, int N, int d, double* out) {
  double* s = (double*)malloc(sizeof(double) * N);
  double scale = 1.0 / sqrt((double)d);
  for (int b = 0; b < B; ++b)
    for (int i = 0; i < N; ++i) {
      const float* qi = q + ((size_t)b * N + i) * d;
      double mx = -INFINITY;
      for (int j = 0; j < N; ++j) {
        if (j == i) { s[j] = -INFINITY; continue; }
        const float* kj = k + ((size_t)b * N + j) * d;
        double acc = 0.0;
        for (int c = 0; c < d; ++c) acc += (double)qi[c] * (double)kj[c];
        s[j] = acc * scale;
        if (s[j] > mx) mx = s[j];
      }
      double den = 0.0;
      double* o = out + ((size_t)b * N + i) * d;
      for (int c = 0; c < d; ++c) o[c] = 0.0;
      for (int j = 0; j < N; ++j) {
        if (j == i) continue;
        double w = exp(s[j] - mx);
        den += w;
        const float* vj = v + ((size_t)b * N + j) * d;
        for (int c = 0; c < d; ++c) o[c] += w * (double)vj[c];
      }
      for (int c = 0; c < d; ++c) o[c] /= den;
    }
  free(s);
  return 0;
}

int or_fixedset(const float* q, const float* k, const float* v, const int64_t* idx, int kk, int B,
                int N, int d, double* out) {
  double scale = 1.0 / sqrt((double)d);
  double* s = (double*)malloc(sizeof(double) * (kk > 0 ? kk : 1));
  for (int b = 0; b < B; ++b)
    for (int i = 0; i < N; ++i) {
      const float* qi = q + ((size_t)b * N + i) * d;
      const int64_t* ii = idx + ((size_t)b * N + i) * kk;
      double mx = -INFINITY;
      for (int m = 0; m < kk; ++m) {
        if (ii[m] < 0 || ii[m] >= N) { free(s); return 2; }
        const float* kj = k + ((size_t)b * N + ii[m]) * d;
        double acc = 0.0;
        for (int c = 0; c < d; ++c) acc += (double)qi[c] * (double)kj[c];
        s[m] = acc * scale;
        if (s[m] > mx) mx = s[m];
      }
      double den = 0.0;
      double* o = out + ((size_t)b * N + i) * d;
      for (int c = 0; c < d; ++c) o[c] = 0.0;
      for (int m = 0; m < kk; ++m) {
        double w = exp(s[m] - mx);
        den += w;
        const float* vj = v + ((size_t)b * N + ii[m]) * d;
        for (int c = 0; c < d; ++c) o[c] += w * (double)vj[c];
      }
      for (int c = 0; c < d; ++c) o[c] /= den;
    }
  free(s);
  return 0;
}

/* Bit-by-bit interleave: x to the even bits, y to the odd bits. Deliberately a
 * different algorithm from the shift-and-mask spread the numpy oracle and the
 * kernels use, so the two check each other. */
static int64_t interleave(int64_t x, int64_t y, int bits) {
  int64_t c = 0;
  for (int b = 0; b < bits; ++b) {
    c |= ((x >> b) & 1) << (2 * b);
    c |= ((y >> b) & 1) << (2 * b + 1);
  }
  return c;
}

int or_morton_codes(const float* pos, int B, int N, int bits, int64_t* codes) {
  if (bits < 1 || bits > 16 || N < 1) return 1;
  const float top = (float)((1 << bits) - 1);
  for (int b = 0; b < B; ++b) {
    const float* p = pos + (size_t)b * N * 2;
    float lo[2] = {p[0], p[1]}, hi[2] = {p[0], p[1]};
    for (int i = 1; i < N; ++i)
      for (int a = 0; a < 2; ++a) {
        float x = p[2 * i + a];
        if (x < lo[a]) lo[a] = x;
        if (x > hi[a]) hi[a] = x;
      }
    float span[2];
    for (int a = 0; a < 2; ++a) {
      volatile float sp = hi[a] - lo[a];
      span[a] = sp < 1e-6f ? 1e-6f : sp;
    }
    for (int i = 0; i < N; ++i) {
      int64_t g[2];
      for (int a = 0; a < 2; ++a) {
        volatile float t = p[2 * i + a] - lo[a];
        volatile float u = t / span[a];
        volatile float w = u * top;
        int64_t gi = (int64_t)w; /* truncation toward zero, as Tensor.long() */
        if (gi < 0) gi = 0;
        if (gi > (1 << bits) - 1) gi = (1 << bits) - 1;
        g[a] = gi;
      }
      codes[(size_t)b * N + i] = interleave(g[0], g[1], bits);
    }
  }
  return 0;
}

typedef struct { int64_t code; int idx; } keyed;

static int cmp_keyed(const void* a, const void* b) {
  const keyed* x = (const keyed*)a;
  const keyed* y = (const keyed*)b;
  if (x->code != y->code) return x->code < y->code ? -1 : 1;
  return x->idx - y->idx;
}

int or_morton_window(const float* pos, int B, int N, int k, int bits, int64_t* idx) {
  if (k < 1 || k > N - 1) return 1;
  int64_t* codes = (int64_t*)malloc(sizeof(int64_t) * (size_t)B * N);
  int rc = or_morton_codes(pos, B, N, bits, codes);
  if (rc) { free(codes); return rc; }
  keyed* kv = (keyed*)malloc(sizeof(keyed) * N);
  int* rank = (int*)malloc(sizeof(int) * N);
  int* order = (int*)malloc(sizeof(int) * N);
  int half = (k + 1) / 2;
  for (int b = 0; b < B; ++b) {
    for (int i = 0; i < N; ++i) { kv[i].code = codes[(size_t)b * N + i]; kv[i].idx = i; }
    qsort(kv, N, sizeof(keyed), cmp_keyed);
    for (int r = 0; r < N; ++r) { order[r] = kv[r].idx; rank[kv[r].idx] = r; }
    for (int i = 0; i < N; ++i) {
      int64_t* o = idx + ((size_t)b * N + i) * k;
      int m = 0;
      for (int off = 1; off <= half; ++off) o[m++] = order[(rank[i] + off) % N];
      for (int off = 1; off <= k - half; ++off) o[m++] = order[((rank[i] - off) % N + N) % N];
    }
  }
  free(codes); free(kv); free(rank); free(order);
  return 0;
}
