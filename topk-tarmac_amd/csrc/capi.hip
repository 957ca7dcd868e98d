// extern "C" boundary of libtarmac.so: argument validation, launch-shape
// policy, error reporting. Declarations and reference citations: include/tarmac.h.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/tarmac.h"
#include "tarmac_internal.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return TARMAC_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(TARMAC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

constexpr size_t kLdsBudget = 64 * 1024;
constexpr size_t kBf16TopkLds = 49 * 1024;
// Head width 128: a 64-key block of fp32 keys and transposed values takes
// 69 KB, so those rows may use up to 80 KB (two workgroups per CU; gfx950
// has 160 KB of LDS per CU).
size_t lds_budget(int d) { return d > 64 ? 80 * 1024 : kLdsBudget; }
// Dense rows staged whole take the fixed exponent offset (no running
// maximum), so the dense kernel may use 80 KB (two workgroups per CU): rows
// of 512 keys at d = 32 then fit one chunk (bf16 B=4096 N=512: 334 -> 242
// us). At d = 64 the 256-key rows that would then fit ran slower at
// B >= 1024 (156 -> 163 us) than two chunks at 64 KB.
size_t dense_lds_budget(int d) { return d == 64 ? kLdsBudget : 80 * 1024; }
constexpr int kZorderMaxN = 4096;  // agents per row the Morton selector sorts
constexpr size_t kZorderLds = 160 * 1024;  // LDS per workgroup on gfx950

float inv_sqrt(int d) { return static_cast<float>(1.0 / std::sqrt(static_cast<double>(d))); }

int check_core(const void* q, const void* k, const void* v, const void* out, int B, int N, int d,
               int dtype, const char* fn) {
  if (!q || !k || !v || !out) return fail(TARMAC_ERR_INVALID, "%s: null tensor pointer", fn);
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16))
    return fail(TARMAC_ERR_INVALID, "%s: q, k, v and out must be 16-byte aligned", fn);
  if (B < 1 || N < 2)
    return fail(TARMAC_ERR_INVALID, "%s: need B >= 1 and N >= 2 (got B=%d, N=%d)", fn, B, N);
  if (dtype == tarmac::kF32) {
    if (d != 8 && d != 16 && d != 32 && d != 64 && d != 128)
      return fail(TARMAC_ERR_UNSUPPORTED, "%s: fp32 head dim must be 8, 16, 32, 64 or 128 (got %d)",
                  fn, d);
  } else if (dtype == tarmac::kBf16) {
    if (d != 16 && d != 32 && d != 64 && d != 128)
      return fail(TARMAC_ERR_UNSUPPORTED, "%s: bf16 head dim must be 16, 32, 64 or 128 (got %d)",
                  fn, d);
  } else {
    return fail(TARMAC_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  }
  if (static_cast<long long>(B) * N * d >= (1ll << 40))
    return fail(TARMAC_ERR_UNSUPPORTED, "%s: tensor too large", fn);
  return TARMAC_OK;
}

// Largest multiple of 64 keys whose padded LDS copy fits the budget.
int max_topk_chunk(int dtype, int d) {
  int kc = 64;
  while (tarmac::topk_lds_bytes(dtype, d, kc + 64) <= lds_budget(d)) kc += 64;
  return kc;
}

int topk_common(const void* q, const void* k, const void* v, void* out, int32_t* idx_out, int B,
                int N, int d, int topk, int dtype, int key_chunk, void* stream, const char* fn) {
  int rc = check_core(q, k, v, out, B, N, d, dtype, fn);
  if (rc) return rc;
  if (topk < 1 || topk > N - 1)
    return fail(TARMAC_ERR_INVALID, "%s: need 1 <= topk <= N-1 (got topk=%d, N=%d)", fn, topk, N);
  if (idx_out && !aligned(idx_out, 4)) return fail(TARMAC_ERR_INVALID, "%s: idx_out misaligned", fn);
  if (topk > tarmac::kTopkSmallMax && N + topk > 16384)
    return fail(TARMAC_ERR_UNSUPPORTED, "%s: topk > 8 needs N + topk <= 16384", fn);
  const int kmax = max_topk_chunk(dtype, d);
  const int n64 = (N + 63) / 64 * 64;
  int kc;
  if (key_chunk <= 0) {
    kc = n64 < kmax ? n64 : kmax;
    // bf16: keep the key copy within 49 KiB so three workgroups share a CU
    // (a whole 512-key row at d = 64 would allow two; a whole 1024-key row
    // at d = 16, 48 KiB of rows, runs 1.2x faster than 832-key chunks)
    if (dtype == tarmac::kBf16)
      while (kc > 64 && tarmac::topk_lds_bytes(dtype, d, kc) > kBf16TopkLds) kc -= 64;
  } else {
    if (key_chunk % 16 != 0)
      return fail(TARMAC_ERR_INVALID, "%s: key_chunk must be a multiple of 16 (got %d)", fn, key_chunk);
    if (tarmac::topk_lds_bytes(dtype, d, key_chunk) > lds_budget(d))
      return fail(TARMAC_ERR_UNSUPPORTED, "%s: key_chunk %d exceeds the LDS budget (max %d at d=%d)",
                  fn, key_chunk, kmax, d);
    kc = key_chunk;
  }
  // a chunk beyond the row is the resident row: LDS is sized for the row, not
  // the chunk (a larger allocation only costs workgroups per CU)
  if (kc > n64) kc = n64;
  tarmac::TopkArgs a{q, k, v, out, idx_out, B, N, d, topk, dtype, kc, inv_sqrt(d), stream};
  return hip_status(tarmac::run_topk(a), fn);
}

}  // namespace

extern "C" {

int tarmac_abi_version(void) { return 1; }

const char* tarmac_last_error(void) { return g_last_error.c_str(); }

namespace {

int dense_common(const void* q, const void* k, const void* v, void* out, float* stats, int B,
                 int N, int d, int dtype, int key_chunk, void* stream, const char* fn) {
  int rc = check_core(q, k, v, out, B, N, d, dtype, fn);
  if (rc) return rc;
  int kc = key_chunk;
  if (kc <= 0) {
    kc = (N + 63) / 64 * 64;
    while (kc > 64 && tarmac::dense_lds_bytes(dtype, d, kc) > dense_lds_budget(d)) kc -= 64;
    // a row in several chunks takes equal ones (N = 1024 as 512 + 512, not
    // 960 + 64): the same rounds, less LDS per workgroup
    const int nch = (N + kc - 1) / kc;
    if (nch > 1) kc = ((N + nch - 1) / nch + 63) / 64 * 64;
  } else if (kc % 16 != 0) {
    return fail(TARMAC_ERR_INVALID, "%s: key_chunk must be a multiple of 16 (got %d)", fn, kc);
  }
  if (tarmac::dense_lds_bytes(dtype, d, kc) > dense_lds_budget(d))
    return fail(TARMAC_ERR_UNSUPPORTED, "%s: key_chunk %d exceeds the LDS budget at d=%d", fn, kc, d);
  tarmac::DenseArgs a{q, k, v, out, B, N, d, dtype, kc, inv_sqrt(d), stream, stats};
  return hip_status(tarmac::run_dense(a), fn);
}

}  // namespace

int tarmac_dense_fwd(const void* q, const void* k, const void* v, void* out, int B, int N, int d,
                     int dtype, int key_chunk, void* stream) {
  return dense_common(q, k, v, out, nullptr, B, N, d, dtype, key_chunk, stream,
                      "tarmac_dense_fwd");
}

int tarmac_dense_fwd_stats(const float* q, const float* k, const float* v, float* out,
                           float* stats, int B, int N, int d, void* stream) {
  const char* fn = "tarmac_dense_fwd_stats";
  if (!stats || !aligned(stats, 8)) return fail(TARMAC_ERR_INVALID, "%s: stats null or misaligned", fn);
  return dense_common(q, k, v, out, stats, B, N, d, TARMAC_DTYPE_F32, 0, stream, fn);
}

int tarmac_topk_fused_fwd(const void* q, const void* k, const void* v, void* out, int32_t* idx_out,
                          int B, int N, int d, int topk, int dtype, void* stream) {
  return topk_common(q, k, v, out, idx_out, B, N, d, topk, dtype, 0, stream, "tarmac_topk_fused_fwd");
}

int tarmac_topk_stream_fwd(const void* q, const void* k, const void* v, void* out,
                           int32_t* idx_out, int B, int N, int d, int topk, int dtype,
                           int key_chunk, void* stream) {
  const char* fn = "tarmac_topk_stream_fwd";
  const int kmax = max_topk_chunk(dtype, d);
  if (key_chunk <= 0) key_chunk = kmax;
  if (key_chunk > kmax) key_chunk = kmax;
  return topk_common(q, k, v, out, idx_out, B, N, d, topk, dtype, key_chunk, stream, fn);
}

int tarmac_topk_variant_fwd(const void* q, const void* k, const void* v, void* out,
                            int32_t* idx_out, int B, int N, int d, int topk, int variant, int bisect,
                            int dtype, void* stream) {
  const char* fn = "tarmac_topk_variant_fwd";
  int rc = check_core(q, k, v, out, B, N, d, dtype, fn);
  if (rc) return rc;
  if (variant != TARMAC_VARIANT_MASKED && variant != TARMAC_VARIANT_SORT)
    return fail(TARMAC_ERR_INVALID, "%s: variant must be %d (masked) or %d (sort) (got %d)", fn,
                TARMAC_VARIANT_MASKED, TARMAC_VARIANT_SORT, variant);
  if (topk < 1 || topk > N - 1)
    return fail(TARMAC_ERR_INVALID, "%s: need 1 <= topk <= N-1 (got topk=%d, N=%d)", fn, topk, N);
  if (bisect < 0) return fail(TARMAC_ERR_INVALID, "%s: bisect must be >= 0 (got %d)", fn, bisect);
  if (variant == TARMAC_VARIANT_MASKED && idx_out)
    return fail(TARMAC_ERR_INVALID, "%s: the masked variant keeps a variable number of peers; "
                "idx_out must be NULL", fn);
  if (idx_out && !aligned(idx_out, 4)) return fail(TARMAC_ERR_INVALID, "%s: idx_out misaligned", fn);
  // key chunk of the register-list kernel, which serves fp32 k <= 8 (the
  // wide kernels ignore it): the whole row when it fits
  const int n64 = (N + 63) / 64 * 64, kmax = max_topk_chunk(dtype, d);
  tarmac::TopkArgs a{q, k, v, out, idx_out, B, N, d, topk, dtype, n64 < kmax ? n64 : kmax,
                     inv_sqrt(d), stream};
  a.select = variant == TARMAC_VARIANT_MASKED ? tarmac::kSelMasked : tarmac::kSelSort;
  a.bisect = bisect;
  if (static_cast<size_t>(N + tarmac::wide_cap(a)) * 4 > kLdsBudget)
    return fail(TARMAC_ERR_UNSUPPORTED, "%s: N=%d too large for one score row in LDS", fn, N);
  return hip_status(tarmac::run_topk(a), fn);
}

int tarmac_fixedset_fwd(const void* q, const void* k, const void* v, const void* idx,
                        int idx_dtype, int kk, void* out, int B, int N, int d, int dtype,
                        void* stream) {
  const char* fn = "tarmac_fixedset_fwd";
  int rc = check_core(q, k, v, out, B, N, d, dtype, fn);
  if (rc) return rc;
  if (kk < 1) return fail(TARMAC_ERR_INVALID, "%s: need kk >= 1 (got %d)", fn, kk);
  if (!idx) return fail(TARMAC_ERR_INVALID, "%s: null idx", fn);
  if (idx_dtype != TARMAC_IDX_I32 && idx_dtype != TARMAC_IDX_I64)
    return fail(TARMAC_ERR_INVALID, "%s: unknown idx dtype %d", fn, idx_dtype);
  if (!aligned(idx, idx_dtype == TARMAC_IDX_I64 ? 8 : 4))
    return fail(TARMAC_ERR_INVALID, "%s: idx misaligned", fn);
  tarmac::FixedsetArgs a{q, k, v, idx, idx_dtype == TARMAC_IDX_I64, out, B, N, d, kk, dtype,
                         inv_sqrt(d), stream};
  return hip_status(tarmac::run_fixedset(a), fn);
}

int tarmac_morton_window(const float* pos, void* idx_out, int idx_dtype, int64_t* codes_out,
                         int B, int N, int k, int bits, void* stream) {
  const char* fn = "tarmac_morton_window";
  if (!pos) return fail(TARMAC_ERR_INVALID, "%s: null pos", fn);
  if (!aligned(pos, 8)) return fail(TARMAC_ERR_INVALID, "%s: pos must be 8-byte aligned", fn);
  if (B < 1 || N < 2) return fail(TARMAC_ERR_INVALID, "%s: need B >= 1 and N >= 2", fn);
  if (bits < 1 || bits > 16) return fail(TARMAC_ERR_INVALID, "%s: bits must be 1..16 (got %d)", fn, bits);
  if (idx_out) {
    if (k < 1 || k > N - 1)
      return fail(TARMAC_ERR_INVALID, "%s: need 1 <= k <= N-1 (got k=%d, N=%d)", fn, k, N);
    if (idx_dtype != TARMAC_IDX_I32 && idx_dtype != TARMAC_IDX_I64)
      return fail(TARMAC_ERR_INVALID, "%s: unknown idx dtype %d", fn, idx_dtype);
    if (!aligned(idx_out, idx_dtype == TARMAC_IDX_I64 ? 8 : 4))
      return fail(TARMAC_ERR_INVALID, "%s: idx_out misaligned", fn);
  }
  if (codes_out && !aligned(codes_out, 8)) return fail(TARMAC_ERR_INVALID, "%s: codes_out misaligned", fn);
  if (N > kZorderMaxN || tarmac::zorder_lds_bytes(N) > kZorderLds)
    return fail(TARMAC_ERR_UNSUPPORTED, "%s: N=%d exceeds the per-row sort capacity (%d)", fn, N,
                kZorderMaxN);
  tarmac::MortonArgs a{pos, idx_out, idx_dtype == TARMAC_IDX_I64, codes_out, B, N, k, bits, stream};
  return hip_status(tarmac::run_morton_window(a), fn);
}

namespace {

int knn_common(const float* pos, void* idx_out, int idx_dtype, int B, int N, int k, int grid,
               void* stream, const char* fn) {
  if (!pos || !idx_out) return fail(TARMAC_ERR_INVALID, "%s: null pos or idx_out", fn);
  if (!aligned(pos, 8)) return fail(TARMAC_ERR_INVALID, "%s: pos must be 8-byte aligned", fn);
  if (B < 1 || N < 2) return fail(TARMAC_ERR_INVALID, "%s: need B >= 1 and N >= 2", fn);
  if (k < 1 || k > N - 1)
    return fail(TARMAC_ERR_INVALID, "%s: need 1 <= k <= N-1 (got k=%d, N=%d)", fn, k, N);
  if (idx_dtype != TARMAC_IDX_I32 && idx_dtype != TARMAC_IDX_I64)
    return fail(TARMAC_ERR_INVALID, "%s: unknown idx dtype %d", fn, idx_dtype);
  if (!aligned(idx_out, idx_dtype == TARMAC_IDX_I64 ? 8 : 4))
    return fail(TARMAC_ERR_INVALID, "%s: idx_out misaligned", fn);
  if (static_cast<long long>(B) * N * k >= (1ll << 40))
    return fail(TARMAC_ERR_UNSUPPORTED, "%s: tensor too large", fn);
  tarmac::KnnArgs a{pos, idx_out, idx_dtype == TARMAC_IDX_I64, B, N, k, 0, 0, 0, stream};
  if (grid) {
    int G = 0, M = 0;
    tarmac::grid_knn_shape(N, k, &G, &M);
    // the reference's own route: all pairs when the 3x3 block would hold N or more
    if (9ll * M < N) {
      a.grid = 1;
      a.G = G;
      a.L = 3 * M;
      if (tarmac::knn_grid_lds_bytes(N, G, tarmac::knn_grid_threads(N)) > kLdsBudget)
        return fail(TARMAC_ERR_UNSUPPORTED, "%s: N=%d exceeds the per-row grid capacity", fn, N);
    }
  }
  if (!a.grid && tarmac::knn_radius_lds_bytes(N) > kLdsBudget)
    return fail(TARMAC_ERR_UNSUPPORTED, "%s: N=%d exceeds the per-row position capacity", fn, N);
  return hip_status(tarmac::run_knn(a), fn);
}

}  // namespace

int tarmac_knn_radius(const float* pos, void* idx_out, int idx_dtype, int B, int N, int k,
                      void* stream) {
  return knn_common(pos, idx_out, idx_dtype, B, N, k, 0, stream, "tarmac_knn_radius");
}

int tarmac_knn_grid(const float* pos, void* idx_out, int idx_dtype, int B, int N, int k,
                    void* stream) {
  return knn_common(pos, idx_out, idx_dtype, B, N, k, 1, stream, "tarmac_knn_grid");
}

int tarmac_grid_knn_shape(int N, int k, int* G, int* M) {
  if (!G || !M) return fail(TARMAC_ERR_INVALID, "tarmac_grid_knn_shape: null output");
  if (N < 1 || k < 1) return fail(TARMAC_ERR_INVALID, "tarmac_grid_knn_shape: need N >= 1, k >= 1");
  tarmac::grid_knn_shape(N, k, G, M);
  return ok();
}

int tarmac_zorder_fwd(const void* q, const void* k, const void* v, const float* pos, void* out,
                      int32_t* idx_out, int B, int N, int d, int topk, int bits, int dtype,
                      void* stream) {
  const char* fn = "tarmac_zorder_fwd";
  int rc = check_core(q, k, v, out, B, N, d, dtype, fn);
  if (rc) return rc;
  if (!pos || !aligned(pos, 8)) return fail(TARMAC_ERR_INVALID, "%s: pos null or misaligned", fn);
  if (topk < 1 || topk > N - 1)
    return fail(TARMAC_ERR_INVALID, "%s: need 1 <= topk <= N-1 (got topk=%d, N=%d)", fn, topk, N);
  if (bits < 1 || bits > 16) return fail(TARMAC_ERR_INVALID, "%s: bits must be 1..16 (got %d)", fn, bits);
  if (idx_out && !aligned(idx_out, 4)) return fail(TARMAC_ERR_INVALID, "%s: idx_out misaligned", fn);
  if (N > kZorderMaxN || tarmac::zorder_lds_bytes(N) > kZorderLds)
    return fail(TARMAC_ERR_UNSUPPORTED, "%s: N=%d exceeds the per-row sort capacity (%d)", fn, N,
                kZorderMaxN);
  tarmac::ZorderArgs a{q, k, v, pos, out, idx_out, B, N, d, topk, bits, dtype, inv_sqrt(d), stream};
  return hip_status(tarmac::run_zorder(a), fn);
}

int tarmac_fixedset_bwd(const float* q, const float* k, const float* v, const float* dout,
                        const void* idx, int idx_dtype, int kk, float* dq, float* dk, float* dv,
                        int B, int N, int d, void* stream) {
  const char* fn = "tarmac_fixedset_bwd";
  int rc = check_core(q, k, v, dout, B, N, d, TARMAC_DTYPE_F32, fn);
  if (rc) return rc;
  if (!idx || !dq || !dk || !dv) return fail(TARMAC_ERR_INVALID, "%s: null pointer", fn);
  if (!aligned(dq, 16) || !aligned(dk, 16) || !aligned(dv, 16))
    return fail(TARMAC_ERR_INVALID, "%s: gradient buffers must be 16-byte aligned", fn);
  if (idx_dtype != TARMAC_IDX_I32 && idx_dtype != TARMAC_IDX_I64)
    return fail(TARMAC_ERR_INVALID, "%s: idx_dtype must be TARMAC_IDX_I32 or TARMAC_IDX_I64", fn);
  if (kk < 1) return fail(TARMAC_ERR_INVALID, "%s: kk must be >= 1 (got %d)", fn, kk);
  tarmac::FixedsetBwdArgs a{q, k, v, dout, idx, idx_dtype == TARMAC_IDX_I64, dq, dk, dv,
                            B, N, d, kk, inv_sqrt(d), stream};
  return hip_status(tarmac::run_fixedset_bwd(a), fn);
}

int tarmac_dense_bwd(const float* q, const float* k, const float* v, const float* out,
                     const float* dout, float* dq, float* dk, float* dv, float* stats,
                     int stats_ready, int B, int N, int d, void* stream) {
  const char* fn = "tarmac_dense_bwd";
  int rc = check_core(q, k, v, out, B, N, d, TARMAC_DTYPE_F32, fn);
  if (rc) return rc;
  if (!dout || !dq || !dk || !dv || !stats) return fail(TARMAC_ERR_INVALID, "%s: null pointer", fn);
  if (!aligned(dout, 16) || !aligned(dq, 16) || !aligned(dk, 16) || !aligned(dv, 16) ||
      !aligned(stats, 8))
    return fail(TARMAC_ERR_INVALID, "%s: misaligned buffer", fn);
  if (stats_ready != 0 && stats_ready != 1)
    return fail(TARMAC_ERR_INVALID, "%s: stats_ready must be 0 or 1", fn);
  tarmac::DenseBwdArgs a{q, k, v, out, dout, dq, dk, dv, stats, stats_ready, B, N, d,
                         inv_sqrt(d), stream};
  return hip_status(tarmac::run_dense_bwd(a), fn);
}

int tarmac_dense_bwd_noalloc(const float* q, const float* k, const float* v, const float* out,
                             const float* dout, float* dq, float* dk, float* dv, int B, int N,
                             int d, void* stream) {
  const char* fn = "tarmac_dense_bwd_noalloc";
  int rc = check_core(q, k, v, out, B, N, d, TARMAC_DTYPE_F32, fn);
  if (rc) return rc;
  if (!dout || !dq || !dk || !dv) return fail(TARMAC_ERR_INVALID, "%s: null pointer", fn);
  if (!aligned(dout, 16) || !aligned(dq, 16) || !aligned(dk, 16) || !aligned(dv, 16))
    return fail(TARMAC_ERR_INVALID, "%s: misaligned buffer", fn);
  const size_t need = size_t(2) * size_t(B) * size_t(N) * sizeof(float);
  if (need > tarmac::kScratchBytes)
    return fail(TARMAC_ERR_UNSUPPORTED,
                "%s: the [B, 2, N] statistics need %zu bytes, more than the library's %zu-byte "
                "scratch (B * N <= %zu); use tarmac_dense_bwd with a caller workspace",
                fn, need, tarmac::kScratchBytes, tarmac::kScratchBytes / (2 * sizeof(float)));
  void* ws = nullptr;
  hipError_t e = tarmac::scratch_address(&ws);
  if (e != hipSuccess) return hip_status(e, fn);
  // every statistic is written by the first pass before the second reads it:
  // nothing in the scratch needs clearing
  tarmac::DenseBwdArgs a{q, k, v, out, dout, dq, dk, dv, static_cast<float*>(ws), 0, B, N, d,
                         inv_sqrt(d), stream};
  return hip_status(tarmac::run_dense_bwd(a), fn);
}

int tarmac_set_topk_filter(int mode) {
  if (mode < tarmac::kFilterOff || mode > tarmac::kFilterSplit32) {
    fail(TARMAC_ERR_INVALID, "tarmac_set_topk_filter: mode must be 0 to 5 (got %d)", mode);
    return -1;
  }
  return tarmac::set_topk_filter_mode(mode);
}

int tarmac_set_query_tiles(int mode) {
  if (mode < tarmac::kTilesAuto || mode > tarmac::kTilesTwo) {
    fail(TARMAC_ERR_INVALID, "tarmac_set_query_tiles: mode must be 0 to 2 (got %d)", mode);
    return -1;
  }
  return tarmac::set_query_tiles_mode(mode);
}

int tarmac_mfma_bf16_probe(const void* a, const void* b, float* out, int tiles, int chain,
                           int shape, void* stream) {
  const char* fn = "tarmac_mfma_bf16_probe";
  if (!a || !b || !out) return fail(TARMAC_ERR_INVALID, "%s: null pointer", fn);
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(out, 16))
    return fail(TARMAC_ERR_INVALID, "%s: operands must be 16-byte aligned", fn);
  if (tiles < 1 || chain < 1 || chain > 64)
    return fail(TARMAC_ERR_INVALID, "%s: need tiles >= 1 and 1 <= chain <= 64", fn);
  if (shape != 16 && shape != 32) return fail(TARMAC_ERR_INVALID, "%s: shape must be 16 or 32", fn);
  return hip_status(tarmac::run_mfma_bf16_probe(a, b, out, tiles, chain, shape, stream), fn);
}

int tarmac_noop(float* out, void* stream) {
  if (!out) return fail(TARMAC_ERR_INVALID, "tarmac_noop: null out");
  return hip_status(tarmac::run_noop(out, stream), "tarmac_noop");
}

}  // extern "C"
