// Internal launch descriptors shared by the kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tarmac {

enum Dtype : int { kF32 = 0, kBf16 = 1 };

constexpr int kTopkSmallMax = 8;    // k handled by the register-list kernel
constexpr int kTopkQueryTiles = 2;  // 16-query tiles per wavefront

inline int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

struct TopkArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int32_t* idx;     // nullable: retained indices [B, N, topk]
  int B, N, d, topk, dtype;
  int key_chunk;    // keys per LDS chunk (multiple of 16)
  float scale;      // fp32(1/sqrt(d))
  void* stream;
  int select = 0;   // kSelTopk / kSelMasked / kSelSort
  int bisect = 0;   // kSelMasked: bisection halvings
};

// Selection rules (TARMAC_VARIANT_* in include/tarmac.h).
constexpr int kSelTopk = 0, kSelMasked = 1, kSelSort = 2;
int wide_cap(const TopkArgs& a);

struct DenseArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int B, N, d, dtype;
  int key_chunk;
  float scale;
  void* stream;
  float* stats = nullptr;  // nullable: [B, 2, N] workspace, plane 0 gets the logsumexp
};

struct FixedsetArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* idx;
  int idx_is_i64;
  void* out;
  int B, N, d, kk, dtype;
  float scale;
  void* stream;
};

struct FixedsetBwdArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* dout;
  const void* idx;
  int idx_is_i64;
  float* dq;        // written
  float* dk;        // written
  float* dv;        // written
  int B, N, d, kk;
  float scale;
  void* stream;
};

struct DenseBwdArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* out;
  const float* dout;
  float* dq;
  float* dk;
  float* dv;
  float* stats;     // workspace [B, 2, N]: logsumexp and dO.O per query
  int stats_ready;  // plane 0 already holds the forward's logsumexp
  int B, N, d;
  float scale;
  void* stream;
};

struct MortonArgs {
  const float* pos;
  void* idx;          // nullable
  int idx_is_i64;
  int64_t* codes;     // nullable: Morton codes [B, N]
  int B, N, k, bits;
  void* stream;
};

struct ZorderArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* pos;
  void* out;
  int32_t* idx;  // nullable
  int B, N, d, topk, bits, dtype;
  float scale;
  void* stream;
};

struct KnnArgs {
  const float* pos;   // [B, N, 2]
  void* idx;          // [B, N, k]
  int idx_is_i64;
  int B, N, k;
  int grid;           // 0: all pairs; 1: 3x3 grid cells
  int G, L;           // grid side and run capacity (3 * cell capacity)
  void* stream;
};

hipError_t run_topk(const TopkArgs& a);
hipError_t run_topk_filter(const TopkArgs& a);
hipError_t run_topk_packed(const TopkArgs& a, bool split);
hipError_t run_topk_packed_d128(const TopkArgs& a);  // topk_packed_d128.hip
bool split32_supported(const TopkArgs& a);  // d = 16, k <= 4, N <= 256 (bf16: 1024), top-k rule
hipError_t run_topk_split32(const TopkArgs& a);
size_t split32_lds_bytes(int dtype, int kc);
bool topk_hist_supported(const TopkArgs& a);  // fp32, d = 16, k > 8, N <= 512
hipError_t run_topk_hist(const TopkArgs& a);
bool packed_split_supported(int dtype, int d);
bool topk_filter_supported(int dtype, int d, int topk);
// tarmac_set_topk_filter modes
constexpr int kFilterOff = 0, kFilterAuto = 1, kFilterAlways = 2, kFilterLegacy = 3,
              kFilterPackedSplit = 4, kFilterSplit32 = 5;
int topk_filter_mode();
int set_topk_filter_mode(int mode);  // returns the previous mode
// tarmac_set_query_tiles modes: 16-query tiles per wave in the dense, packed
// (k <= 4, N <= 1024) and bf16 filter kernels
constexpr int kTilesAuto = 0, kTilesOne = 1, kTilesTwo = 2;
int set_query_tiles_mode(int mode);  // returns the previous mode
bool one_query_tile(int B, int N);   // the launch shape under the current mode
int query_tiles_mode();              // kTilesAuto, kTilesOne or kTilesTwo
hipError_t run_dense(const DenseArgs& a);
hipError_t run_fixedset(const FixedsetArgs& a);
hipError_t run_morton_window(const MortonArgs& a);
hipError_t run_zorder(const ZorderArgs& a);
hipError_t run_noop(float* out, void* stream);
hipError_t run_mfma_bf16_probe(const void* a, const void* b, float* out, int T, int chain,
                               int shape, void* stream);
hipError_t run_fixedset_bwd(const FixedsetBwdArgs& a);
hipError_t run_dense_bwd(const DenseBwdArgs& a);
// Library-held device workspace (one per GPU, kScratchBytes): the current
// device's address of it, looked up on the first call on that device.
constexpr size_t kScratchBytes = size_t(8) << 20;
hipError_t scratch_address(void** out);
hipError_t run_knn(const KnnArgs& a);
void grid_knn_shape(int N, int k, int* G, int* M);
int knn_grid_threads(int N);

size_t topk_lds_bytes(int dtype, int d, int kc);
size_t packed_lds_bytes(int dtype, int d, int kc, bool split);  // topk_packed_kernel's key copy
size_t plain_lds_bytes(int dtype, int d, int kc);  // topk_small_kernel's key copy
size_t topk_filter_lds_bytes(int dtype, int d, int kc);
size_t dense_lds_bytes(int dtype, int d, int kc);
size_t zorder_lds_bytes(int N);
size_t knn_radius_lds_bytes(int N);
size_t knn_grid_lds_bytes(int N, int G, int threads);

}  // namespace tarmac
