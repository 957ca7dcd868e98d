/*
 * tarmac.h -- C ABI of the MI355X-native TarMAC attention core (libtarmac.so).
 *
 * Every entry point takes plain device pointers to row-major contiguous
 * [B, N, d] tensors (16-byte aligned), sizes, and an opaque stream handle
 * (a hipStream_t; NULL is the null stream). Nothing is allocated, nothing is
 * synchronised: the kernels are enqueued on `stream` and the call returns.
 * Return value: TARMAC_OK, or an error code whose message is available from
 * tarmac_last_error() on the calling thread. Calls are reentrant, with one
 * exception: tarmac_dense_bwd_noalloc shares one library-held array per GPU,
 * so its calls that overlap on one GPU race (see its declaration).
 *
 * Head widths d: 8, 16, 32, 64 or 128 for fp32, 16, 32, 64 or 128 for bf16
 * (the module pads other msg_dim up to 128 with zeros). At d = 128, top-k
 * with k <= 8 runs the packed kernel under every mode of
 * tarmac_set_topk_filter, and larger k and the variants the wide kernels.
 *
 * Scores are q.k / sqrt(d) with the self pair (i == i) excluded, as in every
 * path of the reference. Retained sets are the topk largest scores, ties to
 * the lower agent index. fp32 scores are formed in a fixed fmaf order
 * (element c = kk*(d/4) + t at step t, slot kk), so results are reproducible
 * bit for bit; bf16 inputs are ranked by that same fp32 score of the inputs
 * converted to fp32 (the retained set is exact, not an approximation).
 *
 * Reference paths below are relative to the MHHamdan/TopK-TarMAC checkout.
 */
#ifndef TARMAC_H_
#define TARMAC_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TARMAC_OK 0
#define TARMAC_ERR_INVALID 1     /* bad shape, dtype, k, pointer or alignment */
#define TARMAC_ERR_UNSUPPORTED 2 /* valid request outside what the kernels cover */
#define TARMAC_ERR_HIP 3         /* the HIP runtime rejected the launch */

#define TARMAC_DTYPE_F32 0
#define TARMAC_DTYPE_BF16 1

#define TARMAC_IDX_I32 0
#define TARMAC_IDX_I64 1

/* ABI version of this header (bumped on any signature change). */
int tarmac_abi_version(void);

/* Message for the last non-OK return on this thread ("" if none). */
const char* tarmac_last_error(void);

/*
 * Dense attention, softmax over all N-1 peers.
 * Replaces src/kernels/fused_dense_attention.py:106-152 (fused_dense_attention)
 * and the composed dense paths scripts/bench_attention_core.py:74-82
 * (dense_unfused, dense_fused) / src/agents/mappo.py:174-190,361-372,418.
 * key_chunk: keys staged per LDS pass (0 = whole row when it fits).
 */
int tarmac_dense_fwd(const void* q, const void* k, const void* v, void* out, int B, int N, int d,
                     int dtype, int key_chunk, void* stream);

/*
 * Fused score-then-select top-k with the key row resident on chip.
 * Replaces src/kernels/fused_topk_attention.py:296-355
 * (fused_topk_attention_tiled, fused_topk_attention), the composed gather path
 * src/kernels/fused_topk_attention.py:390-402 / src/agents/mappo.py:192-231,
 * and the masked form src/agents/mappo.py:374-382 (same function).
 * Requires 1 <= topk <= N-1. idx_out (nullable): int32 [B, N, topk], ordered
 * by (score desc, index asc) for topk <= 8 and by ascending index above.
 */
int tarmac_topk_fused_fwd(const void* q, const void* k, const void* v, void* out, int32_t* idx_out,
                          int B, int N, int d, int topk, int dtype, void* stream);

/*
 * Streaming top-k: keys pass through LDS in chunks of key_chunk rows (<= 0:
 * the largest chunk the LDS budget holds), so the N-wide score row is never
 * resident; no cap on N.
 * Replaces src/kernels/streaming_topk_attention.py:206-258
 * (streaming_topk_attention, including return_indices).
 */
int tarmac_topk_stream_fwd(const void* q, const void* k, const void* v, void* out,
                           int32_t* idx_out, int B, int N, int d, int topk, int dtype,
                           int key_chunk, void* stream);

/*
 * The reference's two other resident selection rules (one wavefront per query
 * row, the score row in LDS; N + kept <= 16384):
 *   TARMAC_VARIANT_MASKED: every peer whose score key is >= the threshold
 *     left by `bisect` halvings of the integer bisection -- exact top-k plus
 *     every peer tied at the k-th score when bisect >= 32.
 *     Replaces src/kernels/fused_topk_attention.py:127-208,358-387
 *     (_fused_topk_masked_kernel, fused_topk_attention_masked). idx_out must
 *     be NULL (the kept count varies).
 *   TARMAC_VARIANT_SORT: exactly topk, ties at the k-th score keep the higher
 *     indices. Replaces src/kernels/fused_topk_attention.py:405-540
 *     (_fused_topk_sort_kernel, fused_topk_attention_sort). idx_out
 *     (nullable) in ascending index order.
 * bisect is ignored for the sort variant.
 */
#define TARMAC_VARIANT_MASKED 1
#define TARMAC_VARIANT_SORT 2
int tarmac_topk_variant_fwd(const void* q, const void* k, const void* v, void* out,
                            int32_t* idx_out, int B, int N, int d, int topk, int variant, int bisect,
                            int dtype, void* stream);

/*
 * Attention over a given peer set idx [B, N, kk] (int32 or int64).
 * Replaces src/kernels/fused_prescore_attention.py:88-114
 * (fused_prescore_attention) and src/kernels/prescore_selection.py:184-195
 * (prescore_attention). Out-of-range indices are never dereferenced; their
 * query rows come out NaN.
 */
int tarmac_fixedset_fwd(const void* q, const void* k, const void* v, const void* idx,
                        int idx_dtype, int kk, void* out, int B, int N, int d, int dtype,
                        void* stream);

/*
 * Z-order selector: per-batch Morton codes of pos [B, N, 2] (fp32) at `bits`
 * bits per axis, agents sorted by code (equal codes by agent index), and each
 * agent's k curve neighbours (+1..+ceil(k/2), -1..-floor(k/2), wrapping).
 * Replaces src/kernels/prescore_selection.py:62-84
 * (_morton_code, select_morton_window). idx_out [B, N, k] (int32 or int64,
 * nullable); codes_out int64 [B, N] (nullable). Requires 1 <= k <= N-1.
 */
int tarmac_morton_window(const float* pos, void* idx_out, int idx_dtype, int64_t* codes_out,
                         int B, int N, int k, int bits, void* stream);

/*
 * k nearest peers per agent over all pairs: select_radius_knn
 * (src/kernels/prescore_selection.py:35-42). pos fp32 [B, N, 2] (8-byte
 * aligned); idx_out [B, N, k], int32 or int64. Squared fp32 distances
 * (dx*dx + dy*dy, each operation rounded); the k smallest by (distance, agent
 * index), the self pair excluded; emitted in ascending agent index. Requires
 * 1 <= k <= N-1 and N <= 8192.
 */
int tarmac_knn_radius(const float* pos, void* idx_out, int idx_dtype, int B, int N, int k,
                      void* stream);

/*
 * k nearest peers among the 3x3 grid cells around each agent: select_grid_knn
 * (src/kernels/prescore_selection.py:107-164), grid shape from grid_knn_shape
 * (:87-101). Agents are ordered by cell (equal cells by agent index); each
 * neighbour column contributes a run of at most 3M agents; the k smallest
 * slots by (distance, slot) are kept, emitted in ascending slot. Routes to
 * tarmac_knn_radius when 9M >= N, as the reference does. N <= 4096.
 */
int tarmac_knn_grid(const float* pos, void* idx_out, int idx_dtype, int B, int N, int k,
                    void* stream);

/* grid_knn_shape (src/kernels/prescore_selection.py:87-101): grid side G and
 * per-cell capacity M for N agents and k peers. Host only. */
int tarmac_grid_knn_shape(int N, int k, int* G, int* M);

/*
 * Selector and attention in one launch: the zorder_k core of
 * src/agents/mappo.py:265-292 and the "select+attend" total of
 * scripts/bench_prescore.py:253-257. idx_out: int32 [B, N, topk], nullable.
 */
int tarmac_zorder_fwd(const void* q, const void* k, const void* v, const float* pos, void* out,
                      int32_t* idx_out, int B, int N, int d, int topk, int bits, int dtype,
                      void* stream);

/*
 * Backward of attention over a given peer set idx [B, N, kk] (fp32): the
 * gradients of the top-k core with the set its forward retained (gradients
 * flow only through the retained scores and value rows, as for torch.topk's
 * gather), of the Z-order core with its selector's set, and of prescore
 * attention. dq, dk and dv are written. Each key's dk, dv are summed over
 * the queries that retain it in ascending query order, so they are bitwise
 * reproducible, except in a batch row whose sets name a peer twice, when N
 * is too large for the row's N x N bitmask in LDS (N above about 1100 at
 * d = 16), or at d = 128: there they are summed with fp32 atomics, whose low
 * bits depend on the order the adds land in. No kernel counterpart in the reference (its Triton kernels are
 * forward-only, scripts/bench_attention_core.py:172-176); replaces autograd
 * through src/agents/mappo.py:192-231 in src/training/train_mappo.py:366.
 */
int tarmac_fixedset_bwd(const float* q, const float* k, const float* v, const float* dout,
                        const void* idx, int idx_dtype, int kk, float* dq, float* dk, float* dv,
                        int B, int N, int d, void* stream);

/*
 * tarmac_dense_fwd for training (fp32, default key chunk): also writes the
 * queries' log2-domain logsumexp into plane 0 of stats ([B, 2, N] floats),
 * for tarmac_dense_bwd with stats_ready = 1. No kernel counterpart in the
 * reference (its dense kernel is forward-only).
 */
int tarmac_dense_fwd_stats(const float* q, const float* k, const float* v, float* out,
                           float* stats, int B, int N, int d, void* stream);

/*
 * Backward of dense attention (fp32, self pair excluded): dq, dk, dv are
 * written. stats: workspace of 2 * B * N floats, [B, 2, N]: plane 0 the
 * queries' log2-domain logsumexp (taken as given when stats_ready = 1, i.e.
 * written by tarmac_dense_fwd_stats on the same inputs; computed here when
 * 0), plane 1 their dO.O (always computed here). No kernel counterpart in
 * the reference; replaces autograd through src/agents/mappo.py:361-372 in
 * training.
 */
int tarmac_dense_bwd(const float* q, const float* k, const float* v, const float* out,
                     const float* dout, float* dq, float* dk, float* dv, float* stats,
                     int stats_ready, int B, int N, int d, void* stream);

/*
 * tarmac_dense_bwd (stats_ready = 0) that allocates nothing: its [B, 2, N]
 * statistics live in a library-held device array of 8 MiB per GPU (so
 * B * N <= 1048576; larger calls return TARMAC_ERR_UNSUPPORTED), resident
 * until the process ends. Calls no hipMalloc or allocating routine. Every
 * call on one GPU shares that array: calls that overlap on one GPU (two
 * streams, two threads) race and must be serialised by the caller. No
 * counterpart in the reference; for callers that cannot allocate device
 * memory (code under graph capture, serving loops that forbid hipMalloc).
 */
int tarmac_dense_bwd_noalloc(const float* q, const float* k, const float* v, const float* out,
                             const float* dout, float* dq, float* dk, float* dv, int B, int N,
                             int d, void* stream);

/*
 * Which of four equally exact implementations serves topk <= 8 (the retained
 * set is identical whichever runs, and for fp32 the outputs too, bit for bit;
 * for bf16 the outputs agree to bf16 rounding: the packed pass may compute
 * the softmax of a proven set on its truncated scores, within the proof's
 * bound, the other paths on the canonical scores; only the time differs):
 *   packed       -- scores with the key's position in their low mantissa
 *                   bits, lists of k+2 values kept with max / med3, a proof
 *                   that the truncation (fp32) or the bf16 score error bound
 *                   (bf16) cannot change the top k, and exact canonical
 *                   rescoring of the k+1 candidates where it is needed;
 *   packed split -- the packed pass on split-bf16 scores (fp32 inputs,
 *                   d = 16: x = hi + mid + lo, six bf16 products per score),
 *                   proven against the split error bound;
 *   split32      -- the same on 32-key x 32-query tiles (d = 16, k <= 4,
 *                   N <= 256, bf16 N <= 1024): two lanes per query instead
 *                   of four; bf16
 *                   inputs take one bf16 product per tile (the inputs as
 *                   they are) instead of six split products;
 *   filter       -- all pairs scored on split-bf16 MFMA (fp32 inputs) or
 *                   bf16 MFMA (bf16, d = 16), k+1 candidates rescored in the
 *                   canonical fp32 order and proven against the bf16 bound;
 *   lists        -- fp32 MFMA scores and per-score (score, index) register
 *                   lists (fp32 inputs; bf16 widened to fp32 at d = 16).
 * In the packed and filter paths a query whose proof fails (near-ties) is
 * recomputed by one wavefront from its canonical scores (per-lane lists
 * merged across the wave); the other queries of its tile keep their proven
 * sets. The lists path selects on canonical scores and needs no proof.
 * The exactness of the bf16 and split-bf16 proofs rests on a bound for the
 * bf16 MFMA's fp32 accumulation error that is measured, not derived: at most
 * 2^-20.25 of the sum of product magnitudes (worst seen on gfx950: 2^-20.5,
 * one dominant product among small ones; tarmac_mfma_bf16_probe measures
 * it), inside eps = 2^-18 at d <= 32, 2^-17 at d = 64 and 2^-16 at d = 128
 * together with the canonical chain's d 2^-24.
 * mode: 0 = packed always, 1 = automatic (default; the fastest measured on
 * MI355X for the shape), 2 = filter where supported (fp32 d = 16, 32, 64;
 * bf16 d = 16), 3 = lists for fp32 (bf16 runs packed), 4 = packed split where
 * supported (fp32 d = 16; packed elsewhere), 5 = split32 where supported
 * (d = 16, k <= 4, N <= 256 for fp32 and 1024 for bf16; packed split,
 * then packed, elsewhere). bf16 retained sets are always
 * the exact top k of the canonical fp32 scores of the inputs converted to
 * fp32. Process-wide (an atomic setting: concurrent calls stay safe and get
 * identical results). Returns the previous mode, or -1 (and sets the last
 * error) for an invalid mode. No counterpart in the reference (its kernels
 * have one path).
 */
#define TARMAC_FILTER_OFF 0
#define TARMAC_FILTER_AUTO 1
#define TARMAC_FILTER_ALWAYS 2
#define TARMAC_FILTER_LISTS 3
#define TARMAC_FILTER_PACKED_SPLIT 4
#define TARMAC_FILTER_SPLIT32 5
int tarmac_set_topk_filter(int mode);

/*
 * 16-query tiles per wavefront in the dense kernel, the packed top-k pass
 * (topk <= 4, N <= 1024) and the bf16 filter kernel: 0 = automatic (default:
 * two, or one when B * ceil(N / 32) < 1024, which would leave SIMDs idle;
 * bf16 dense at d <= 32 takes four on rows of 256+ keys staged whole at
 * large batches), 1 = one tile per wave, 2 = two tiles per wave. Results are identical either
 * way, bit for bit; only the time differs (it lets a small test batch run the
 * instantiation a large batch uses). Process-wide, atomic. Returns the
 * previous mode, or -1 (and sets the last error) for an invalid mode. No
 * counterpart in the reference.
 */
#define TARMAC_TILES_AUTO 0
#define TARMAC_TILES_ONE 1
#define TARMAC_TILES_TWO 2
int tarmac_set_query_tiles(int mode);

/* Writes 1.0f to *out: the launch-floor probe of scripts/launch_overhead.py:28-30. */
int tarmac_noop(float* out, void* stream);

/*
 * Diagnostic: chains `chain` bf16 MFMA instructions from +0 per tile and
 * stores the fp32 results, so a test can measure the MFMA's fp32 accumulation
 * error against exact sums -- the quantity the bf16 and split-bf16 top-k
 * proofs bound (see tarmac_set_topk_filter). shape 16:
 * v_mfma_f32_16x16x32_bf16; a, b: bf16 [tiles][chain][64 lanes][8] in the
 * instruction's operand layout (lane l: A row l % 16, columns 8 (l / 16) ..
 * +7; B column l % 16, rows 8 (l / 16) .. +7); out: fp32 [tiles][64 lanes][4]
 * (lane l, element r: row 4 (l / 16) + r, column l % 16). shape 32:
 * v_mfma_f32_32x32x16_bf16; a, b as above with l % 32 and l / 32 (A row
 * l % 32, columns 8 (l / 32) .. +7; B column l % 32, rows 8 (l / 32) .. +7);
 * out: fp32 [tiles][64 lanes][16] (lane l, element i: row 8 (i / 4) +
 * 4 (l / 32) + i % 4, column l % 32). 16-byte aligned; 1 <= chain <= 64.
 * No counterpart in the reference.
 */
int tarmac_mfma_bf16_probe(const void* a, const void* b, float* out, int tiles, int chain,
                           int shape, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TARMAC_H_ */
