/*
 * maxsim_hip.h -- C ABI of the MI355X (gfx950) MaxSim scoring engine.
 *
 * Drop-in boundary for the reference's native handle module
 * `maxsim._maxsim_cuda` (pybind11 module cpp/maxsim/cuda_extension.cu:3416-3514).
 * Every entry point below replaces one method, property or routing knob of
 * that module; the comment on each cites the reference line it replaces.
 * Plain C types only: host pointers, device pointers, sizes, and an opaque
 * HIP stream passed as void*.  No torch, no pybind, no CUDA headers.
 *
 * Errors: every function returns MSIM_OK or an error code and records a
 * message readable with msim_last_error() on the calling thread.
 * MSIM_EINVAL corresponds to the reference's std::invalid_argument
 * (Python ValueError); MSIM_ERUNTIME to check_cuda failures (RuntimeError).
 * A call that fails validation leaves the handle unchanged.
 *
 * Host-buffer methods (`const float* query` host pointers) are synchronous
 * like the reference: they copy the query in, run, and copy results out.
 * The *_async variants take device pointers and a stream and only enqueue.
 * Handles are not thread-safe (the reference's per-handle workspaces are
 * not either); use one handle per thread or serialise calls.
 */
#ifndef MAXSIM_HIP_H
#define MAXSIM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSIM_OK 0
#define MSIM_EINVAL 1
#define MSIM_ERUNTIME 2
#define MSIM_ENOTSUP 3

/* Message of the last failed call on this thread ("" if none). */
const char* msim_last_error(void);
/* ABI version (major * 100 + minor). */
int msim_abi_version(void);

/* Routing knobs: documents scored per wave by the streaming kernels
 * (0 = automatic from the device's CU count).  Replaces the reference's
 * launch-shape knobs set_shared_reducer_warps / set_residual_reducer_warps
 * (cuda_extension.cu:3489-3513), whose SM89 warp shapes have no gfx950 meaning. */
int msim_set_docs_per_wave(int value);
int msim_get_docs_per_wave(void);
/* Top-k selection of the int8-query search: 1 (default) = the scan's
 * workgroup 0 selects, once the other workgroups' results have arrived, when
 * the call fits (k <= 32, 256..4096 documents, <= 8 batch rows per scan
 * pass), 0 = always a separate selection launch, 2 = fused with the
 * selection's k-round path forced (tests both paths).
 * No counterpart in the reference, which selects on the host
 * (cuda_extension.cu:1629-1692 returns full score rows). */
int msim_set_fused_topk(int mode);
int msim_get_fused_topk(void);
/* How long the fused selection waits for the other workgroups' results, in
 * ticks of the GPU's 100 MHz real-time counter (default 10,000,000 = 100 ms;
 * the wait normally ends within microseconds).  A selection whose wait runs
 * out gives up: it writes id -1 and a NaN score into every slot of its batch
 * row and adds one to the handle's give-up counter (msim_int4_fused_giveups).
 * 0 makes every fused selection give up before reading anything (for tests of
 * that path).  No counterpart in the reference. */
int msim_set_fused_wait_ticks(int64_t ticks);
int64_t msim_get_fused_wait_ticks(void);
/* Prefix (sign) pass of the binary-prefix + int4-residual cascade
 * (msim_binary_cascade_topk*): 1 (default) = the int8-query scan kernel
 * over the sign stream when it applies (query rows of <= 128 tokens, token
 * scales in [2^-122, 2^109)), 0 = the generalized scorer (tests both).  No
 * counterpart in the reference, which has no such format. */
int msim_set_prefix_scan(int mode);
int msim_get_prefix_scan(void);
/* Sign-query (Hamming) scoring of binary handles (msim_binary_hamming_batch,
 * msim_binary_topk_hamming*): 1 (default) = the fp4 kernel (one
 * v_mfma_scale_f32_16x16x128_f8f6f4 on +-1 fp4 operands per 16 tokens x 16
 * query rows x 128 dims, 256 query rows per pass), 0 = the int8 MFMA scorer
 * (tests both; results identical).  No counterpart in the reference. */
int msim_set_hamming_fp4(int mode);
int msim_get_hamming_fp4(void);
/* Work split of the int8-query scan: 0 (default) = documents to waves
 * longest first, each to the least-loaded wave (whole corpus addressed from
 * one base; up to 2^25 tokens and 2^24 documents, beyond that as 1);
 * 1 = contiguous document ranges balanced by cost.  Results are identical.
 * No counterpart in the reference (its kernels take one block per document). */
int msim_set_scan_partition(int mode);
int msim_get_scan_partition(void);

/* Symmetric int4 packing on the device: pack_int4_symmetric
 * (experimental.py:218-268) with codes in _pack_signed_int4_values' nibble
 * order (experimental.py:604-609), bit-identical to the host packer.
 * token_granularity 1 = "token" (per-token scales into token_scales[T]),
 * 0 = "tensor"; scale 0 means None (tensor: max|x| / 7).  values [T, dim]
 * int8 is optional (NULL).  The reference's argument checks and messages.
 *
 * Host arrays in and out (uploads, packs, downloads; *scale_out receives the
 * tensor scale, 1.0 for token granularity): */
int msim_pack_int4(const float* x, int64_t num_tokens, int dim, int token_granularity, double scale,
                   uint8_t* codes, float* token_scales, int8_t* values, double* scale_out);
/* Device arrays (x 16-byte aligned), enqueued on `stream`; work = 2 device
 * words: work[0] receives max|x| bits (tensor granularity), work[1] != 0 when
 * x holds a non-finite value (the caller checks it after the stream). */
int msim_pack_int4_async(const float* d_x, int64_t num_tokens, int dim, int token_granularity, double scale,
                         uint8_t* d_codes, float* d_token_scales, int8_t* d_values, uint32_t* d_work,
                         void* stream);

/* ===================================================================== */
/* Int4 corpus handle: CudaInt4PackedDocs (cuda_extension.cu:2677-3306). */
/* ===================================================================== */
typedef struct msim_int4_docs msim_int4_docs;

/* CudaInt4PackedDocs.__init__(packed u8[T, dim/2], offsets i64[N+1], dim, scale)
 * (cu:2679-2728).  Copies codes and offsets to the current device. */
int msim_int4_create(const uint8_t* packed, int64_t num_tokens, int64_t row_bytes,
                     const int64_t* offsets, int64_t num_offsets, int dim, double scale,
                     msim_int4_docs** out);
/* Destructor (cu:2733-2747). */
int msim_int4_destroy(msim_int4_docs* h);
/* set_token_scale_vector(f32[T]) (cu:2749-2773). */
int msim_int4_set_token_scale(msim_int4_docs* h, const float* token_scales, int64_t count);
/* clear_token_scale_vector() (cu:2775). */
int msim_int4_clear_token_scale(msim_int4_docs* h);
/* set_residual_int4(u8[T, dim/2], scale, f32[T]) (cu:2777-2831). */
int msim_int4_set_residual(msim_int4_docs* h, const uint8_t* packed, int64_t num_tokens,
                           int64_t row_bytes, double scale, const float* token_scales,
                           int64_t count);
/* clear_residual_int4() (cu:2833). */
int msim_int4_clear_residual(msim_int4_docs* h);

/* Read-only properties dim, num_docs, num_tokens, scale, packed_size,
 * has_token_scale_vector, token_scale_vector_size, has_residual_int4,
 * resident_bytes, workspace_bytes (cu:3035-3055, 3496-3505). */
typedef struct msim_int4_props {
  int64_t dim;
  int64_t num_docs;
  int64_t num_tokens;
  double scale;
  double residual_scale;
  uint64_t packed_size;
  int64_t has_token_scale_vector;
  uint64_t token_scale_vector_size;
  int64_t has_residual_int4;
  uint64_t resident_bytes;
  uint64_t workspace_bytes;
} msim_int4_props;
int msim_int4_get_props(const msim_int4_docs* h, msim_int4_props* out);

/* maxsim_batch_int8q(query f32[B,Q,128]) -> f32[B,N] (cu:2993-3006).
 * out: host [B, N]. */
int msim_int4_maxsim_batch_int8q(msim_int4_docs* h, const float* query, int64_t batch,
                                 int64_t query_tokens, int64_t dim, float* out);
/* topk_batch_int8q(query, k) -> (f32[B,k], i64[B,k]) (cu:3008-3033).
 * Fails with MSIM_ERUNTIME if the fused selection gave up (see
 * msim_set_fused_wait_ticks): it never returns id -1. */
int msim_int4_topk_batch_int8q(msim_int4_docs* h, const float* query, int64_t batch,
                               int64_t query_tokens, int64_t dim, int64_t k,
                               float* out_scores, int64_t* out_indices);
/* Device-resident forms of the two calls above: d_query, d_out, d_scores,
 * d_indices are device pointers; work is enqueued on `stream` (a
 * hipStream_t, NULL = default stream) and not waited for.  Every *_async
 * entry point may allocate its workspaces (hipMalloc) and upload tables on
 * the first call with a given shape; a call under HIP graph capture needs an
 * earlier call with the same shapes (or msim_int4_topk_int8q_noalloc). */
int msim_int4_maxsim_int8q_async(msim_int4_docs* h, const float* d_query, int64_t batch,
                                 int64_t query_tokens, float* d_out, void* stream);
int msim_int4_topk_int8q_async(msim_int4_docs* h, const float* d_query, int64_t batch,
                               int64_t query_tokens, int64_t k, float* d_scores,
                               int64_t* d_indices, void* stream);
/* Sentinel of the *_async and _noalloc top-k calls of the int8-query path:
 * a batch row whose fused selection gave up holds id -1 and a NaN score in
 * every slot (see msim_set_fused_wait_ticks); callers that read results
 * without a synchronous call check d_indices for -1.  The number of
 * selections that gave up on this handle so far (noalloc calls are not
 * counted here): waits for the device, then reads it.  No counterpart in the
 * reference. */
int msim_int4_fused_giveups(const msim_int4_docs* h, uint64_t* out);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): msim_int4_topk_int8q_async with the same arguments and
 * results, whose scratch memory (quantised query, score rows, the fused
 * selection's key rows, workgroup records and launch counter) is a fixed
 * 526,592-byte device array per GPU instead of
 * handle workspaces, so the call allocates nothing.  Limits: 1 <= batch *
 * query_tokens <= 128, k <= 32, and either the fused selection applies
 * (256 <= num_docs <= 4096, batch <= 8, msim_set_fused_topk mode 1 or 2) or
 * batch * num_docs <= 32768; other sizes fail with MSIM_EINVAL.  The handle's
 * scan tables are built by msim_int4_create; after msim_set_docs_per_wave or
 * msim_set_scan_partition changes, one msim_int4_topk_int8q_async call must
 * rebuild them first.  The first call on a device looks the array up
 * (make it outside graph capture).  All calls on one GPU share the array:
 * calls that overlap on one GPU race.  A row whose fused selection gave up
 * holds the id -1 / NaN sentinel described above. */
int msim_int4_topk_int8q_noalloc(msim_int4_docs* h, const float* d_query, int64_t batch,
                                 int64_t query_tokens, int64_t k, float* d_scores,
                                 int64_t* d_indices, void* stream);

/* Stage-level device entry points of the int8-query path (no reference
 * counterpart; the reference fuses them inside launch_int8q_maxsim,
 * cu:3237-3271): quantise a device query into the handle's workspace, score
 * the last quantised query, and select top-k on device scores.  The score
 * call must use the batch/query_tokens of the preceding quantise call. */
int msim_int4_quantize_int8q_async(msim_int4_docs* h, const float* d_query, int64_t batch,
                                   int64_t query_tokens, void* stream);
int msim_int4_score_int8q_async(msim_int4_docs* h, int64_t batch, int64_t query_tokens,
                                float* d_out, void* stream);
/* Top-k [batch, k] of the last quantised query: the scan with its fused
 * selection when the call fits (see msim_set_fused_topk), else the scan and a
 * selection launch; the second half of msim_int4_topk_int8q_async. */
int msim_int4_topk_quantized_async(msim_int4_docs* h, int64_t batch, int64_t query_tokens, int64_t k,
                                   float* d_scores, int64_t* d_indices, void* stream);
/* Top-k of device score rows d_scores[b * row_stride + i], i < n, ordered by
 * (score desc, position asc); the block selector of topk_kernel (cu:1629-1692). */
int msim_topk_async(const float* d_scores, int64_t batch, int64_t n, int64_t row_stride,
                    int64_t k, float* d_out_scores, int64_t* d_out_indices, void* stream);

/* maxsim_batch(query f32[B,Q,dim]) -> f32[B,N], fp32-query MaxSim
 * (cu:2835-2858, kernel cu:1268-1323). */
int msim_int4_maxsim_batch(msim_int4_docs* h, const float* query, int64_t batch,
                           int64_t query_tokens, int64_t dim, float* out);
/* topk_batch(query, k) (cu:2957-2991). */
int msim_int4_topk_batch(msim_int4_docs* h, const float* query, int64_t batch,
                         int64_t query_tokens, int64_t dim, int64_t k, float* out_scores,
                         int64_t* out_indices);

/* score_batch / score_candidates_batch / score_residual_batch /
 * score_residual_candidates_batch (cu:2860-2955, score_impl cu:3124-3206).
 * reducer: "maxsim" | "weighted_maxsim" | "topk2" | "topk4" | "smoothsim".
 * weights: NULL or f32 of shape [weights_dim0] (weights_ndim 1) or
 * [weights_dim0, weights_dim1] (weights_ndim 2), as upload_reducer_weights
 * (cu:3080-3122) accepts.  candidates: NULL (all docs) or i64[num_candidates]
 * shared by every batch row, output in caller order.  residual != 0 scores
 * the fused prefix+residual similarity.  out: host [B, targets]. */
int msim_int4_score(msim_int4_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                    int64_t dim, const char* reducer, const float* weights, int64_t weights_ndim,
                    int64_t weights_dim0, int64_t weights_dim1, double temperature,
                    const int64_t* candidates, int64_t num_candidates, int residual, float* out);

/* Top-k of msim_int4_score over every document, selected on the device
 * (the reference selects non-MaxSim reducers on the host,
 * experimental.py:523-535). */
int msim_int4_topk_score(msim_int4_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                         int64_t dim, int64_t k, const char* reducer, const float* weights,
                         int64_t weights_ndim, int64_t weights_dim0, int64_t weights_dim1,
                         double temperature, int residual, float* out_scores, int64_t* out_indices);

/* Device-resident form of msim_int4_score over every document (dim 128):
 * d_query f32 [B, Q, 128] and d_out f32 [B, N] on the device; weights as
 * msim_int4_score (host memory, read during the call); enqueued on
 * `stream`. */
int msim_int4_score_async(msim_int4_docs* h, const float* d_query, int64_t batch,
                          int64_t query_tokens, const char* reducer, const float* weights,
                          int64_t weights_ndim, int64_t weights_dim0, int64_t weights_dim1,
                          double temperature, int residual, float* d_out, void* stream);

/* cascade_topk(query, packed, k, candidates=M, reducer, query_weights,
 * temperature) of a residual int4 corpus (cascade.py:294-393): prefix scores
 * of every document, the top-M per batch row (score desc, id asc), fused
 * prefix+residual scores of those M, top-k with ties by document id
 * (cascade.py:436-453).  M == num_docs scores every document fused
 * (cascade.py:342-351).  The reference selects and loops over batch rows on
 * the host; here every stage stays on the device. */
int msim_int4_cascade_topk(msim_int4_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                           int64_t dim, int64_t k, int64_t candidates, const char* reducer,
                           const float* weights, int64_t weights_ndim, int64_t weights_dim0,
                           int64_t weights_dim1, double temperature, float* out_scores,
                           int64_t* out_indices);

/* ===================================================================== */
/* Binary corpus handle: CudaPackedDocs (cuda_extension.cu:1872-2675).    */
/* ===================================================================== */
typedef struct msim_binary_docs msim_binary_docs;

/* CudaPackedDocs.__init__(packed u8[T, dim/8], offsets i64[N+1], dim) (cu:1874-1917). */
int msim_binary_create(const uint8_t* packed, int64_t num_tokens, int64_t row_bytes,
                       const int64_t* offsets, int64_t num_offsets, int dim,
                       msim_binary_docs** out);
int msim_binary_destroy(msim_binary_docs* h);
/* set_scale_vector(f32[N]) / clear_scale_vector() (cu:1943-1956). */
int msim_binary_set_scale_vector(msim_binary_docs* h, const float* scale, int64_t count);
int msim_binary_clear_scale_vector(msim_binary_docs* h);
/* set_token_scale_vector(f32[T]) / clear_token_scale_vector() (cu:1958-1973). */
int msim_binary_set_token_scale(msim_binary_docs* h, const float* token_scales, int64_t count);
int msim_binary_clear_token_scale(msim_binary_docs* h);

typedef struct msim_binary_props {
  int64_t dim;
  int64_t num_docs;
  int64_t num_tokens;
  uint64_t packed_size;
  int64_t has_scale_vector;
  uint64_t scale_vector_size;
  int64_t has_token_scale_vector;
  uint64_t token_scale_vector_size;
  uint64_t resident_bytes;
  uint64_t workspace_bytes;
} msim_binary_props;
/* Properties (cu:2331-2347, 3437-3447). */
int msim_binary_get_props(const msim_binary_docs* h, msim_binary_props* out);

/* maxsim_batch(query f32[B,Q,dim], scale, use_scale_vector, use_token_scale)
 * (cu:1975-2003): fp32 query x sign bits. out host [B, N]. */
int msim_binary_maxsim_batch(msim_binary_docs* h, const float* query, int64_t batch,
                             int64_t query_tokens, int64_t dim, double scale,
                             int use_scale_vector, int use_token_scale, float* out);
/* topk_batch / topk_lut_batch (cu:2069-2109, 2165-2211). */
int msim_binary_topk_batch(msim_binary_docs* h, const float* query, int64_t batch,
                           int64_t query_tokens, int64_t dim, int64_t k, double scale,
                           int use_scale_vector, int use_token_scale, float* out_scores,
                           int64_t* out_indices);
/* maxsim_batch_int8q / topk_batch_int8q (cu:2213-2268): the query is
 * quantised per row to int8 as q * (1 / sigma) (cu:1328-1366) and scored as
 * 2 (q8 . bits) - sum(q8) (cu:1368-1447); dim 128 only. */
int msim_binary_maxsim_batch_int8q(msim_binary_docs* h, const float* query, int64_t batch,
                                   int64_t query_tokens, int64_t dim, double scale,
                                   int use_scale_vector, int use_token_scale, float* out);
int msim_binary_topk_batch_int8q(msim_binary_docs* h, const float* query, int64_t batch,
                                 int64_t query_tokens, int64_t dim, int64_t k, double scale,
                                 int use_scale_vector, int use_token_scale, float* out_scores,
                                 int64_t* out_indices);
/* score_batch / score_candidates_batch with the generalized reducers
 * (cu:2005-2067, score_impl).  scale_vector_override: NULL or f32[N]. */
int msim_binary_score(msim_binary_docs* h, const float* query, int64_t batch,
                      int64_t query_tokens, int64_t dim, const char* reducer,
                      const float* weights, int64_t weights_ndim, int64_t weights_dim0,
                      int64_t weights_dim1, double temperature, double scale,
                      int use_scale_vector, int use_token_scale,
                      const float* scale_vector_override, const int64_t* candidates,
                      int64_t num_candidates, float* out);
/* Top-k of msim_binary_score over every document, selected on the device
 * (the reference selects non-MaxSim reducers on the host, _api.py:481-497). */
int msim_binary_topk_score(msim_binary_docs* h, const float* query, int64_t batch,
                           int64_t query_tokens, int64_t dim, int64_t k, const char* reducer,
                           const float* weights, int64_t weights_ndim, int64_t weights_dim0,
                           int64_t weights_dim1, double temperature, double scale,
                           int use_scale_vector, int use_token_scale,
                           const float* scale_vector_override, float* out_scores,
                           int64_t* out_indices);
/* Sign-binarised queries (XOR / popcount): qbits u8[B, Q, dim/8] in the
 * pack_signs bit order.  Scores are sum_q max_t (dim - 2 popcount(q ^ d)),
 * exactly what maxsim_batch returns for the +/-1 query (no reference kernel;
 * the reference routes integer queries through topk_lut_batch, cu:2165-2211). */
int msim_binary_hamming_batch(msim_binary_docs* h, const uint8_t* qbits, int64_t batch,
                              int64_t query_tokens, int64_t dim, int32_t* out);
int msim_binary_topk_hamming(msim_binary_docs* h, const uint8_t* qbits, int64_t batch,
                             int64_t query_tokens, int64_t dim, int64_t k, float* out_scores,
                             int64_t* out_indices);
int msim_binary_topk_hamming_async(msim_binary_docs* h, const uint8_t* d_qbits, int64_t batch,
                                   int64_t query_tokens, int64_t k, float* d_scores,
                                   int64_t* d_indices, void* stream);

/* ------------------------------------------------------------------- */
/* Binary prefix + int4 residual format (no reference function: the     */
/* reference ships int4 + int4 only, cascade.py:60-93).  Per token: sign  */
/* bits (the handle's codes), prefix scale a_t = mean|x_t| (the handle's  */
/* token scale vector) and a per-token int4 residual of x - a_t sign(x).  */
/* Queries are quantised to int8 per row as in maxsim_batch_int8q of the  */
/* int4 handle.  Coarse similarity a_t (q . sign_t); fused similarity     */
/* a_t (q . sign_t) + s^r_t r (q . v^r_t); MaxSim reduction.              */
/* ------------------------------------------------------------------- */
/* Residual stream: u8 [T, 64] int4 codes, scale, f32 [T] token scales
 * (as set_residual_int4 of the int4 handle, cu:2777-2831). */
int msim_binary_set_residual(msim_binary_docs* h, const uint8_t* packed, int64_t num_tokens,
                             int64_t row_bytes, double scale, const float* token_scales,
                             int64_t count);
int msim_binary_clear_residual(msim_binary_docs* h);
/* No counterpart in the reference (its format has no binary prefix).  Query
 * precision of the fused scoring (msim_binary_binres_score with fused = 1)
 * and of a cascade's rescoring pass: limbs 1 (default) = the int8 query
 * (v_mfma_i32_16x16x64_i8 on the int8 codes), 3 = the fp32 query as three
 * int8 limbs (resolves q to 2^-24 of max|q|).  The coarse pass keeps the int8
 * query.  Other values fail with MSIM_EINVAL. */
int msim_binary_set_rescore_limbs(msim_binary_docs* h, int limbs);
int msim_binary_get_rescore_limbs(const msim_binary_docs* h, int* limbs);
/* Coarse (fused = 0) or fused (fused = 1) scores; candidates NULL (every
 * document, out [B, N]) or i64 [B, num_candidates] per batch row (out
 * [B, num_candidates]). */
int msim_binary_binres_score(msim_binary_docs* h, const float* query, int64_t batch,
                             int64_t query_tokens, int64_t dim, int fused, const int64_t* candidates,
                             int64_t num_candidates, float* out);
/* No counterpart in the reference (its format has no binary prefix).  Top-k
 * of the fused scores of every document (score desc, id asc), selected on
 * the device: what a full search of this format returns, without the
 * [B, N] scores leaving the device.  out_scores f32 [B, k], out_indices
 * i64 [B, k]; 1 <= k <= num_docs. */
int msim_binary_binres_topk(msim_binary_docs* h, const float* query, int64_t batch,
                            int64_t query_tokens, int64_t dim, int64_t k, float* out_scores,
                            int64_t* out_indices);
/* Coarse top-M -> fused rescoring -> top-k, on the device (the cascade of
 * msim_int4_cascade_topk over this format). */
int msim_binary_cascade_topk(msim_binary_docs* h, const float* query, int64_t batch,
                             int64_t query_tokens, int64_t dim, int64_t k, int64_t candidates,
                             float* out_scores, int64_t* out_indices);
/* Device-resident form: d_query f32 [B, Q, 128], outputs [B, k]; enqueued on
 * `stream`. */
int msim_binary_cascade_topk_async(msim_binary_docs* h, const float* d_query, int64_t batch,
                                   int64_t query_tokens, int64_t k, int64_t candidates,
                                   float* d_scores, int64_t* d_indices, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MAXSIM_HIP_H */
