/*
 * maxsim_oracle.h -- CPU restatement of the reference MaxSim semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (maxsim_amd/, include/)
 * may include, link or call this library.  It is the checker used by tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py.
 *
 * Every function cites the reference file:line whose behaviour it restates.
 * Paths are relative to the reference checkout (Aryagm/maxsim).
 */
#ifndef MAXSIM_ORACLE_H
#define MAXSIM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* numpy add.reduce order for contiguous float64 / float32 vectors
 * (pairwise: <8 sequential, <=128 eight accumulators, else split). */
double orc_pairwise_sum_f64(const double* a, int64_t n);
float orc_pairwise_sum_f32(const float* a, int64_t n);

/* Per-token symmetric int4: src/maxsim/experimental.py:218-268 (token branch)
 * and _pack_signed_int4_values experimental.py:604-609. */
void orc_pack_int4_token(const float* x, int64_t num_tokens, int dim,
                         uint8_t* codes, int8_t* values, float* token_scale);
/* Tensor-scale symmetric int4: experimental.py:246-258.  Returns the double
 * scale (max|x|/7, 1.0 when all zero). */
double orc_pack_int4_tensor(const float* x, int64_t num_tokens, int dim,
                            uint8_t* codes, int8_t* values);
/* Nibble unpack: src/maxsim/sdk.py:1085-1093. */
void orc_unpack_int4(const uint8_t* codes, int64_t num_tokens, int dim, int8_t* values);
/* Sign bits, LSB-first, x >= 0 -> 1: src/maxsim/_api.py:34-77. */
void orc_pack_signs(const float* x, int64_t num_tokens, int dim, uint8_t* out);

/* Per-row symmetric int8 query: tests/test_int4_int8q.py:11-14. */
void orc_quantize_int8(const float* q, int64_t rows, int dim, int8_t* q8, float* qscale);

/* int4 x int8-query MaxSim: tests/test_int4_int8q.py:7-26
 * (= benchmarks/run_cuda_step1.py:1054-1078).  token_scale may be NULL. */
void orc_int4_int8q_scores(const int8_t* q8, const float* qscale, int64_t batch,
                           int64_t query_tokens, int dim, const int8_t* values,
                           const float* token_scale, double scale,
                           const int64_t* offsets, int64_t num_docs, float* out);
/* Raw integer dots q8[r] . values[t] for every (r, t): out[r * T + t]. */
void orc_int8_dots(const int8_t* q8, int64_t rows, int dim, const int8_t* values,
                   int64_t num_tokens, int32_t* out);

/* Reducers (src/maxsim/_api.py:19-20, 558-585). */
enum { ORC_MAXSIM = 0, ORC_WEIGHTED = 1, ORC_TOPK2 = 2, ORC_TOPK4 = 3, ORC_SMOOTHSIM = 4 };

/* fp32-query int4 scoring, CPU semantics of experimental.py:403-420:
 * docs = values * f32(scale) [* token_scale]; sims = q @ doc.T; reducer.
 * candidates may be NULL (all docs); weights is [batch, query_tokens] or NULL. */
void orc_int4_fp32_scores(const float* q, int64_t batch, int64_t query_tokens, int dim,
                          const int8_t* values, float scale, const float* token_scale,
                          const int64_t* offsets, int64_t num_docs,
                          const int64_t* candidates, int64_t num_candidates,
                          int reducer, const float* weights, float temperature, float* out);

/* Generic dense-token scoring with a reducer: docs are fp32 [T, dim]
 * (already reconstructed).  Used for binary and residual CPU semantics:
 * _api.py:396-420, cascade.py:272-291. */
void orc_dense_scores(const float* q, int64_t batch, int64_t query_tokens, int dim,
                      const float* docs, const int64_t* offsets, int64_t num_docs,
                      const int64_t* candidates, int64_t num_candidates,
                      int reducer, const float* weights, float temperature, float* out);

/* Binary LUT MaxSim of the reference CPU extension: cpp/maxsim/cpu_extension.cpp:59-126. */
void orc_binary_lut_maxsim(const float* q, int64_t query_tokens, int dim,
                           const uint8_t* codes, const int64_t* offsets,
                           int64_t num_docs, float scale, float* out);
/* Sign-binarised query x binary doc MaxSim: sum_q max_t (dim - 2 popcount(q ^ d)),
 * the exact value maxsim_lut returns for a +/-1 query (benchmarks/blog_baseline.py:65-75). */
void orc_binary_hamming_maxsim(const uint8_t* qbits, int64_t batch, int64_t query_tokens,
                               int dim, const uint8_t* codes, const int64_t* offsets,
                               int64_t num_docs, int32_t* out);

/* Stable top-k: order by (score desc, tie id asc), _api.py:732-735 and
 * cascade.py:436-453.  tie_ids NULL means the row position. */
void orc_topk(const float* scores, int64_t batch, int64_t n, int64_t k,
              const int64_t* tie_ids, float* out_scores, int64_t* out_indices);

/* Binary-prefix + int4-residual format (this build's config-5 format; the
 * reference ships only int4+int4, cascade.py:60-93).  Prefix a_t = mean|x_t|
 * (float64 pairwise / dim, to f32), signs as orc_pack_signs, residual
 * r = x - a_t * sign(x) packed per token as orc_pack_int4_token. */
void orc_pack_binary_residual(const float* x, int64_t num_tokens, int dim,
                              uint8_t* sign_codes, float* prefix_scale,
                              uint8_t* residual_codes, int8_t* residual_values,
                              float* residual_scale);
/* Coarse prefix score with an int8 query: sim = f32(a_t * dot(q8, sign_t)),
 * max over tokens, sum_q max * qscale in float64 pairwise order. */
void orc_binres_prefix_scores(const int8_t* q8, const float* qscale, int64_t batch,
                              int64_t query_tokens, int dim, const uint8_t* sign_codes,
                              const float* prefix_scale, const int64_t* offsets,
                              int64_t num_docs, float* out);
/* Fused score: sim = f32(f32(a_t * dotS) + f32(r_t * dotR)); same reduction.
 * candidates [batch, num_candidates] (per batch row) or NULL for all docs. */
void orc_binres_fused_scores(const int8_t* q8, const float* qscale, int64_t batch,
                             int64_t query_tokens, int dim, const uint8_t* sign_codes,
                             const float* prefix_scale, const int8_t* residual_values,
                             const float* residual_scale, const int64_t* offsets,
                             int64_t num_docs, const int64_t* candidates,
                             int64_t num_candidates, float* out);

#ifdef __cplusplus
}
#endif
#endif
