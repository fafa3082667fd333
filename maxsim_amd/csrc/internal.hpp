// internal.hpp -- launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace msim {

// Arguments of the int4 x int8-query scoring kernel (int8q.hip).
struct Int8qArgs {
  const uint8_t* codes;       // [num_tokens, 64] int4 nibbles
  const float* token_scale;   // [num_tokens] or nullptr
  const int64_t* offsets;     // [num_docs + 1]
  int64_t num_tokens;
  int64_t num_docs;
  int32_t docs_per_wave;
  const int8_t* qpack;        // [rows (+pad), 128] MFMA B-order int8 query rows of this pass
  const float* qscale;        // [rows] per-row query scale
  const int32_t* qbias;       // [rows] -8 * sum(q8)
  int32_t batch;              // batch rows finished by this pass
  int32_t query_tokens;
  double scale;               // tensor scale (1.0 for per-token corpora)
  float* out;                 // [batch, out_stride] scores of this pass
  int64_t out_stride;
  float* rowmax_out;          // per-row maxima when the pass does not finish
  int32_t rows_valid;
};

hipError_t launch_quantize_int8(const float* d_query, int64_t rows, int64_t rows_padded,
                                int8_t* d_qpack, float* d_qscale, int32_t* d_qbias,
                                hipStream_t stream);
hipError_t launch_int8q_maxsim(const Int8qArgs& args, int rows_in_pass, bool token_scale,
                               bool finish, hipStream_t stream);
hipError_t launch_int8q_finish(const float* d_rowmax, const float* d_qscale, int64_t batch,
                               int64_t query_tokens, int64_t num_docs, double scale,
                               const int64_t* d_offsets, float* d_out, hipStream_t stream);

// Arguments of the fused one-launch search (int8q_fused.hip): quantise, score
// every document, and (k > 0) select the top-k of each batch row.
constexpr int kFusedMaxK = 256;
struct FusedArgs {
  const uint8_t* codes;
  const float* token_scale;   // nullptr for tensor-scale corpora
  const int64_t* offsets;
  int64_t num_docs;
  const int64_t* wave_docs;   // [num_waves + 1] document range of each wave
  int64_t num_waves;
  const float* query;         // f32 [batch * query_tokens, 128] of this pass
  int32_t batch;
  int32_t query_tokens;
  double scale;
  float* scores;              // [batch, score_stride]
  int64_t score_stride;
  int32_t k;                  // 0: scores only
  float* top_scores;          // [batch, k]
  int64_t* top_ids;           // [batch, k]
  uint32_t* counter;          // zero before the launch; the last workgroup resets it
};
hipError_t launch_int8q_search(const FusedArgs& args, bool token_scale, hipStream_t stream);
// Waves per workgroup of the fused search kernel; the fused top-k tail needs
// num_docs <= kFusedTailMaxDocs.
int fused_waves_per_block();
constexpr int64_t kFusedTailMaxDocs = 4096;

// Block top-k (topk.hip): per row b of scores[b * row_stride + i], i < n, the k
// largest by (score desc, position asc).  id_map (nullable, [batch, n]) maps a
// position to the reported id.
constexpr int kTopkMaxK = 4096;
hipError_t launch_topk(const float* d_scores, int64_t batch, int64_t n, int64_t row_stride,
                       int64_t k, const int64_t* d_id_map, float* d_out_scores,
                       int64_t* d_out_ids, hipStream_t stream);

}  // namespace msim
