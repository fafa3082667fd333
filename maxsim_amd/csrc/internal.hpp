// internal.hpp -- launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

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

// Full-corpus scan over pre-quantised query rows (int8q_scan.hip).  Each wave
// owns a contiguous range of at most kScanMaxDocsPerWave documents, described
// by kWaveInfoWords int64 words:
//   [0] d0          first document
//   [1] ndocs       documents [d0, d0 + ndocs)
//   [2] T0, [3] T1  token range of the wave (offsets[d0], offsets[d0 + ndocs]),
//                   with (T1 - T0) * 64 < 2^32
//   [4] ntiles      sum over documents of ceil(len / 16)
//   [5] n_ne        non-empty documents
//   [6] tab0        index of the wave's first entry in the document table
//   [7] end of the first non-empty document relative to T0 (low 32 bits),
//       1 << 32 if the wave has empty documents
// The document table holds, per non-empty document in order, (end - T0) in
// the low 32 bits and the document's index relative to d0 in the high bits.
constexpr int kWaveInfoWords = 8;
constexpr int kScanMaxDocsPerWave = 63;
// Ring depth of the scan (tiles in flight per wave) and the per-wave ring
// table: the first kScanPrefetch tile starts (relative to T0; kScanPastEnd
// past the last tile), then the load cursor after them: document index,
// next tile start, end of that document.
#ifndef MSIM_SCAN_PREFETCH
#define MSIM_SCAN_PREFETCH 8
#endif
constexpr int kScanPrefetch = MSIM_SCAN_PREFETCH;
constexpr int kScanRingWords = kScanPrefetch + 3;
constexpr uint32_t kScanPastEnd = 0x3FFFFF0u;  // (kScanPastEnd + 15) * 64 + 48 < 2^32
struct ScanArgs {
  const uint8_t* codes;       // [num_tokens, 64] int4 nibbles
  const float* token_scale;   // [num_tokens] or nullptr (tensor scale)
  const int64_t* offsets;     // [num_docs + 1]
  const int64_t* wave_info;   // [num_waves, kWaveInfoWords]
  const uint64_t* doc_table;  // per-wave non-empty document ends
  const uint32_t* ring_starts; // [num_waves, kScanRingWords]
  int64_t num_waves;
  const int8_t* qpack;        // >= 16 * ceil(rows / 16) rows of MFMA B-order int8 codes
  const float* qscale;        // per-row query scale, same row count
  int32_t batch;              // batch rows of this pass (batch * query_tokens <= 128)
  int32_t query_tokens;
  double scale;               // tensor scale (1.0 for per-token corpora)
  float* scores;              // [batch, score_stride]
  int64_t score_stride;
};
// Builds the wave table and document table for `waves` requested waves
// (the result may hold more rows: ranges are split at kScanMaxDocsPerWave
// documents and at 2^25 tokens).
void build_scan_tables(const int64_t* offsets, int64_t num_docs, int64_t waves,
                       std::vector<int64_t>& wave_info, std::vector<uint64_t>& doc_table,
                       std::vector<uint32_t>& ring_starts);
hipError_t launch_int8q_scan(const ScanArgs& args, bool token_scale, hipStream_t stream);

// Block top-k (topk.hip): per row b of scores[b * row_stride + i], i < n, the k
// largest by (score desc, position asc).  id_map (nullable, [batch, n]) maps a
// position to the reported id.
constexpr int kTopkMaxK = 4096;
hipError_t launch_topk(const float* d_scores, int64_t batch, int64_t n, int64_t row_stride,
                       int64_t k, const int64_t* d_id_map, float* d_out_scores,
                       int64_t* d_out_ids, hipStream_t stream);

}  // namespace msim
