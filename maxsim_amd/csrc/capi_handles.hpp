// capi_handles.hpp -- the resident corpus handles behind the C ABI and the
// workspaces of the generalized scoring path (score.hip).
#pragma once

#include <vector>

#include "capi_internal.hpp"

namespace msim {

// Device workspaces of one handle's generalized scoring calls (grow
// monotonically, freed with the handle; cu:3057-3067).
struct ScoreWorkspace {
  DeviceBuffer qpack, colmul, qsum, weights, pooled, qbits;
  DeviceBuffer qpack_alt;  // the query also in the int4 layout (QueryInput::alt_int4)
  std::vector<float> weights_host;  // what `weights` holds (a repeated weight vector is not copied again)
  DeviceBuffer full_info, full_tiles;  // cached whole-corpus tables
  int64_t full_key = -1;               // wave count the cached tables were built for (units: -2 - workgroups)
  int64_t full_waves = 0;              // records in the cached table
  int64_t full_units = 0;              // records per workgroup (work-unit tables), else 0
  DeviceBuffer cand_ids, cand_info, cand_tiles;
  // cascade: coarse scores, top-M candidates (scores / ids), fine scores
  DeviceBuffer coarse, top_m_scores, top_m_ids, fine;
  // Synchronous calls: the fp32 query and the top-k results, in pinned host
  // memory that the kernels read and write directly.
  HostBuffer host_query, host_out;
  uint64_t bytes() const {
    return qpack.cap + qpack_alt.cap + colmul.cap + qsum.cap + weights.cap + pooled.cap + qbits.cap + full_info.cap +
           full_tiles.cap + cand_ids.cap + cand_info.cap + cand_tiles.cap + coarse.cap + top_m_scores.cap +
           top_m_ids.cap + fine.cap;
  }
};

// Which query the generalized path scores.
struct QueryInput {
  const float* d_query = nullptr;    // fp32 [rows, 128 chunks] (device or pinned host memory), or
  const uint8_t* d_qbits = nullptr;  // sign bits [rows, 16] (pack_signs order)
  int limbs = 3;                     // 3: fp32 split into int8 limbs, 1: int8
  bool recip = false;                // int8 rounding q * (1 / sigma) (binary int8q)
  bool quantized = false;            // the workspace already holds this query in this layout
  bool alt_int4 = false;             // also quantise into qpack_alt in the int4 layout
  bool from_alt = false;             // score the rows an earlier alt_int4 call left in qpack_alt
};

// The document streams and scales of one scoring call.
struct DocStreams {
  int doc = kDocInt4;
  bool residual = false;
  const uint8_t* codes = nullptr;
  const float* tscale = nullptr;
  float tmul = 1.0f;
  const uint8_t* rcodes = nullptr;
  const float* rtscale = nullptr;
  float rmul = 1.0f;
  const float* doc_scale = nullptr;
  float scale = 1.0f;
  bool unit_tscale = false;  // tscale is all ones
  int chunks = 1;            // 128-dim chunks per token (score_chunks(dim))
};

// Candidate targets: none (every document), one list shared by all batch
// rows, or one list of `count` per batch row.
struct Targets {
  const int64_t* host = nullptr;
  int64_t count = 0;
  bool per_row = false;
  // Candidate lists already on the device ([batch][count], per_row): tables
  // are written on the device; documents have at most max_doc_tiles tiles.
  const int64_t* device = nullptr;
  const int64_t* d_offsets = nullptr;
  int64_t max_doc_tiles = 1;
  bool tables_ready = false;  // the candidate tables are already in the workspace (select_topm wrote them)
};

// Wave layout of a per-row candidate rescoring pass (device targets): what
// run_generic_score uses, so that the candidate selector can write the
// tables for it.
struct CandidateLayout {
  int64_t waves = 0, per_wave = 0, cap = 0;
};
CandidateLayout candidate_layout(int64_t batch, int64_t query_tokens, int limbs, int64_t per_target,
                                 int64_t max_doc_tiles, int chunks = 1);

// Scores of `batch` x `query_tokens` query rows against the targets into
// d_out[b * out_stride + t] (and d_iout[b * targets + t] as int32 if set).
void run_generic_score(ScoreWorkspace& ws, const std::vector<int64_t>& host_offsets, int64_t num_tokens,
                       const DocStreams& s, const QueryInput& q, int reducer, float temperature,
                       int64_t batch, int64_t query_tokens, const float* h_row_weights, const Targets& t,
                       float* d_out, int64_t out_stride, int32_t* d_iout, hipStream_t stream);

}  // namespace msim

struct msim_int4_docs {
  int device = 0;
  int64_t dim = 0;
  int64_t num_docs = 0;
  int64_t num_tokens = 0;
  double scale = 1.0;
  double residual_scale = 1.0;
  uint64_t packed_size = 0;
  uint64_t offsets_size = 0;
  bool has_token_scale = false;
  bool token_scales_fma = false;  // every token scale in [kScanFmaMinScale, kScanFmaMaxScale)
  bool has_residual = false;
  int64_t quantized_rows = -1;  // rows of the query currently quantised in qpack
  int64_t max_doc_tiles = 1;    // 16-token tiles of the longest document
  std::vector<int64_t> host_offsets;
  int64_t partition_waves = 0;    // wave count the cached scan table was built for
  int partition_mode = 0;         // msim_set_scan_partition mode it was built with
  int64_t num_scan_waves = 0;     // rows of wave_info
  int64_t tile_stride = 0;        // tile-table entries per wave
  int64_t block_pos_off = 0;      // index of the workgroup start positions in wave_info
  msim::DeviceBuffer wave_info, tile_table;
  msim::DeviceBuffer packed, offsets, token_scales, token_scales16, residual_packed, residual_token_scales16;
  // Generalized path: codes widened to whole 128-dim chunks (64 bytes each)
  // when dim is not a multiple of 128, per-token 1/16 when the corpus has no
  // token scales.
  msim::DeviceBuffer codes_wide, residual_wide, ones16;
  // workspaces (grow monotonically, freed with the handle; cu:3057-3067)
  msim::DeviceBuffer qpack, qscale, qbias, scores, rowmax;
  msim::HostBuffer host_io;  // synchronous calls: query in, results out (pinned)
  // Scan with fused top-k: launch counter, key rows of kScanTailRow tagged
  // 64-bit keys and workgroup records (3 x kScanTailBlocks tagged words per row).
  msim::DeviceBuffer tail_epoch, tail_keys, tail_rec;
  msim::ScoreWorkspace ws;

  uint64_t resident_bytes() const {
    return packed_size + offsets_size * 8 + token_scales.cap + token_scales16.cap + residual_packed.cap +
           residual_token_scales16.cap + codes_wide.cap + residual_wide.cap + ones16.cap;
  }
  uint64_t workspace_bytes() const {
    return qpack.cap + qscale.cap + qbias.cap + scores.cap +
           rowmax.cap + wave_info.cap + tile_table.cap + tail_epoch.cap + tail_keys.cap + tail_rec.cap + ws.bytes();
  }
};

struct msim_binary_docs {
  int device = 0;
  int64_t dim = 0;
  int64_t num_docs = 0;
  int64_t num_tokens = 0;
  uint64_t packed_size = 0;
  bool has_scale_vector = false;
  bool has_token_scale = false;
  std::vector<int64_t> host_offsets;
  // codes padded to whole 128-dim chunks (16 bytes each) per token
  msim::DeviceBuffer packed, offsets, scale_vector, token_scales, ones, scale_override;
  // int4 residual stream of the binary-prefix + int4-residual format
  bool has_residual = false;
  double residual_scale = 1.0;
  int64_t max_doc_tiles = 1;  // 16-token tiles of the longest document
  msim::DeviceBuffer residual_packed, residual_token_scales16;
  // Query limbs of the fused (prefix + residual) scoring and of a cascade's
  // rescoring pass: 1 = the int8 query, 3 = the fp32 query (three int8 limbs).
  int rescore_limbs = 1;
  // The int8-query scan over the sign stream (a cascade's prefix pass): its
  // tables (cached by wave count) and whether every token scale suits its
  // one-fma epilogue ([kScanFmaMinScale, kScanFmaMaxScale)).
  bool token_scales_fma = false;
  int64_t scan_partition_waves = 0, num_scan_waves = 0, scan_tile_stride = 0;
  msim::DeviceBuffer scan_wave_info, scan_tile_table;
  msim::DeviceBuffer scores, iscores;
  msim::ScoreWorkspace ws;

  uint64_t resident_bytes() const {
    return packed.cap + offsets.cap + scale_vector.cap + token_scales.cap + ones.cap + residual_packed.cap +
           residual_token_scales16.cap;
  }
  uint64_t workspace_bytes() const {
    return scores.cap + iscores.cap + scale_override.cap + scan_wave_info.cap +
           scan_tile_table.cap + ws.bytes();
  }
};

namespace msim {
// int8-query scan tables of a handle (capi.cpp): build (cached by wave count
// and partition mode), the wave count the current settings ask for, whether
// the resident tables match it, and the corpus fields of ScanArgs.
void build_wave_info(msim_int4_docs* h, int64_t waves);
int64_t scan_waves(const msim_int4_docs* h);
bool scan_tables_current(const msim_int4_docs* h);
int scan_epilogue(const msim_int4_docs* h);
void scan_corpus_args(const msim_int4_docs* h, int64_t query_tokens, ScanArgs& a);
}  // namespace msim
