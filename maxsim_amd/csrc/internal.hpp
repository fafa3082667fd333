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

// Quantises rows x 128 fp32 query rows: qscale / qbias [rows_padded] (zero
// past rows) and the codes in the row-pass kernel's row order (pass_rows ==
// 0, rows_padded rows) or the scan's lane order (pass_rows > 0: per scan pass
// of pass_rows rows a region of ceil(pass_rows / 16) tiles of 2 KiB,
// scan_qpack_bytes in all).
hipError_t launch_quantize_int8(const float* d_query, int64_t rows, int64_t rows_padded,
                                int8_t* d_qpack, float* d_qscale, int32_t* d_qbias,
                                hipStream_t stream, int64_t pass_rows = 0);
int64_t scan_qpack_bytes(int64_t rows, int64_t pass_rows);
hipError_t launch_int8q_maxsim(const Int8qArgs& args, int rows_in_pass, bool token_scale,
                               bool finish, hipStream_t stream);
hipError_t launch_int8q_finish(const float* d_rowmax, const float* d_qscale, int64_t batch,
                               int64_t query_tokens, int64_t num_docs, double scale,
                               const int64_t* d_offsets, float* d_out, hipStream_t stream);

// Full-corpus scan over pre-quantised query rows (int8q_scan.hip).  Each wave
// scores a set of documents (scan_tables.cpp), described by kWaveInfoWords
// int64 words:
//   [0] d0          document base (0 when the wave's documents are scattered)
//   [1] ndocs       non-empty documents of the wave
//   [2] T0, [3] T1  token range the wave's tiles lie in, (T1 - T0) * 64 < 2^31
//   [4] ntiles      16-token tiles of the wave: sum over documents of ceil(len / 16)
//   [5] pos0        first position of the wave's documents in the fused
//                   selection's order (wave order: each wave's empty documents,
//                   then its other documents in tile order)
//   [6] nempty      empty documents the wave writes 0 for
//   [7] e0          their first entry in the empty-document list, which
//                   follows the num_waves rows in the same buffer
// The table is padded to whole workgroups with waves of no tiles.  Tile table
// entries (one per tile, then kScanPrefetch + 1 padding entries per wave):
// low 32 bits the tile's first token relative to T0 (0 for padding: the
// prefetch of a padding entry reads the wave's first tokens again), then
// (rows - 1) in bits 32..36, "last tile of its document" in bit 37 and the
// document's index relative to d0 in bits 40..63.  The kernel adds a tile's
// byte offset to its loads outside the buffer range check (soffset), so every
// address it forms must lie in the corpus buffers: they hold kScanPadTokens
// zero tokens past the last one, which covers the rows a tile of a document
// shorter than 16 tokens reads past its end.
constexpr int kWaveInfoWords = 8;
constexpr int kScanMaxDocsPerWave = 63;
constexpr int kScanWavesPerGroup = 4;
#ifndef MSIM_SCAN_PREFETCH
#define MSIM_SCAN_PREFETCH 8
#endif
constexpr int kScanPrefetch = MSIM_SCAN_PREFETCH;  // ring depth: tiles in flight per wave
constexpr int64_t kScanMinStride = 16;             // tile-table entries per wave at least
#ifndef MSIM_SCAN_WAVES_PER_CU
#define MSIM_SCAN_WAVES_PER_CU 8
#endif
constexpr int kScanWavesPerCu = MSIM_SCAN_WAVES_PER_CU;  // scan waves launched per CU
constexpr uint32_t kScanPadEntry = 0u;  // tile entry of a padding slot
constexpr int64_t kScanPadTokens = 16;  // zero tokens past the end of every corpus buffer the scan reads
struct ScanArgs {
  const uint8_t* codes;         // [num_tokens, 64] int4 nibbles
  const float* token_scale16;   // [num_tokens] token scales / 16 (kScanEpiFma), the token scales
                                //   themselves (kScanEpiCvt), or nullptr (tensor scale)
  const int64_t* offsets;       // [num_docs + 1]
  const int64_t* wave_info;     // [num_waves, kWaveInfoWords]
  const uint64_t* tile_table;   // per-wave tile entries, wave w's at w * tile_stride
  int64_t tile_stride;
  int64_t num_waves;            // a multiple of kScanWavesPerGroup
  const int8_t* qpack;          // >= rows + 128 rows of MFMA B-order int8 codes (zero past rows)
  int32_t q_row_order;          // qpack rows of 128 bytes (quantize_limbs) instead of the scan's lane order
  int32_t doc_sign;             // sign documents: codes 16 bytes per token (32 sign bits per lane group,
                                //   bit b = dim 32g + b), token_scale16 the per-token scales themselves,
                                //   qpack in the sign layout of quantize_limbs
  const int32_t* qsum;          // sign documents: per query row the sum of its int8 codes
  const float* qscale;          // per-row query scale, same row count
  int32_t batch;                // batch rows of this pass (batch * query_tokens <= 128)
  int32_t query_tokens;
  double scale;                 // tensor scale (1.0 for per-token corpora)
  float* scores;                // [batch, score_stride] (not used by a fused launch)
  int64_t score_stride;
  // Fused selection (topk_k > 0, kScanTailMinDocs <= num_docs <=
  // kScanTailMaxDocs, num_waves <= 4 * kScanTailBlocks): the launch's tag is
  // *epoch + 1; every document's score goes write-through, as a tagged 64-bit
  // selection key (tail_full_key), to its wave-order position of tail_keys
  // [batch, kScanTailRow]; every workgroup writes a tagged record per batch
  // row to tail_rec [batch, 3, kScanTailBlocks] (its two largest keys, the
  // third one's score key); workgroup 0 waits until its reads carry the tag,
  // selects the top-k of every batch row into top_scores / top_ids [batch,
  // topk_k] and stores the tag to *epoch (after a give-up of row 0, first
  // the dispatch's identity to epoch[2..5]: a workgroup of that dispatch
  // that starts later keeps the launch's tag).  tail_keys and tail_rec hold no
  // entry with a later launch's tag (zero them when allocated).  block_pos
  // [num_waves / 4 + 1] holds each workgroup's first position (then num_docs).
  // A selection that waits longer than tail_wait_ticks (s_memrealtime ticks,
  // 100 MHz; 0 = give up at once) writes id -1 / NaN to its batch row and adds
  // one to epoch[1].
  int32_t topk_k;
  int32_t tail_cap;             // 0 forces the selection's k-round path
  int64_t num_docs;
  uint32_t* epoch;              // [0]: launch counter, [1]: selections given up, [2..5]: give-up mark (zeroed)
  uint64_t tail_wait_ticks;
  float* top_scores;
  int64_t* top_ids;
  uint64_t* tail_keys;
  uint64_t* tail_rec;
  const int64_t* block_pos;
  int64_t tail_key_words;       // u64 words of the tail_keys allocation (>= batch * kScanTailRow)
};
constexpr int kScanTailMaxK = 32;
constexpr int64_t kScanTailMaxDocs = 4096;
constexpr int64_t kScanTailMinDocs = 256;  // every lane of the selecting wave holds a score
constexpr int64_t kScanTailRow = 4096;  // key positions per batch row of the fused selection
constexpr int kScanTailMaxRows = 8;  // batch rows of one pass (two per wave)
constexpr int kScanTailBlocks = 512;  // workgroups of a fused launch at most
constexpr uint64_t kScanTailWaitTicks = 10000000;  // default wait of the fused selection: 100 ms
// Launch tags repeat in the 19 tag bits of a key every kScanTailKeyPeriod
// launches of one launch counter (tag % period + 1): workgroup 0 of every
// launch whose tag is period - 1 modulo the period zeroes all tail_key_words
// after its selection, so a key that carries the current tag was stored by
// the current launch.  The device does it, so replays of a captured call,
// which the host does not see, are covered too.
constexpr uint64_t kScanTailKeyPeriod = (1u << 19) - 1u;
// Epilogue forms of the scan (the token scales decide which is exact):
//  * kScanEpiIntMax: tensor-scale corpora (token_scale16 == nullptr): integer
//    maximum of the dots, scaled at the document end;
//  * kScanEpiFma: every token scale s in [2^-122, 2^109): one fma per
//    element on accumulators offset by 2^23 (int8q_scan.hip);
//  * kScanEpiCvt: any other positive finite token scales: float(dot) * s
//    (token_scale16 then holds the scales themselves).
enum : int { kScanEpiIntMax = 0, kScanEpiFma = 1, kScanEpiCvt = 2 };
constexpr float kScanFmaMinScale = 0x1p-122f, kScanFmaMaxScale = 0x1p109f;
hipError_t launch_int8q_scan(const ScanArgs& args, int epilogue, hipStream_t stream);
// Query rows of one scan launch: whole batch rows, at most 128 rows (one
// batch row of more than 128 tokens goes to the row-pass kernel instead).
constexpr int64_t kScanPassRows = 128;
inline int64_t scan_pass_rows(int64_t query_tokens) {
  return query_tokens <= 0 ? 0 : (query_tokens >= kScanPassRows ? 1 : kScanPassRows / query_tokens) * query_tokens;
}
// Builds the wave table and tile table for `waves` requested waves (the
// result may hold more rows: ranges are split at kScanMaxDocsPerWave
// documents and 2^25 tokens, and padded to whole workgroups).  Each wave's
// tile entries start at wave * tile_stride.  wave_info ends with the
// empty-document list and then the num_waves / 4 + 1 workgroup start
// positions (block_pos of ScanArgs).
// `contiguous` forces contiguous document ranges (otherwise used only for
// corpora beyond 2^25 tokens or 2^24 documents).
void build_scan_tables(const int64_t* offsets, int64_t num_docs, int64_t waves, bool contiguous,
                       std::vector<int64_t>& wave_info, std::vector<uint64_t>& tile_table, int64_t& tile_stride,
                       int64_t& num_waves);

// Generalized scoring (score.hip): int4 or sign-bit documents, optional int4
// residual stream, 1 (int8) or 3 (fp32 split into int8 limbs) query limbs,
// reducers.  Targets are documents or candidate positions, walked from a
// host-built table (build_score_tables): per wave kScoreInfoWords int64
// words {target base, targets, tiles, first tile-table entry}, padded to
// whole workgroups; per tile one entry: bits 0..33 first token, 34..37
// rows - 1, 38 last tile of its target, 39 empty target (no tokens, token 0
// is read and masked), 40..63 target index relative to the wave's base;
// one padding entry (token 0) follows every wave's tiles.
constexpr uint64_t kTileStartMask = (uint64_t(1) << 34) - 1;
constexpr int kTileRowsShift = 34, kTileLastShift = 38, kTileEmptyShift = 39, kTileLocalShift = 40;
__host__ __device__ inline uint64_t score_tile_entry(int64_t start, int64_t rows, bool last, bool empty,
                                                     int64_t local) {
  return ((uint64_t)start & kTileStartMask) | ((uint64_t)(rows - 1) << kTileRowsShift) |
         ((uint64_t)last << kTileLastShift) | ((uint64_t)empty << kTileEmptyShift) |
         ((uint64_t)local << kTileLocalShift);
}
constexpr int kScoreInfoWords = 4;
enum : int { kDocInt4 = 0, kDocSign = 1 };
enum : int { kRedMax = 0, kRedTop2 = 1, kRedTop4 = 2, kRedLse = 3 };
struct ScoreArgs {
  const uint8_t* codes;        // int4 [T, 64 chunks] or sign bits [T, 16 chunks]
  const float* tscale;         // [T] per-token scale of `codes` (never null)
  float tmul;                  // constant factor of the `codes` similarity
  const uint8_t* rcodes;       // residual int4 codes [T, 64 chunks] (residual kernels)
  const float* rtscale;        // [T] residual per-token scale
  float rmul;
  const int64_t* wave_info;    // [groups][num_waves][kScoreInfoWords]
  const uint64_t* tiles;
  // Work units (row-block pipeline kernels, eight waves per workgroup): 0 =
  // wave w of a group takes record w of wave_info; n > 0 = workgroup x of a
  // group owns records [n x, n x + n) (num_waves = n x workgroups), taken by
  // its waves one after another from a counter in LDS; a record with no
  // tiles ends the workgroup's list.
  int32_t group_units;
  // Direct mode (wave_info / tiles unused): wave w of a group scores target w
  // (w < direct_count), the document targets[w] whose tokens are
  // [direct_offsets[doc], direct_offsets[doc + 1]).
  const int64_t* direct_offsets;
  int64_t direct_count;
  int64_t num_waves;           // per group, a multiple of 4
  int64_t info_grp_stride;     // int64 words between groups' wave tables (0 = shared)
  const int64_t* targets;      // document of each target, or nullptr (target = document)
  int64_t targets_grp_stride;  // entries between groups' target lists
  const int8_t* qpack;         // [limbs][rows_padded][128 chunks] B-operand order per 128-dim chunk
  int64_t rows_padded;
  const float* colmul;         // [rows_padded] per query row factor (sigma)
  const int32_t* qsum;         // [limbs][rows_padded] limb sums (sign documents)
  const float* weights;        // [rows_padded] weighted MaxSim factors or nullptr
  int32_t subs;                // passes per group (query rows / rows per pass)
  int32_t grp_rows;            // query rows per group
  const float* doc_scale;      // [num_docs] per-document scale or nullptr
  float scale;                 // document scale when doc_scale is null
  float temperature;
  float* pooled;               // pooled[g * pooled_grp_stride + target * grp_rows + row]
  int64_t pooled_grp_stride;
  // When every pass holds whole batch rows (rows per pass a multiple of
  // query_tokens, or one batch row per group), the kernel sums each batch
  // row itself: out[b * out_stride + target] (and iout as int32) instead of
  // `pooled`.
  float* out;
  int64_t out_stride;
  int32_t* iout;
  int64_t iout_stride;
  int32_t query_tokens;
  bool unit_tscale;            // tscale is all ones (sign documents): integer maximum
  int32_t chunks;              // 128-dim chunks per token and query row (1, 2 or 4)
  // Sign-bit queries [rows][16] (pack_signs order) scored against sign
  // documents by the fp4 Hamming kernel (launch_hamming); null otherwise.
  const uint8_t* qbits;
};
// Query rows per pass of the fp4 Hamming kernel (sixteen 16-row blocks).
constexpr int kHammingRowsPerPass = 256;
hipError_t launch_hamming(const ScoreArgs& a, hipStream_t stream);
// Dims above 128 are scored in 128-dim chunks whose MFMA dots accumulate in
// one int32 accumulator: 2 chunks up to 256 dims, 4 up to 512 (0: above).
// 512 is the limit of the three-limb combination 254 a1 + a2 in int32
// (|a| <= 128 * 127 * 512 < 2^23).
constexpr int64_t kScoreMaxDim = 512;
inline int score_chunks(int64_t dim) { return dim <= 128 ? 1 : dim <= 256 ? 2 : dim <= 512 ? 4 : 0; }
int score_rows_per_pass(int limbs, int64_t rows, int chunks = 1);
hipError_t launch_score(const ScoreArgs& a, int doc, bool residual, int limbs, int reducer, int64_t groups,
                        hipStream_t stream);
// Query rows of 128 * chunks floats (dims past the query's own zero).
hipError_t launch_quantize_limbs(const float* d_query, int64_t rows, int64_t rows_padded, int limbs, int layout,
                                 bool recip, int8_t* qpack, float* colmul, int32_t* qsum, hipStream_t stream,
                                 int layout2 = 0, int8_t* qpack2 = nullptr, int chunks = 1);
hipError_t launch_quantize_bits(const uint8_t* d_qbits, int64_t rows, int64_t rows_padded, int8_t* qpack,
                                float* colmul, int32_t* qsum, hipStream_t stream);
hipError_t launch_pool_sum(const float* pooled, int64_t batch, int64_t query_tokens, int64_t targets, int64_t bs,
                           int64_t ts, float* out, int64_t out_stride, int32_t* iout, hipStream_t stream);
// Tables for `num_targets` targets (targets == nullptr: every document) split
// over about `waves` waves, balanced by tiles + 1 per target.
void build_score_tables(const int64_t* offsets, const int64_t* targets, int64_t num_targets, int64_t waves,
                        std::vector<int64_t>& info, std::vector<uint64_t>& tiles);
// Work units of the row-block pipeline kernels (ScoreArgs::group_units): the
// targets balanced over `workgroups` lists (tiles + 1 per target, longest
// first onto the least-loaded list), each list cut into units of whole
// targets, longest first, every unit but the list's last of at least
// kScoreUnitMinTiles tiles; lists padded with empty records to the same
// count, which is returned.  Tile entries hold absolute target indices, so
// num_targets must be below 2^24 (kScoreMaxUnitTargets).
constexpr int64_t kScoreUnitMinTiles = 4;
constexpr int64_t kScoreMaxUnitTargets = int64_t(1) << 24;
int64_t build_score_units(const int64_t* offsets, const int64_t* targets, int64_t num_targets, int64_t workgroups,
                          std::vector<int64_t>& info, std::vector<uint64_t>& tiles);

// Cascade helpers (cascade.hip): tile tables of per-group candidate lists
// written on the device (groups x waves waves of at most per_wave
// candidates, cap table entries each), and an ascending sort of int64 rows
// of at most kSortMaxRow values.
constexpr int64_t kSortMaxRow = 4096;
hipError_t launch_candidate_tables(const int64_t* d_cands, int64_t m, int64_t groups, const int64_t* d_offsets,
                                   int64_t waves, int64_t per_wave, int64_t cap, int64_t* d_info,
                                   uint64_t* d_tiles, hipStream_t stream);
hipError_t launch_sort_rows(int64_t* d_rows, int64_t batch, int64_t n, hipStream_t stream);
// The m best of each row of n <= kSortMaxRow scores by (score desc,
// position asc), output as positions in ascending order [batch, m].
// With `tables` set, each row's block also writes the rescoring pass's
// candidate tables (the layout launch_candidate_tables writes, group = row).
struct CandidateTables {
  const int64_t* d_offsets = nullptr;
  int64_t waves = 0, per_wave = 0, cap = 0;
  int64_t* d_info = nullptr;
  uint64_t* d_tiles = nullptr;
};
hipError_t launch_select_topm(const float* d_scores, int64_t batch, int64_t n, int64_t stride, int64_t m,
                              int64_t* d_out, hipStream_t stream, const CandidateTables* tables = nullptr);

// Block top-k (topk.hip): per row b of scores[b * row_stride + i], i < n, the k
// largest by (score desc, position asc).  id_map (nullable, [batch, n]) maps a
// position to the reported id.
constexpr int kTopkMaxK = 4096;
hipError_t launch_topk(const float* d_scores, int64_t batch, int64_t n, int64_t row_stride,
                       int64_t k, const int64_t* d_id_map, float* d_out_scores,
                       int64_t* d_out_ids, hipStream_t stream);

}  // namespace msim
