// capi.cpp -- C ABI (include/maxsim_hip.h): resident corpus handles,
// input validation with the reference's messages, device workspaces and
// kernel orchestration.  Handle semantics follow CudaInt4PackedDocs
// (cuda_extension.cu:2677-3306) and CudaPackedDocs (cu:1872-2675).
#include "capi_handles.hpp"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace msim {

thread_local std::string g_last_error;
int g_docs_per_wave = 0;
int g_fused_topk = 1;  // msim_set_fused_topk
int g_scan_partition = 0;  // msim_set_scan_partition
int g_scan_prefix = 1;     // msim_set_prefix_scan
int g_hamming_fp4 = 1;     // msim_set_hamming_fp4
uint64_t g_fused_wait_ticks = kScanTailWaitTicks;  // msim_set_fused_wait_ticks

void set_error(const std::string& msg) { g_last_error = msg; }

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) throw RuntimeError(std::string(what) + ": " + hipGetErrorString(e));
}

DeviceBuffer::~DeviceBuffer() {
  if (ptr) (void)hipFree(ptr);
}

void DeviceBuffer::ensure(size_t bytes, const char* what) {
  if (bytes <= cap) return;
  void* next = nullptr;
  check_hip(hipMalloc(&next, bytes), what);
  if (ptr) (void)hipFree(ptr);
  ptr = next;
  cap = bytes;
}

HostBuffer::~HostBuffer() {
  if (ptr) (void)hipHostFree(ptr);
}

void HostBuffer::ensure(size_t bytes, const char* what) {
  if (bytes <= cap) return;
  void* next = nullptr;
  check_hip(hipHostMalloc(&next, bytes, hipHostMallocCoherent), what);
  if (ptr) (void)hipHostFree(ptr);
  ptr = next;
  cap = bytes;
}

void DeviceBuffer::reset() {
  if (ptr) (void)hipFree(ptr);
  ptr = nullptr;
  cap = 0;
}

void validate_offsets(const int64_t* offsets, int64_t count, int64_t num_tokens) {
  if (offsets == nullptr || count < 2) throw InvalidArgument("offsets must contain at least [0, num_doc_tokens]");
  if (offsets[0] != 0) throw InvalidArgument("offsets must start at 0");
  if (offsets[count - 1] != num_tokens) throw InvalidArgument("offsets must end at num_doc_tokens");
  for (int64_t i = 1; i < count; ++i)
    if (offsets[i] < offsets[i - 1]) throw InvalidArgument("offsets must be monotonically nondecreasing");
}

void validate_positive_scales(const float* v, int64_t n, const char* msg) {
  for (int64_t i = 0; i < n; ++i)
    if (!(v[i] > 0.0f) || !std::isfinite(v[i])) throw InvalidArgument(msg);
}

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

int32_t docs_per_wave_for(int64_t num_docs, int waves_per_cu) {
  if (g_docs_per_wave > 0) return g_docs_per_wave;
  const int64_t target = (int64_t)device_cu_count() * waves_per_cu;
  int64_t dpw = (num_docs + target - 1) / target;
  return (int32_t)(dpw < 1 ? 1 : dpw);
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace msim

using namespace msim;

// ------------------------------------------------------------------ global

extern "C" const char* msim_last_error(void) { return g_last_error.c_str(); }

extern "C" int msim_abi_version(void) { return 100; }

extern "C" int msim_set_docs_per_wave(int value) {
  return guarded([&] {
    if (value < 0) throw InvalidArgument("docs per wave must be >= 0 (0 = automatic)");
    g_docs_per_wave = value;
  });
}

extern "C" int msim_get_docs_per_wave(void) { return g_docs_per_wave; }

extern "C" int msim_set_fused_topk(int mode) {
  return guarded([&] {
    if (mode < 0 || mode > 2) throw InvalidArgument("fused top-k mode must be 0, 1 or 2");
    g_fused_topk = mode;
  });
}

extern "C" int msim_get_fused_topk(void) { return g_fused_topk; }

extern "C" int msim_set_fused_wait_ticks(int64_t ticks) {
  return guarded([&] {
    if (ticks < 0) throw InvalidArgument("fused selection wait must be >= 0 ticks");
    g_fused_wait_ticks = (uint64_t)ticks;
  });
}

extern "C" int64_t msim_get_fused_wait_ticks(void) { return (int64_t)g_fused_wait_ticks; }

extern "C" int msim_set_scan_partition(int mode) {
  return guarded([&] {
    if (mode < 0 || mode > 1) throw InvalidArgument("scan partition mode must be 0 or 1");
    g_scan_partition = mode;
  });
}

extern "C" int msim_get_scan_partition(void) { return g_scan_partition; }

extern "C" int msim_set_prefix_scan(int mode) {
  return guarded([&] {
    if (mode < 0 || mode > 1) throw InvalidArgument("prefix scan mode must be 0 or 1");
    g_scan_prefix = mode;
  });
}

extern "C" int msim_get_prefix_scan(void) { return g_scan_prefix; }

extern "C" int msim_set_hamming_fp4(int mode) {
  return guarded([&] {
    if (mode < 0 || mode > 1) throw InvalidArgument("hamming fp4 mode must be 0 or 1");
    g_hamming_fp4 = mode;
  });
}

extern "C" int msim_get_hamming_fp4(void) { return g_hamming_fp4; }

// -------------------------------------------------------------- int4 handle

namespace {

void select_device(int device) { check_hip(hipSetDevice(device), "hipSetDevice"); }

void check_query_dim(int64_t dim, int64_t expected) {
  if (dim != expected) throw InvalidArgument("query shape does not match dim");
}

void check_k(int64_t k, int64_t num_docs) {
  if (k < 1 || k > num_docs) throw InvalidArgument("k must be between 1 and num_docs");
  if (k > kTopkMaxK) throw NotSupported("k above 4096 is not supported by the device top-k selector");
}

void check_int8q(const msim_int4_docs* h) {
  if (h->dim != 128) throw InvalidArgument("int8 query scoring currently requires dim=128");
}

// Upload `count` floats times `factor` (a power of two: exact), followed by
// kScanPadTokens zeros (the scan's loads may read that far past the end).
void upload_scaled(DeviceBuffer& dst, const float* src, int64_t count, float factor, const char* what) {
  std::vector<float> scaled((size_t)(count + kScanPadTokens), 0.0f);
  for (int64_t i = 0; i < count; ++i) scaled[(size_t)i] = src[i] * factor;
  dst.ensure(scaled.size() * 4, what);
  check_hip(hipMemcpy(dst.ptr, scaled.data(), scaled.size() * 4, hipMemcpyHostToDevice), what);
}

// int4 rows of row_bytes bytes (dim / 2) widened to the generalized
// scorer's whole 128-dim chunks (64 bytes each) with zero nibbles, which add
// nothing to a dot product; nothing is kept when the rows already are whole
// chunks, or when dim is beyond what that scorer takes.
void upload_codes_wide(DeviceBuffer& dst, const uint8_t* src, int64_t num_tokens, int64_t row_bytes,
                       const char* what) {
  const int chunks = score_chunks(2 * row_bytes);
  const int64_t width = 64 * (int64_t)chunks;
  if (chunks == 0 || row_bytes == width) {
    dst.reset();
    return;
  }
  std::vector<uint8_t> wide((size_t)(std::max<int64_t>(num_tokens, 1) * width), 0);
  for (int64_t t = 0; t < num_tokens; ++t) std::memcpy(&wide[t * width], src + t * row_bytes, (size_t)row_bytes);
  dst.ensure(wide.size(), what);
  check_hip(hipMemcpy(dst.ptr, wide.data(), wide.size(), hipMemcpyHostToDevice), what);
}

// Quantise d_query [B,Q,128] into the handle's query workspace.
void quantize_int8q(msim_int4_docs* h, const float* d_query, int64_t batch, int64_t query_tokens,
                    hipStream_t stream) {
  const int64_t rows = batch * query_tokens;
  h->quantized_rows = -1;
  if (rows == 0) return;
  // Kernels read whole 16-row query tiles, up to 128 rows from a pass's
  // first row; pad (with zero rows) so those reads stay in bounds.
  const int64_t rows_padded = ((rows + 15) / 16) * 16 + 128;
  // The scan (query_tokens <= 128) reads the codes in lane order, one region
  // per pass; the row-pass kernel in row order.
  const int64_t pass_rows = query_tokens <= 128 ? scan_pass_rows(query_tokens) : 0;
  h->qpack.ensure(std::max<int64_t>(rows_padded * 128, scan_qpack_bytes(rows, pass_rows)), "hipMalloc int8q query codes");
  h->qscale.ensure(rows_padded * 4, "hipMalloc int8q query scales");
  h->qbias.ensure(rows_padded * 4, "hipMalloc int8q query bias");
  check_hip(launch_quantize_int8(d_query, rows, rows_padded, h->qpack.as<int8_t>(),
                                 h->qscale.as<float>(), h->qbias.as<int32_t>(), stream, pass_rows),
            "launch int8 query quantize kernel");
  h->quantized_rows = rows;
}

// Score the quantised query in the workspace against every document: d_out [B, N].
void score_int8q(msim_int4_docs* h, int64_t batch, int64_t query_tokens, float* d_out,
                 hipStream_t stream) {
  const int64_t rows = batch * query_tokens;
  if (rows == 0 || h->num_docs == 0) {
    if (batch > 0 && h->num_docs > 0)
      check_hip(launch_fill_f32(d_out, batch * h->num_docs, 0.0f, stream), "zero scores");
    return;
  }
  if (h->quantized_rows != rows)
    throw InvalidArgument("no quantised query of this shape: call quantize first with the same batch and query_tokens");
  int8_t* qpack = h->qpack.as<int8_t>();
  float* qscale = h->qscale.as<float>();
  int32_t* qbias = h->qbias.as<int32_t>();

  Int8qArgs a{};
  a.codes = h->packed.as<uint8_t>();
  a.token_scale = h->has_token_scale ? h->token_scales.as<float>() : nullptr;
  a.offsets = h->offsets.as<int64_t>();
  a.num_tokens = h->num_tokens;
  a.num_docs = h->num_docs;
  a.docs_per_wave = docs_per_wave_for(h->num_docs, 8);
  a.query_tokens = (int32_t)query_tokens;
  a.scale = h->scale;
  a.out_stride = h->num_docs;
  if (query_tokens <= 128) {
    const int64_t per_pass = 128 / query_tokens;
    for (int64_t b0 = 0; b0 < batch; b0 += per_pass) {
      const int64_t nb = std::min(per_pass, batch - b0);
      a.qpack = qpack + b0 * query_tokens * 128;
      a.qscale = qscale + b0 * query_tokens;
      a.qbias = qbias + b0 * query_tokens;
      a.batch = (int32_t)nb;
      a.out = d_out + b0 * h->num_docs;
      a.rowmax_out = nullptr;
      a.rows_valid = (int32_t)(nb * query_tokens);
      check_hip(launch_int8q_maxsim(a, (int)(nb * query_tokens), h->has_token_scale, true, stream),
                "launch int4 int8q maxsim kernel");
    }
  } else {
    h->rowmax.ensure(sizeof(float) * rows * h->num_docs, "hipMalloc int8q row maxima");
    float* rowmax = h->rowmax.as<float>();
    for (int64_t r0 = 0; r0 < rows; r0 += 128) {
      const int64_t nr = std::min<int64_t>(128, rows - r0);
      a.qpack = qpack + r0 * 128;
      a.qscale = qscale + r0;
      a.qbias = qbias + r0;
      a.batch = 0;
      a.out = nullptr;
      a.rowmax_out = rowmax + r0 * h->num_docs;
      a.rows_valid = (int32_t)nr;
      check_hip(launch_int8q_maxsim(a, (int)nr, h->has_token_scale, false, stream),
                "launch int4 int8q maxsim kernel");
    }
    check_hip(launch_int8q_finish(rowmax, qscale, batch, query_tokens, h->num_docs, h->scale,
                                  h->offsets.as<int64_t>(), d_out, stream),
              "launch int8q finish kernel");
  }
}

}  // namespace

namespace msim {

// Scan tables of the handle for the requested wave count (cached).
void build_wave_info(msim_int4_docs* h, int64_t waves) {
  if (h->partition_waves == waves && h->partition_mode == g_scan_partition) return;
  std::vector<int64_t> info;
  std::vector<uint64_t> tiles;
  build_scan_tables(h->host_offsets.data(), h->num_docs, waves, g_scan_partition == 1, info, tiles, h->tile_stride,
                    h->num_scan_waves);
  h->block_pos_off = (int64_t)info.size() - (h->num_scan_waves / kScanWavesPerGroup + 1);
  h->wave_info.ensure(sizeof(int64_t) * std::max<size_t>(1, info.size()), "hipMalloc scan wave table");
  if (!info.empty())
    check_hip(hipMemcpy(h->wave_info.ptr, info.data(), sizeof(int64_t) * info.size(), hipMemcpyHostToDevice),
              "copy scan wave table to device");
  h->tile_table.ensure(sizeof(uint64_t) * std::max<size_t>(1, tiles.size()), "hipMalloc scan tile table");
  if (!tiles.empty())
    check_hip(hipMemcpy(h->tile_table.ptr, tiles.data(), sizeof(uint64_t) * tiles.size(), hipMemcpyHostToDevice),
              "copy scan tile table to device");
  h->partition_waves = waves;
  h->partition_mode = g_scan_partition;
}

int64_t scan_waves(const msim_int4_docs* h) {
  // Default: eight waves per CU (two per SIMD); a docs-per-wave override sets
  // the count directly.
  int64_t waves = g_docs_per_wave > 0 ? (h->num_docs + g_docs_per_wave - 1) / g_docs_per_wave
                                      : (int64_t)device_cu_count() * kScanWavesPerCu;
  return std::max<int64_t>(1, std::min<int64_t>(waves, h->num_docs));
}

int scan_epilogue(const msim_int4_docs* h) {
  if (!h->has_token_scale) return kScanEpiIntMax;
  return h->token_scales_fma ? kScanEpiFma : kScanEpiCvt;
}

bool scan_tables_current(const msim_int4_docs* h) {
  return h->partition_waves == scan_waves(h) && h->partition_mode == g_scan_partition;
}

void scan_corpus_args(const msim_int4_docs* h, int64_t query_tokens, ScanArgs& a) {
  a.codes = h->packed.as<uint8_t>();
  const int epi = scan_epilogue(h);
  a.token_scale16 = epi == kScanEpiIntMax ? nullptr
                    : (epi == kScanEpiFma ? h->token_scales16.as<float>() : h->token_scales.as<float>());
  a.offsets = h->offsets.as<int64_t>();
  a.wave_info = h->wave_info.as<int64_t>();
  a.tile_table = h->tile_table.as<uint64_t>();
  a.tile_stride = h->tile_stride;
  a.num_waves = h->num_scan_waves;
  a.query_tokens = (int32_t)query_tokens;
  a.scale = h->scale;
  a.score_stride = h->num_docs;
  a.num_docs = h->num_docs;
  a.block_pos = h->wave_info.as<int64_t>() + h->block_pos_off;
}

}  // namespace msim

namespace {

// The scan selects the top-k itself (last-workgroup tail) when every pass's
// batch rows, the corpus and the scan's workgroup count fit the tail's
// limits (builds the scan tables if needed).
bool scan_fuses_topk(msim_int4_docs* h, int64_t batch, int64_t query_tokens, int64_t k) {
  if (g_fused_topk == 0 || k <= 0 || query_tokens == 0 || query_tokens > 128 || h->num_docs == 0) return false;
  const int64_t per_pass = std::max<int64_t>(1, kScanPassRows / query_tokens);
  if (!(k <= msim::kScanTailMaxK && h->num_docs >= msim::kScanTailMinDocs && h->num_docs <= msim::kScanTailMaxDocs &&
        std::min(per_pass, batch) <= msim::kScanTailMaxRows))
    return false;
  build_wave_info(h, scan_waves(h));
  return h->num_scan_waves <= (int64_t)kScanWavesPerGroup * kScanTailBlocks;
}

// Scores of the quantised query against every document into d_scores [B, N];
// with k > 0 (scan_fuses_topk true) the scores go to the handle's padded
// tail rows instead (d_scores unused) and the top-k of each batch row to
// d_top_s / d_top_i [B, k].
void score_quantized(msim_int4_docs* h, int64_t batch, int64_t query_tokens, float* d_scores,
                     hipStream_t stream, int64_t k = 0, float* d_top_s = nullptr, int64_t* d_top_i = nullptr) {
  if (query_tokens == 0 || h->num_docs == 0 || query_tokens > 128) {
    score_int8q(h, batch, query_tokens, d_scores, stream);
    return;
  }
  if (h->quantized_rows != batch * query_tokens)
    throw InvalidArgument("no quantised query of this shape: call quantize first with the same batch and query_tokens");
  build_wave_info(h, scan_waves(h));
  ScanArgs a{};
  scan_corpus_args(h, query_tokens, a);
  if (k > 0) {
    // Fill kernels, not memsets, so that a captured call records no memset
    // node; they run once per allocation: the launch counter starts at 0 and
    // the key rows and workgroup records hold no tag of a later launch.
    if (h->tail_epoch.ptr == nullptr) {
      h->tail_epoch.ensure(256, "hipMalloc scan launch counter");
      check_hip(launch_fill_f32(h->tail_epoch.as<float>(), 64, 0.0f, stream), "zero scan launch counters");
    }
    const int64_t rows = std::min(batch, std::max<int64_t>(1, kScanPassRows / query_tokens));
    const size_t key_bytes = sizeof(uint64_t) * (size_t)(rows * kScanTailRow);
    const size_t rec_bytes = sizeof(uint64_t) * (size_t)(rows * 3 * kScanTailBlocks);
    if (h->tail_keys.cap < key_bytes) {
      h->tail_keys.ensure(key_bytes, "hipMalloc scan tail key rows");
      check_hip(launch_fill_f32(h->tail_keys.as<float>(), (int64_t)(key_bytes / 4), 0.0f, stream), "zero scan tail key rows");
    }
    if (h->tail_rec.cap < rec_bytes) {
      h->tail_rec.ensure(rec_bytes, "hipMalloc scan tail workgroup records");
      check_hip(launch_fill_f32(h->tail_rec.as<float>(), (int64_t)(rec_bytes / 4), 0.0f, stream),
                "zero scan tail workgroup records");
    }
    a.tail_keys = h->tail_keys.as<uint64_t>();
    a.tail_rec = h->tail_rec.as<uint64_t>();
    a.tail_key_words = (int64_t)(h->tail_keys.cap / sizeof(uint64_t));
    a.topk_k = (int32_t)k;
    a.tail_cap = g_fused_topk == 2 ? 0 : INT32_MAX;
    a.epoch = h->tail_epoch.as<uint32_t>();
    a.tail_wait_ticks = g_fused_wait_ticks;
  }
  const int64_t per_pass = std::max<int64_t>(1, kScanPassRows / query_tokens);
  for (int64_t b0 = 0; b0 < batch; b0 += per_pass) {
    const int64_t nb = std::min(per_pass, batch - b0);
    a.qpack = h->qpack.as<int8_t>() + (b0 / per_pass) * scan_qpack_bytes(per_pass * query_tokens, per_pass * query_tokens);
    a.qscale = h->qscale.as<float>() + b0 * query_tokens;
    a.batch = (int32_t)nb;
    a.scores = k > 0 ? nullptr : d_scores + b0 * a.score_stride;
    if (k > 0) {
      a.top_scores = d_top_s + b0 * k;
      a.top_ids = d_top_i + b0 * k;
    }
    check_hip(launch_int8q_scan(a, scan_epilogue(h), stream), "launch int8q scan kernel");
  }
}

// Full int8-query search: scores of every document into d_scores [B, N] and,
// when k > 0, the top-k of each batch row into d_top_s / d_top_i [B, k].
// Quantisation and the scan are launches on one stream; the selection is the
// scan's tail when it fits (scan_fuses_topk), else a launch of its own.
void select_quantized(msim_int4_docs* h, int64_t batch, int64_t query_tokens, float* d_scores, int64_t k,
                      float* d_top_s, int64_t* d_top_i, hipStream_t stream);

void search_int8q(msim_int4_docs* h, const float* d_query, int64_t batch, int64_t query_tokens,
                  float* d_scores, int64_t k, float* d_top_s, int64_t* d_top_i, hipStream_t stream) {
  if (batch == 0) return;
  quantize_int8q(h, d_query, batch, query_tokens, stream);
  select_quantized(h, batch, query_tokens, d_scores, k, d_top_s, d_top_i, stream);
}

// Scores (and with k > 0 the top-k) of the last quantised query.
void select_quantized(msim_int4_docs* h, int64_t batch, int64_t query_tokens, float* d_scores, int64_t k,
                      float* d_top_s, int64_t* d_top_i, hipStream_t stream) {
  if (scan_fuses_topk(h, batch, query_tokens, k)) {
    score_quantized(h, batch, query_tokens, d_scores, stream, k, d_top_s, d_top_i);
    return;
  }
  score_quantized(h, batch, query_tokens, d_scores, stream);
  if (k > 0)
    check_hip(launch_topk(d_scores, batch, h->num_docs, h->num_docs, k, nullptr, d_top_s, d_top_i, stream),
              "launch int8q topk selection kernel");
}

void run_int8q(msim_int4_docs* h, const float* d_query, int64_t batch, int64_t query_tokens,
               float* d_out, hipStream_t stream) {
  search_int8q(h, d_query, batch, query_tokens, d_out, 0, nullptr, nullptr, stream);
}

// A fused selection that gave up (its wait for the other workgroups ran out)
// left id -1 in its row: a synchronous call reports it instead of returning it.
void require_selected(const int64_t* ids, int64_t count) {
  for (int64_t i = 0; i < count; ++i)
    if (ids[i] < 0)
      throw RuntimeError(
          "int8q top-k: the fused selection gave up waiting for the scan's workgroups (device stalled or "
          "oversubscribed); no result was returned");
}

float* ensure_scores(msim_int4_docs* h, int64_t batch, int64_t targets) {
  h->scores.ensure(sizeof(float) * std::max<int64_t>(1, batch * targets), "hipMalloc score cache");
  return h->scores.as<float>();
}

}  // namespace

extern "C" int msim_int4_create(const uint8_t* packed, int64_t num_tokens, int64_t row_bytes,
                                const int64_t* offsets, int64_t num_offsets, int dim, double scale,
                                msim_int4_docs** out) {
  return guarded([&] {
    if (out == nullptr) throw InvalidArgument("out handle pointer must not be NULL");
    *out = nullptr;
    if (dim <= 0 || dim % 2 != 0) throw InvalidArgument("dim must be positive and divisible by 2");
    if (row_bytes != dim / 2) throw InvalidArgument("packed shape does not match dim");
    if (num_tokens < 0) throw InvalidArgument("packed must have shape [num_doc_tokens, dim / 2]");
    if (num_offsets < 2) throw InvalidArgument("offsets must contain at least [0, num_doc_tokens]");
    if (!(scale > 0.0) || !std::isfinite(scale)) throw InvalidArgument("scale must be finite and > 0");
    validate_offsets(offsets, num_offsets, num_tokens);
    if (num_tokens > 0 && packed == nullptr) throw InvalidArgument("packed must not be NULL");
    auto h = std::make_unique<msim_int4_docs>();
    check_hip(hipGetDevice(&h->device), "hipGetDevice");
    h->dim = dim;
    h->num_docs = num_offsets - 1;
    h->num_tokens = num_tokens;
    h->scale = scale;
    h->packed_size = (uint64_t)num_tokens * (uint64_t)row_bytes;
    h->offsets_size = (uint64_t)num_offsets;
    h->host_offsets.assign(offsets, offsets + num_offsets);
    for (int64_t d = 0; d + 1 < num_offsets; ++d)
      h->max_doc_tiles = std::max<int64_t>(h->max_doc_tiles, (offsets[d + 1] - offsets[d] + 15) / 16);
    // kScanPadTokens zero tokens follow the corpus (the scan's loads may read
    // that far past the end).
    const uint64_t pad_bytes = (uint64_t)kScanPadTokens * (uint64_t)row_bytes;
    h->packed.ensure(std::max<uint64_t>(h->packed_size + pad_bytes, 64), "hipMalloc int4 packed docs");
    h->offsets.ensure(h->offsets_size * 8, "hipMalloc int4 offsets");
    if (h->packed_size)
      check_hip(hipMemcpy(h->packed.ptr, packed, h->packed_size, hipMemcpyHostToDevice), "copy int4 packed docs to device");
    check_hip(hipMemset(h->packed.as<uint8_t>() + h->packed_size, 0, pad_bytes), "zero int4 packed docs padding");
    check_hip(hipMemcpy(h->offsets.ptr, offsets, h->offsets_size * 8, hipMemcpyHostToDevice), "copy int4 offsets to device");
    upload_codes_wide(h->codes_wide, packed, num_tokens, row_bytes, "int4 packed docs (whole 128-dim chunks)");
    // The int8-query scan's tables, built here so that the first search (and
    // msim_int4_topk_int8q_noalloc) finds them resident.
    if (dim == 128 && h->num_docs > 0) build_wave_info(h.get(), scan_waves(h.get()));
    *out = h.release();
  });
}

extern "C" int msim_int4_destroy(msim_int4_docs* h) {
  return guarded([&] {
    if (h == nullptr) return;
    (void)hipSetDevice(h->device);
    delete h;
  });
}

extern "C" int msim_int4_set_token_scale(msim_int4_docs* h, const float* token_scales, int64_t count) {
  return guarded([&] {
    require_handle(h);
    if (count != h->num_tokens) throw InvalidArgument("token scale vector must have shape [num_doc_tokens]");
    validate_positive_scales(token_scales, count, "token scales must be finite and > 0");
    select_device(h->device);
    upload_scaled(h->token_scales, token_scales, count, 1.0f, "int4 token scale vector");
    // The MFMA kernels multiply 16 * dot by s / 16 (a power-of-two rescale,
    // exact for normal floats).
    upload_scaled(h->token_scales16, token_scales, count, 0.0625f, "int4 token scale vector / 16");
    h->token_scales_fma = std::all_of(token_scales, token_scales + count,
                                      [](float v) { return v >= kScanFmaMinScale && v < kScanFmaMaxScale; });
    h->has_token_scale = true;
  });
}

extern "C" int msim_int4_clear_token_scale(msim_int4_docs* h) {
  return guarded([&] {
    require_handle(h);
    h->has_token_scale = false;
  });
}

extern "C" int msim_int4_set_residual(msim_int4_docs* h, const uint8_t* packed, int64_t num_tokens,
                                      int64_t row_bytes, double scale, const float* token_scales,
                                      int64_t count) {
  return guarded([&] {
    require_handle(h);
    if (num_tokens != h->num_tokens || row_bytes != h->dim / 2)
      throw InvalidArgument("residual packed data must have shape [num_doc_tokens, dim / 2]");
    if (!(scale > 0.0) || !std::isfinite(scale)) throw InvalidArgument("residual scale must be finite and > 0");
    if (count != h->num_tokens) throw InvalidArgument("residual token scale vector must have shape [num_doc_tokens]");
    validate_positive_scales(token_scales, count, "residual token scales must be finite and > 0");
    select_device(h->device);
    const size_t pbytes = (size_t)num_tokens * (size_t)row_bytes;
    h->residual_packed.ensure(std::max<size_t>(pbytes, 64), "hipMalloc resident int4 residual data");
    if (pbytes) check_hip(hipMemcpy(h->residual_packed.ptr, packed, pbytes, hipMemcpyHostToDevice), "copy int4 residual data to device");
    upload_codes_wide(h->residual_wide, packed, num_tokens, row_bytes, "int4 residual data");
    upload_scaled(h->residual_token_scales16, token_scales, count, 0.0625f, "int4 residual token scales");
    h->residual_scale = scale;
    h->has_residual = true;
  });
}

extern "C" int msim_int4_clear_residual(msim_int4_docs* h) {
  return guarded([&] {
    require_handle(h);
    h->has_residual = false;
  });
}

extern "C" int msim_int4_get_props(const msim_int4_docs* h, msim_int4_props* out) {
  return guarded([&] {
    require_handle(h);
    if (out == nullptr) throw InvalidArgument("props pointer must not be NULL");
    out->dim = h->dim;
    out->num_docs = h->num_docs;
    out->num_tokens = h->num_tokens;
    out->scale = h->scale;
    out->residual_scale = h->residual_scale;
    out->packed_size = h->packed_size;
    out->has_token_scale_vector = h->has_token_scale ? 1 : 0;
    out->token_scale_vector_size = h->has_token_scale ? (uint64_t)h->num_tokens : 0;
    out->has_residual_int4 = h->has_residual ? 1 : 0;
    out->resident_bytes = h->resident_bytes();
    out->workspace_bytes = h->workspace_bytes();
  });
}

extern "C" int msim_int4_maxsim_batch_int8q(msim_int4_docs* h, const float* query, int64_t batch,
                                            int64_t query_tokens, int64_t dim, float* out) {
  return guarded([&] {
    require_handle(h);
    check_int8q(h);
    check_query_dim(dim, h->dim);
    require_shape(batch, query_tokens);
    if (batch == 0 || h->num_docs == 0) return;
    select_device(h->device);
    hipStream_t stream = nullptr;
    // The query and the score rows pass through the handle's pinned buffer:
    // the quantisation kernel reads the query there, and the scores come
    // back by one DMA copy into it.
    const size_t qbytes = sizeof(float) * (size_t)(batch * query_tokens * dim);
    const size_t obytes = sizeof(float) * (size_t)(batch * h->num_docs);
    const size_t q_al = (qbytes + 255) & ~(size_t)255;
    h->host_io.ensure(q_al + obytes, "hipHostMalloc int8q query and score staging");
    char* io = h->host_io.as<char>();
    std::memcpy(io, query, qbytes);
    float* d_scores = ensure_scores(h, batch, h->num_docs);
    run_int8q(h, reinterpret_cast<const float*>(io), batch, query_tokens, d_scores, stream);
    check_hip(hipMemcpyAsync(io + q_al, d_scores, obytes, hipMemcpyDeviceToHost, stream), "copy int8q output to host");
    check_hip(hipStreamSynchronize(stream), "synchronize int4 int8q maxsim");
    std::memcpy(out, io + q_al, obytes);
  });
}

extern "C" int msim_int4_topk_batch_int8q(msim_int4_docs* h, const float* query, int64_t batch,
                                          int64_t query_tokens, int64_t dim, int64_t k,
                                          float* out_scores, int64_t* out_indices) {
  return guarded([&] {
    require_handle(h);
    check_k(k, h->num_docs);
    check_int8q(h);
    check_query_dim(dim, h->dim);
    require_shape(batch, query_tokens);
    if (batch == 0) return;
    select_device(h->device);
    hipStream_t stream = nullptr;
    // The query, the top scores and the top ids share one pinned buffer: the
    // quantisation kernel reads the query from it and the selection writes
    // its results into it.
    const size_t qbytes = sizeof(float) * (size_t)(batch * query_tokens * dim);
    const size_t sbytes = sizeof(float) * (size_t)(batch * k), ibytes = sizeof(int64_t) * (size_t)(batch * k);
    const size_t q_al = (qbytes + 255) & ~(size_t)255, s_al = (sbytes + 255) & ~(size_t)255;
    h->host_io.ensure(q_al + s_al + ibytes, "hipHostMalloc int8q query and result staging");
    char* io = h->host_io.as<char>();
    std::memcpy(io, query, qbytes);
    float* h_top_s = reinterpret_cast<float*>(io + q_al);
    int64_t* h_top_i = reinterpret_cast<int64_t*>(io + q_al + s_al);
    float* d_scores = ensure_scores(h, batch, h->num_docs);
    search_int8q(h, reinterpret_cast<const float*>(io), batch, query_tokens, d_scores, k, h_top_s, h_top_i, stream);
    check_hip(hipStreamSynchronize(stream), "synchronize int8q topk kernels");
    require_selected(h_top_i, batch * k);
    std::memcpy(out_scores, h_top_s, sbytes);
    std::memcpy(out_indices, h_top_i, ibytes);
  });
}

extern "C" int msim_int4_fused_giveups(const msim_int4_docs* h, uint64_t* out) {
  return guarded([&] {
    require_handle(h);
    if (out == nullptr) throw InvalidArgument("out pointer must not be NULL");
    *out = 0;
    if (h->tail_epoch.ptr == nullptr) return;
    select_device(h->device);
    uint32_t words[2] = {0, 0};
    check_hip(hipDeviceSynchronize(), "synchronize before reading the fused selection counters");
    check_hip(hipMemcpy(words, h->tail_epoch.ptr, sizeof(words), hipMemcpyDeviceToHost),
              "copy fused selection counters to host");
    *out = words[1];
  });
}

extern "C" int msim_int4_maxsim_int8q_async(msim_int4_docs* h, const float* d_query, int64_t batch,
                                            int64_t query_tokens, float* d_out, void* stream) {
  return guarded([&] {
    require_handle(h);
    check_int8q(h);
    require_shape(batch, query_tokens);
    if (batch == 0 || h->num_docs == 0) return;
    select_device(h->device);
    run_int8q(h, d_query, batch, query_tokens, d_out, as_stream(stream));
  });
}

extern "C" int msim_int4_topk_int8q_async(msim_int4_docs* h, const float* d_query, int64_t batch,
                                          int64_t query_tokens, int64_t k, float* d_scores,
                                          int64_t* d_indices, void* stream) {
  return guarded([&] {
    require_handle(h);
    check_k(k, h->num_docs);
    check_int8q(h);
    require_shape(batch, query_tokens);
    if (batch == 0) return;
    select_device(h->device);
    float* d_full = ensure_scores(h, batch, h->num_docs);
    search_int8q(h, d_query, batch, query_tokens, d_full, k, d_scores, d_indices, as_stream(stream));
  });
}

extern "C" int msim_int4_quantize_int8q_async(msim_int4_docs* h, const float* d_query, int64_t batch,
                                              int64_t query_tokens, void* stream) {
  return guarded([&] {
    require_handle(h);
    check_int8q(h);
    require_shape(batch, query_tokens);
    select_device(h->device);
    quantize_int8q(h, d_query, batch, query_tokens, as_stream(stream));
  });
}

extern "C" int msim_int4_score_int8q_async(msim_int4_docs* h, int64_t batch, int64_t query_tokens,
                                           float* d_out, void* stream) {
  return guarded([&] {
    require_handle(h);
    check_int8q(h);
    require_shape(batch, query_tokens);
    if (batch == 0 || h->num_docs == 0) return;
    select_device(h->device);
    score_quantized(h, batch, query_tokens, d_out, as_stream(stream));
  });
}

extern "C" int msim_int4_topk_quantized_async(msim_int4_docs* h, int64_t batch, int64_t query_tokens, int64_t k,
                                              float* d_scores, int64_t* d_indices, void* stream) {
  return guarded([&] {
    require_handle(h);
    check_k(k, h->num_docs);
    check_int8q(h);
    require_shape(batch, query_tokens);
    if (batch == 0) return;
    if (h->quantized_rows != batch * query_tokens)
      throw InvalidArgument("no quantised query of this shape: call quantize first with the same batch and query_tokens");
    select_device(h->device);
    float* d_full = ensure_scores(h, batch, h->num_docs);
    select_quantized(h, batch, query_tokens, d_full, k, d_scores, d_indices, as_stream(stream));
  });
}

extern "C" int msim_topk_async(const float* d_scores, int64_t batch, int64_t n, int64_t row_stride,
                               int64_t k, float* d_out_scores, int64_t* d_out_indices, void* stream) {
  return guarded([&] {
    if (batch < 0 || n < 0) throw InvalidArgument("scores must have shape [batch, n]");
    if (row_stride < n) throw InvalidArgument("row_stride must be >= n");
    check_k(k, n);
    if (batch == 0) return;
    check_hip(launch_topk(d_scores, batch, n, row_stride, k, nullptr, d_out_scores, d_out_indices,
                          as_stream(stream)),
              "launch topk selection kernel");
  });
}
