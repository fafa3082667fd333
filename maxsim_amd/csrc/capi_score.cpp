// capi_score.cpp -- C ABI of the generalized scoring path: fp32-query int4
// scoring with reducers and candidates (CudaInt4PackedDocs.maxsim_batch /
// topk_batch / score_*_batch, cu:2835-2991, score_impl cu:3124-3206), the
// fused int4 residual (cu:2911-2955), and the binary corpus handle
// CudaPackedDocs (cu:1872-2675).  Kernels: score.hip.
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "capi_handles.hpp"

#include <algorithm>

namespace msim {

namespace {

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Upload host tables; returns the device pointers.
template <typename T>
T* upload_vec(DeviceBuffer& buf, const std::vector<T>& v, const char* what) {
  buf.ensure(std::max<size_t>(sizeof(T) * v.size(), sizeof(T)), what);
  if (!v.empty()) check_hip(hipMemcpy(buf.ptr, v.data(), sizeof(T) * v.size(), hipMemcpyHostToDevice), what);
  return buf.as<T>();
}

// The same, enqueued on `stream`: a per-call table (weights, candidate
// tables) is overwritten only after the kernels queued before it on that
// stream, which may still read the previous call's contents.  From pageable
// host memory the runtime stages or copies before returning, so `v` may go
// out of scope afterwards.
template <typename T>
T* upload_vec(DeviceBuffer& buf, const std::vector<T>& v, const char* what, hipStream_t stream) {
  buf.ensure(std::max<size_t>(sizeof(T) * v.size(), sizeof(T)), what);
  if (!v.empty())
    check_hip(hipMemcpyAsync(buf.ptr, v.data(), sizeof(T) * v.size(), hipMemcpyHostToDevice, stream), what);
  return buf.as<T>();
}

}  // namespace

CandidateLayout candidate_layout(int64_t batch, int64_t query_tokens, int limbs, int64_t per_target,
                                 int64_t max_doc_tiles, int chunks) {
  const int64_t rpp = score_rows_per_pass(limbs, query_tokens, chunks);
  const int64_t subs = ceil_div(query_tokens, rpp);
  int64_t waves = ceil_div((int64_t)device_cu_count() * 8, batch * subs);
  waves = std::max<int64_t>(1, std::min(waves, per_target));
  CandidateLayout cl;
  cl.per_wave = ceil_div(per_target, waves);
  cl.waves = ceil_div(ceil_div(per_target, cl.per_wave), 4) * 4;
  cl.cap = cl.per_wave * std::max<int64_t>(1, max_doc_tiles) + 1;
  return cl;
}

void run_generic_score(ScoreWorkspace& ws, const std::vector<int64_t>& off, int64_t num_tokens,
                       const DocStreams& s, const QueryInput& q, int reducer, float temperature,
                       int64_t batch, int64_t query_tokens, const float* h_row_weights, const Targets& t,
                       float* d_out, int64_t out_stride, int32_t* d_iout, hipStream_t stream) {
  const int64_t num_docs = (int64_t)off.size() - 1;
  const int64_t targets = (t.host || t.device) ? t.count : num_docs;
  if (batch == 0 || targets == 0) return;
  const int64_t rows = batch * query_tokens;
  if (query_tokens == 0 || num_tokens == 0) {
    // No query tokens, or every document is empty: every score is 0.
    for (int64_t b = 0; b < batch; ++b)
      if (d_out) check_hip(launch_fill_f32(d_out + b * out_stride, targets, 0.0f, stream), "zero scores");
    // int32 zero has the bit pattern of 0.0f.
    if (d_iout) check_hip(launch_fill_f32(reinterpret_cast<float*>(d_iout), batch * targets, 0.0f, stream), "zero scores");
    return;
  }
  const int limbs = q.limbs;
  const int64_t rows_padded = ceil_div(rows, 16) * 16 + 128;
  const int chunks = s.chunks;
  if (chunks != 1 && (limbs != 3 || q.d_qbits || q.alt_int4 || q.from_alt || (s.doc == kDocSign && s.residual)))
    throw NotSupported("dims above 128 are scored for fp32 queries against int4 or sign documents only");

  // Sign-bit queries against sign documents over every document, MaxSim on
  // unit token scales: the fp4 Hamming kernel reads the query bits itself.
  const bool fp4 = g_hamming_fp4 != 0 && q.d_qbits && s.doc == kDocSign && !s.residual && reducer == kRedMax &&
                   s.unit_tscale && chunks == 1 && !t.host && !t.device && h_row_weights == nullptr;

  // 1. Quantise the query rows.
  ws.qpack.ensure((size_t)limbs * rows_padded * 128 * chunks, "hipMalloc query limbs");
  ws.colmul.ensure(sizeof(float) * rows_padded, "hipMalloc query scales");
  ws.qsum.ensure(sizeof(int32_t) * limbs * rows_padded, "hipMalloc query limb sums");
  if (q.alt_int4) ws.qpack_alt.ensure((size_t)limbs * rows_padded * 128, "hipMalloc query limbs (int4 layout)");
  if (q.quantized || q.from_alt || fp4) {
    // reuse the workspace's quantised rows (the fp4 kernel reads the bits)
  } else if (q.d_qbits)
    check_hip(launch_quantize_bits(q.d_qbits, rows, rows_padded, ws.qpack.as<int8_t>(), ws.colmul.as<float>(),
                                   ws.qsum.as<int32_t>(), stream),
              "launch sign query kernel");
  else
    // A sign stream paired with an int4 residual is unpacked in the int4
    // lane order, so both share the int4 query layout.
    check_hip(launch_quantize_limbs(q.d_query, rows, rows_padded, limbs, s.residual ? kDocInt4 : s.doc, q.recip,
                                    ws.qpack.as<int8_t>(), ws.colmul.as<float>(), ws.qsum.as<int32_t>(), stream,
                                    kDocInt4, q.alt_int4 ? ws.qpack_alt.as<int8_t>() : nullptr, chunks),
              "launch query quantize kernel");

  // 2. Reducer weights, one per query row (padding rows 0).
  const float* d_weights = nullptr;
  if (h_row_weights) {
    std::vector<float> w((size_t)rows_padded, 0.0f);
    std::memcpy(w.data(), h_row_weights, sizeof(float) * rows);
    if (ws.weights.ptr != nullptr && w.size() == ws.weights_host.size() &&
        std::memcmp(w.data(), ws.weights_host.data(), sizeof(float) * w.size()) == 0) {
      d_weights = ws.weights.as<float>();
    } else {
      d_weights = upload_vec(ws.weights, w, "copy reducer query weights to device", stream);
      ws.weights_host = std::move(w);
    }
  }

  // 3. Work split.
  const int64_t groups = t.per_row ? batch : 1;
  const int64_t grp_rows = t.per_row ? query_tokens : rows;
  const int64_t rpp = fp4 ? kHammingRowsPerPass : score_rows_per_pass(limbs, grp_rows, chunks);
  const int64_t subs = ceil_div(grp_rows, rpp);
  const int64_t per_target = t.per_row ? t.count : targets;
  int64_t waves = ceil_div((int64_t)device_cu_count() * 8, groups * subs);
  waves = std::max<int64_t>(1, std::min(waves, per_target));

  ScoreArgs a{};
  const int64_t* d_targets = nullptr;
  if (t.device) {
    // Candidate lists on the device: fixed-size target ranges per wave; with
    // more than one per wave, tables written by candidate_tables_kernel (or
    // already by the selector).
    if (!t.per_row) throw InvalidArgument("device candidate lists must be per batch row");
    const CandidateLayout cl = candidate_layout(batch, query_tokens, limbs, per_target, t.max_doc_tiles, chunks);
    const int64_t w4 = cl.waves;
    d_targets = t.device;
    if (cl.per_wave == 1) {
      // One candidate per wave: the kernel takes its tiles from the
      // document's token range (no tables).
      if (t.d_offsets == nullptr) throw InvalidArgument("device candidate lists need the token offsets");
      a.direct_offsets = t.d_offsets;
      a.direct_count = per_target;
      a.num_waves = w4;
    } else {
      ws.cand_info.ensure(sizeof(int64_t) * groups * w4 * kScoreInfoWords, "hipMalloc candidate wave table");
      ws.cand_tiles.ensure(sizeof(uint64_t) * groups * w4 * cl.cap, "hipMalloc candidate tile table");
      if (!t.tables_ready)
        check_hip(launch_candidate_tables(t.device, per_target, groups, t.d_offsets, w4, cl.per_wave, cl.cap,
                                          ws.cand_info.as<int64_t>(), ws.cand_tiles.as<uint64_t>(), stream),
                  "launch candidate table kernel");
      a.wave_info = ws.cand_info.as<int64_t>();
      a.tiles = ws.cand_tiles.as<uint64_t>();
      a.num_waves = w4;
      a.info_grp_stride = w4 * kScoreInfoWords;
    }
  } else if (!t.host) {
    // The row-block pipeline kernels (three limbs, four 16-row blocks per
    // pass, one 128-dim chunk, no residual) take work units: a list per
    // workgroup of eight waves, about `waves` waves in all.
    const bool unit_tables = !fp4 && limbs == 3 && rpp == 64 && chunks == 1 && !s.rcodes &&
                             num_docs < kScoreMaxUnitTargets;
    const int64_t key = unit_tables ? -2 - ceil_div(waves, 8) : waves;
    if (ws.full_key != key) {
      std::vector<int64_t> info;
      std::vector<uint64_t> tiles;
      ws.full_units = 0;
      if (unit_tables)
        ws.full_units = build_score_units(off.data(), nullptr, num_docs, ceil_div(waves, 8), info, tiles);
      else
        build_score_tables(off.data(), nullptr, num_docs, waves, info, tiles);
      upload_vec(ws.full_info, info, "copy score wave table to device", stream);
      upload_vec(ws.full_tiles, tiles, "copy score tile table to device", stream);
      ws.full_key = key;
      ws.full_waves = (int64_t)info.size() / kScoreInfoWords;
    }
    a.wave_info = ws.full_info.as<int64_t>();
    a.tiles = ws.full_tiles.as<uint64_t>();
    a.num_waves = ws.full_waves;
    a.group_units = (int32_t)ws.full_units;
    a.info_grp_stride = 0;
  } else {
    // Per group: its own table, all padded to the same wave count.
    std::vector<std::vector<int64_t>> infos((size_t)groups);
    std::vector<uint64_t> tiles;
    int64_t max_waves = 0;
    for (int64_t gi = 0; gi < groups; ++gi) {
      std::vector<uint64_t> gt;
      build_score_tables(off.data(), t.host + gi * (t.per_row ? t.count : 0), per_target, waves, infos[gi], gt);
      for (size_t w = 0; w < infos[gi].size(); w += kScoreInfoWords) infos[gi][w + 3] += (int64_t)tiles.size();
      tiles.insert(tiles.end(), gt.begin(), gt.end());
      max_waves = std::max<int64_t>(max_waves, (int64_t)infos[gi].size() / kScoreInfoWords);
    }
    std::vector<int64_t> info;
    for (int64_t gi = 0; gi < groups; ++gi) {
      auto& gi_info = infos[gi];
      while ((int64_t)gi_info.size() / kScoreInfoWords < max_waves) {
        const int64_t pad[kScoreInfoWords] = {per_target, 0, 0, 0};
        gi_info.insert(gi_info.end(), pad, pad + kScoreInfoWords);
      }
      info.insert(info.end(), gi_info.begin(), gi_info.end());
    }
    a.wave_info = upload_vec(ws.cand_info, info, "copy candidate wave table to device", stream);
    a.tiles = upload_vec(ws.cand_tiles, tiles, "copy candidate tile table to device", stream);
    a.num_waves = max_waves;
    a.info_grp_stride = max_waves * kScoreInfoWords;
    std::vector<int64_t> ids(t.host, t.host + groups * per_target);
    d_targets = upload_vec(ws.cand_ids, ids, "copy candidates to device", stream);
  }

  // 4. Score; the batch-row sums over query tokens are taken in the kernel
  // or by pool_sum_kernel over pooled[target][row].
  a.codes = s.codes;
  a.tscale = s.tscale;
  a.tmul = s.tmul;
  a.rcodes = s.rcodes;
  a.rtscale = s.rtscale;
  a.rmul = s.rmul;
  a.targets = d_targets;
  a.targets_grp_stride = t.per_row ? t.count : 0;
  a.qpack = q.from_alt ? ws.qpack_alt.as<int8_t>() : ws.qpack.as<int8_t>();
  a.rows_padded = rows_padded;
  a.colmul = ws.colmul.as<float>();
  a.qsum = ws.qsum.as<int32_t>();
  a.weights = d_weights;
  a.subs = (int32_t)subs;
  a.grp_rows = (int32_t)grp_rows;
  a.doc_scale = s.doc_scale;
  a.scale = s.scale;
  a.temperature = temperature;
  a.unit_tscale = s.unit_tscale;
  a.query_tokens = (int32_t)query_tokens;
  a.chunks = chunks;
  a.qbits = fp4 ? q.d_qbits : nullptr;
  // Passes that hold whole batch rows let the kernel sum them itself.
  const bool in_kernel_sum = t.per_row ? subs == 1 : rpp % query_tokens == 0;
  if (in_kernel_sum) {
    a.out = d_out;
    a.out_stride = out_stride;
    a.iout = d_iout;
    a.iout_stride = per_target;
    if (fp4)
      check_hip(launch_hamming(a, stream), "launch fp4 hamming kernel");
    else
      check_hip(launch_score(a, s.doc, s.residual, limbs, reducer, groups, stream), "launch score kernel");
    return;
  }
  ws.pooled.ensure(sizeof(float) * std::max<int64_t>(1, groups * per_target * grp_rows), "hipMalloc pooled rows");
  a.pooled = ws.pooled.as<float>();
  a.pooled_grp_stride = per_target * grp_rows;
  if (fp4)
    check_hip(launch_hamming(a, stream), "launch fp4 hamming kernel");
  else
    check_hip(launch_score(a, s.doc, s.residual, limbs, reducer, groups, stream), "launch score kernel");
  const int64_t bs = t.per_row ? per_target * query_tokens : query_tokens;
  const int64_t ts = t.per_row ? query_tokens : rows;
  check_hip(launch_pool_sum(ws.pooled.as<float>(), batch, query_tokens, per_target, bs, ts, d_out, out_stride, d_iout,
                            stream),
            "launch pooled sum kernel");
}

}  // namespace msim

using namespace msim;

namespace {

int parse_reducer(const char* name) {
  const std::string r = name ? name : "";
  if (r == "maxsim" || r == "weighted_maxsim") return kRedMax;
  if (r == "topk2") return kRedTop2;
  if (r == "topk4") return kRedTop4;
  if (r == "smoothsim") return kRedLse;
  throw InvalidArgument("reducer must be one of 'maxsim', 'weighted_maxsim', 'topk2', 'topk4', or 'smoothsim'");
}

// Per-row weights [batch * query_tokens] from the caller's [Q], [1, Q] or
// [B, Q] array (upload_reducer_weights, cu:3080-3122).
std::vector<float> row_weights(const char* reducer, const float* w, int64_t ndim, int64_t d0, int64_t d1,
                               int64_t batch, int64_t query_tokens) {
  const bool requires = std::string(reducer ? reducer : "") == "weighted_maxsim";
  if (w == nullptr || ndim == 0) {
    if (requires) throw InvalidArgument("query_weights are required for reducer='weighted_maxsim'");
    return {};
  }
  if (!requires) throw InvalidArgument("query_weights are only valid for reducer='weighted_maxsim'");
  bool batched = false;
  if (ndim == 1 && d0 == query_tokens) {
    batched = false;
  } else if (ndim == 2 && d1 == query_tokens && (d0 == 1 || d0 == batch)) {
    batched = d0 == batch;
  } else {
    throw InvalidArgument("query_weights must have shape [query_tokens] or [batch, query_tokens]");
  }
  std::vector<float> out((size_t)(batch * query_tokens));
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t q = 0; q < query_tokens; ++q) out[b * query_tokens + q] = w[(batched ? b * query_tokens : 0) + q];
  return out;
}

void check_temperature(double t) {
  if (!(t > 0.0) || !std::isfinite(t)) throw InvalidArgument("temperature must be finite and > 0");
}

void check_candidates(const int64_t* c, int64_t m, int64_t num_docs) {
  if (m < 0) throw InvalidArgument("candidate_indices must be a 1-D array");
  for (int64_t i = 0; i < m; ++i)
    if (c[i] < 0 || c[i] >= num_docs)
      throw InvalidArgument("candidate_indices entries must be between 0 and num_docs - 1");
}

void select_device(int device) { check_hip(hipSetDevice(device), "hipSetDevice"); }

void check_k(int64_t k, int64_t n) {
  if (k < 1 || k > n) throw InvalidArgument("k must be between 1 and num_docs");
  if (k > kTopkMaxK) throw NotSupported("k above 4096 is not supported by the device top-k selector");
}

// The fp32 query [B, Q, dim] of a synchronous call as [rows, 128 chunks]
// (zero-padded from dim to whole 128-dim chunks) in the workspace's pinned
// host buffer: the quantisation kernels read it there, so no staging copy is
// queued.
const float* stage_query(ScoreWorkspace& ws, const float* query, int64_t rows, int64_t dim) {
  const int64_t width = 128 * (int64_t)std::max(1, score_chunks(dim));
  const size_t bytes = sizeof(float) * (size_t)(std::max<int64_t>(rows, 1) * width);
  ws.host_query.ensure(bytes, "hipHostMalloc query staging");
  float* q = ws.host_query.as<float>();
  if (rows == 0) return q;
  if (dim == width) {
    std::memcpy(q, query, sizeof(float) * (size_t)(rows * width));
  } else {
    for (int64_t r = 0; r < rows; ++r) {
      std::memcpy(q + r * width, query + r * dim, sizeof(float) * (size_t)dim);
      std::memset(q + r * width + dim, 0, sizeof(float) * (size_t)(width - dim));
    }
  }
  return q;
}

// Top-k results of a synchronous call: the selection kernel writes them into
// the workspace's pinned host buffer; finish() waits for the stream and
// copies them out.
struct HostTopk {
  float* s = nullptr;
  int64_t* i = nullptr;
  size_t sbytes = 0, ibytes = 0;
  HostTopk(ScoreWorkspace& ws, int64_t batch, int64_t k)
      : sbytes(sizeof(float) * (size_t)(batch * k)), ibytes(sizeof(int64_t) * (size_t)(batch * k)) {
    const size_t s_al = (sbytes + 255) & ~(size_t)255;
    ws.host_out.ensure(std::max<size_t>(s_al + ibytes, 8), "hipHostMalloc top-k result staging");
    s = ws.host_out.as<float>();
    i = reinterpret_cast<int64_t*>(ws.host_out.as<char>() + s_al);
  }
  void finish(float* out_s, int64_t* out_i, hipStream_t stream) const {
    check_hip(hipStreamSynchronize(stream), "synchronize top-k selection");
    std::memcpy(out_s, s, sbytes);
    std::memcpy(out_i, i, ibytes);
  }
};

// A full score matrix of a synchronous call: one DMA copy into the
// workspace's pinned host buffer, then out of it once the stream is done.
void copy_scores_out(ScoreWorkspace& ws, void* out, const void* d, size_t bytes) {
  ws.host_out.ensure(std::max<size_t>(bytes, 8), "hipHostMalloc score staging");
  check_hip(hipMemcpyAsync(ws.host_out.ptr, d, bytes, hipMemcpyDeviceToHost, nullptr), "copy output to host");
  check_hip(hipStreamSynchronize(nullptr), "synchronize score copy");
  std::memcpy(out, ws.host_out.ptr, bytes);
}

// ------------------------------------------------------------------ int4

DocStreams int4_streams(msim_int4_docs* h, bool residual) {
  if (h->dim > kScoreMaxDim) throw NotSupported("fp32-query int4 scoring currently supports dim <= 512");
  if (h->num_tokens > 0 && !h->has_token_scale && h->ones16.cap < (size_t)h->num_tokens * 4) {
    std::vector<float> ones((size_t)h->num_tokens, 0.0625f);
    h->ones16.ensure(ones.size() * 4, "hipMalloc int4 unit token scales");
    check_hip(hipMemcpy(h->ones16.ptr, ones.data(), ones.size() * 4, hipMemcpyHostToDevice), "copy unit token scales");
  }
  DocStreams s;
  s.doc = kDocInt4;
  s.chunks = score_chunks(h->dim);
  s.codes = h->codes_wide.ptr ? h->codes_wide.as<uint8_t>() : h->packed.as<uint8_t>();
  s.tscale = h->has_token_scale ? h->token_scales16.as<float>() : h->ones16.as<float>();
  s.tmul = (float)h->scale;
  s.scale = 1.0f;
  if (residual) {
    if (!h->has_residual)
      throw InvalidArgument("residual int4 data was requested but is not loaded on this CUDA handle");
    s.residual = true;
    s.rcodes = h->residual_wide.ptr ? h->residual_wide.as<uint8_t>() : h->residual_packed.as<uint8_t>();
    s.rtscale = h->residual_token_scales16.as<float>();
    s.rmul = (float)h->residual_scale;
  }
  return s;
}

void check_dim(int64_t dim, int64_t expected) {
  if (dim != expected) throw InvalidArgument("query shape does not match dim");
}

// Scores of the fp32 query against every document (or candidates) into a
// device buffer of [batch, targets]; returns it.
float* int4_score_device(msim_int4_docs* h, const float* query, int64_t batch, int64_t query_tokens, int64_t dim,
                         int reducer, const std::vector<float>& w, float temperature, const int64_t* cand,
                         int64_t m, bool residual, hipStream_t stream) {
  const int64_t targets = cand ? m : h->num_docs;
  const DocStreams s = int4_streams(h, residual);
  const float* d_query = stage_query(h->ws, query, batch * query_tokens, dim);
  h->scores.ensure(sizeof(float) * std::max<int64_t>(1, batch * targets), "hipMalloc score cache");
  QueryInput qi;
  qi.d_query = d_query;
  qi.limbs = 3;
  Targets t{cand, m, false};
  run_generic_score(h->ws, h->host_offsets, h->num_tokens, s, qi, reducer, temperature, batch, query_tokens,
                    w.empty() ? nullptr : w.data(), t, h->scores.as<float>(), targets, nullptr, stream);
  return h->scores.as<float>();
}

}  // namespace

extern "C" int msim_int4_maxsim_batch(msim_int4_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                                      int64_t dim, float* out) {
  return guarded([&] {
    require_handle(h);
    check_dim(dim, h->dim);
    require_shape(batch, query_tokens);
    if (batch == 0 || h->num_docs == 0) return;
    select_device(h->device);
    float* d = int4_score_device(h, query, batch, query_tokens, dim, kRedMax, {}, 1.0f, nullptr, 0, false, nullptr);
    copy_scores_out(h->ws, out, d, sizeof(float) * batch * h->num_docs);
  });
}

extern "C" int msim_int4_topk_batch(msim_int4_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                                    int64_t dim, int64_t k, float* out_scores, int64_t* out_indices) {
  return guarded([&] {
    require_handle(h);
    check_k(k, h->num_docs);
    check_dim(dim, h->dim);
    require_shape(batch, query_tokens);
    if (batch == 0) return;
    select_device(h->device);
    float* d = int4_score_device(h, query, batch, query_tokens, dim, kRedMax, {}, 1.0f, nullptr, 0, false, nullptr);
    const HostTopk out(h->ws, batch, k);
    check_hip(launch_topk(d, batch, h->num_docs, h->num_docs, k, nullptr, out.s, out.i, nullptr),
              "launch topk selection kernel");
    out.finish(out_scores, out_indices, nullptr);
  });
}

extern "C" int msim_int4_score(msim_int4_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                               int64_t dim, const char* reducer, const float* weights, int64_t weights_ndim,
                               int64_t weights_dim0, int64_t weights_dim1, double temperature,
                               const int64_t* candidates, int64_t num_candidates, int residual, float* out) {
  return guarded([&] {
    require_handle(h);
    check_dim(dim, h->dim);
    require_shape(batch, query_tokens);
    if (candidates) check_candidates(candidates, num_candidates, h->num_docs);
    const int red = parse_reducer(reducer);
    check_temperature(temperature);
    const std::vector<float> w =
        row_weights(reducer, weights, weights_ndim, weights_dim0, weights_dim1, batch, query_tokens);
    if (residual && !h->has_residual)
      throw InvalidArgument("residual int4 data was requested but is not loaded on this CUDA handle");
    const int64_t targets = candidates ? num_candidates : h->num_docs;
    if (batch == 0 || targets == 0) return;
    select_device(h->device);
    float* d = int4_score_device(h, query, batch, query_tokens, dim, red, w, (float)temperature, candidates,
                                 num_candidates, residual != 0, nullptr);
    copy_scores_out(h->ws, out, d, sizeof(float) * batch * targets);
  });
}

// ------------------------------------------------------------------ binary

namespace {

DocStreams binary_streams(msim_binary_docs* h, double scale, bool use_scale_vector, bool use_token_scale,
                          const float* d_scale_override) {
  if (use_scale_vector && !h->has_scale_vector)
    throw InvalidArgument("scale vector was requested but is not loaded on this CUDA handle");
  if (use_token_scale && !h->has_token_scale)
    throw InvalidArgument("token scale vector was requested but is not loaded on this CUDA handle");
  if (h->num_tokens > 0 && !(use_token_scale) && h->ones.cap < (size_t)h->num_tokens * 4) {
    std::vector<float> ones((size_t)h->num_tokens, 1.0f);
    h->ones.ensure(ones.size() * 4, "hipMalloc binary unit token scales");
    check_hip(hipMemcpy(h->ones.ptr, ones.data(), ones.size() * 4, hipMemcpyHostToDevice), "copy unit token scales");
  }
  DocStreams s;
  s.doc = kDocSign;
  s.codes = h->packed.as<uint8_t>();
  s.tscale = use_token_scale ? h->token_scales.as<float>() : h->ones.as<float>();
  s.tmul = 1.0f;
  s.doc_scale = d_scale_override ? d_scale_override : (use_scale_vector ? h->scale_vector.as<float>() : nullptr);
  s.scale = (float)scale;
  s.unit_tscale = !use_token_scale;
  s.chunks = score_chunks(h->dim);
  return s;
}

float* binary_score_device(msim_binary_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                           int64_t dim, int limbs, bool recip, const DocStreams& s, int reducer,
                           const std::vector<float>& w, float temperature, const int64_t* cand, int64_t m) {
  const int64_t targets = cand ? m : h->num_docs;
  const float* d_query = stage_query(h->ws, query, batch * query_tokens, dim);
  h->scores.ensure(sizeof(float) * std::max<int64_t>(1, batch * targets), "hipMalloc score cache");
  QueryInput qi;
  qi.d_query = d_query;
  qi.limbs = limbs;
  qi.recip = recip;
  Targets t{cand, m, false};
  run_generic_score(h->ws, h->host_offsets, h->num_tokens, s, qi, reducer, temperature, batch, query_tokens,
                    w.empty() ? nullptr : w.data(), t, h->scores.as<float>(), targets, nullptr, nullptr);
  return h->scores.as<float>();
}

void copy_topk_out(msim_binary_docs* h, const float* d_scores, int64_t batch, int64_t k, float* out_scores,
                   int64_t* out_indices, hipStream_t stream) {
  const HostTopk out(h->ws, batch, k);
  check_hip(launch_topk(d_scores, batch, h->num_docs, h->num_docs, k, nullptr, out.s, out.i, stream),
            "launch topk selection kernel");
  out.finish(out_scores, out_indices, stream);
}

void check_binary_query(const msim_binary_docs* h, int64_t batch, int64_t query_tokens, int64_t dim) {
  require_shape(batch, query_tokens);
  if (dim != h->dim) throw InvalidArgument("query shape does not match dim");
}

void check_int8q_dim(const msim_binary_docs* h) {
  if (h->dim != 128) throw InvalidArgument("int8 query scoring currently requires dim=128");
}

}  // namespace

extern "C" int msim_binary_create(const uint8_t* packed, int64_t num_tokens, int64_t row_bytes,
                                  const int64_t* offsets, int64_t num_offsets, int dim, msim_binary_docs** out) {
  return guarded([&] {
    if (out == nullptr) throw InvalidArgument("out handle pointer must not be NULL");
    *out = nullptr;
    if (dim <= 0 || dim % 8 != 0) throw InvalidArgument("dim must be positive and divisible by 8");
    if (row_bytes != dim / 8) throw InvalidArgument("packed shape does not match dim");
    if (dim > kScoreMaxDim) throw NotSupported("binary scoring currently supports dim <= 512");
    if (num_tokens < 0) throw InvalidArgument("packed must have shape [num_doc_tokens, dim / 8]");
    validate_offsets(offsets, num_offsets, num_tokens);
    if (num_tokens > 0 && packed == nullptr) throw InvalidArgument("packed must not be NULL");
    auto h = std::make_unique<msim_binary_docs>();
    check_hip(hipGetDevice(&h->device), "hipGetDevice");
    h->dim = dim;
    h->num_docs = num_offsets - 1;
    h->num_tokens = num_tokens;
    h->packed_size = (uint64_t)num_tokens * (uint64_t)row_bytes;
    h->host_offsets.assign(offsets, offsets + num_offsets);
    for (int64_t d = 0; d + 1 < num_offsets; ++d)
      h->max_doc_tiles = std::max<int64_t>(h->max_doc_tiles, (offsets[d + 1] - offsets[d] + 15) / 16);
    // Rows widened to whole 128-dim chunks (16 bytes each): padding bits meet
    // zero query dims.  The int8-query scan of the sign stream (dim 128) may
    // read kScanPadTokens rows past the end: zero rows follow.
    const int64_t width = 16 * (int64_t)score_chunks(dim);
    std::vector<uint8_t> wide((size_t)((num_tokens + kScanPadTokens) * width), 0);
    for (int64_t t = 0; t < num_tokens; ++t) std::memcpy(&wide[t * width], packed + t * row_bytes, (size_t)row_bytes);
    upload_vec(h->packed, wide, "copy binary packed docs to device");
    std::vector<int64_t> offs(offsets, offsets + num_offsets);
    upload_vec(h->offsets, offs, "copy binary offsets to device");
    *out = h.release();
  });
}

extern "C" int msim_binary_destroy(msim_binary_docs* h) {
  return guarded([&] {
    if (h == nullptr) return;
    (void)hipSetDevice(h->device);
    delete h;
  });
}

extern "C" int msim_binary_set_scale_vector(msim_binary_docs* h, const float* scale, int64_t count) {
  return guarded([&] {
    require_handle(h);
    if (count != h->num_docs) throw InvalidArgument("scale vector must have shape [num_docs]");
    select_device(h->device);
    std::vector<float> v(scale, scale + count);
    upload_vec(h->scale_vector, v, "copy binary scale vector to device");
    h->has_scale_vector = true;
  });
}

extern "C" int msim_binary_clear_scale_vector(msim_binary_docs* h) {
  return guarded([&] {
    require_handle(h);
    h->has_scale_vector = false;
  });
}

extern "C" int msim_binary_set_token_scale(msim_binary_docs* h, const float* token_scales, int64_t count) {
  return guarded([&] {
    require_handle(h);
    if (count != h->num_tokens) throw InvalidArgument("token scale vector must have shape [num_doc_tokens]");
    select_device(h->device);
    h->token_scales_fma = std::all_of(token_scales, token_scales + count,
                                      [](float x) { return x >= kScanFmaMinScale && x < kScanFmaMaxScale; });
    std::vector<float> v(token_scales, token_scales + count);
    v.resize((size_t)(count + kScanPadTokens), 0.0f);  // rows the scan may read past the end
    upload_vec(h->token_scales, v, "copy binary token scale vector to device");
    h->has_token_scale = true;
  });
}

extern "C" int msim_binary_clear_token_scale(msim_binary_docs* h) {
  return guarded([&] {
    require_handle(h);
    h->has_token_scale = false;
  });
}

extern "C" int msim_binary_get_props(const msim_binary_docs* h, msim_binary_props* out) {
  return guarded([&] {
    require_handle(h);
    if (out == nullptr) throw InvalidArgument("props pointer must not be NULL");
    out->dim = h->dim;
    out->num_docs = h->num_docs;
    out->num_tokens = h->num_tokens;
    out->packed_size = h->packed_size;
    out->has_scale_vector = h->has_scale_vector ? 1 : 0;
    out->scale_vector_size = h->has_scale_vector ? (uint64_t)h->num_docs : 0;
    out->has_token_scale_vector = h->has_token_scale ? 1 : 0;
    out->token_scale_vector_size = h->has_token_scale ? (uint64_t)h->num_tokens : 0;
    out->resident_bytes = h->resident_bytes();
    out->workspace_bytes = h->workspace_bytes();
  });
}

extern "C" int msim_binary_maxsim_batch(msim_binary_docs* h, const float* query, int64_t batch,
                                        int64_t query_tokens, int64_t dim, double scale, int use_scale_vector,
                                        int use_token_scale, float* out) {
  return guarded([&] {
    require_handle(h);
    check_binary_query(h, batch, query_tokens, dim);
    if (batch == 0 || h->num_docs == 0) return;
    select_device(h->device);
    const DocStreams s = binary_streams(h, scale, use_scale_vector, use_token_scale, nullptr);
    float* d = binary_score_device(h, query, batch, query_tokens, dim, 3, false, s, kRedMax, {}, 1.0f, nullptr, 0);
    copy_scores_out(h->ws, out, d, sizeof(float) * batch * h->num_docs);
  });
}

extern "C" int msim_binary_topk_batch(msim_binary_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                                      int64_t dim, int64_t k, double scale, int use_scale_vector, int use_token_scale,
                                      float* out_scores, int64_t* out_indices) {
  return guarded([&] {
    require_handle(h);
    check_k(k, h->num_docs);
    check_binary_query(h, batch, query_tokens, dim);
    if (batch == 0) return;
    select_device(h->device);
    const DocStreams s = binary_streams(h, scale, use_scale_vector, use_token_scale, nullptr);
    float* d = binary_score_device(h, query, batch, query_tokens, dim, 3, false, s, kRedMax, {}, 1.0f, nullptr, 0);
    copy_topk_out(h, d, batch, k, out_scores, out_indices, nullptr);
  });
}

extern "C" int msim_binary_maxsim_batch_int8q(msim_binary_docs* h, const float* query, int64_t batch,
                                              int64_t query_tokens, int64_t dim, double scale, int use_scale_vector,
                                              int use_token_scale, float* out) {
  return guarded([&] {
    require_handle(h);
    check_int8q_dim(h);
    check_binary_query(h, batch, query_tokens, dim);
    if (batch == 0 || h->num_docs == 0) return;
    select_device(h->device);
    const DocStreams s = binary_streams(h, scale, use_scale_vector, use_token_scale, nullptr);
    float* d = binary_score_device(h, query, batch, query_tokens, dim, 1, true, s, kRedMax, {}, 1.0f, nullptr, 0);
    copy_scores_out(h->ws, out, d, sizeof(float) * batch * h->num_docs);
  });
}

extern "C" int msim_binary_topk_batch_int8q(msim_binary_docs* h, const float* query, int64_t batch,
                                            int64_t query_tokens, int64_t dim, int64_t k, double scale,
                                            int use_scale_vector, int use_token_scale, float* out_scores,
                                            int64_t* out_indices) {
  return guarded([&] {
    require_handle(h);
    check_k(k, h->num_docs);
    check_int8q_dim(h);
    check_binary_query(h, batch, query_tokens, dim);
    if (batch == 0) return;
    select_device(h->device);
    const DocStreams s = binary_streams(h, scale, use_scale_vector, use_token_scale, nullptr);
    float* d = binary_score_device(h, query, batch, query_tokens, dim, 1, true, s, kRedMax, {}, 1.0f, nullptr, 0);
    copy_topk_out(h, d, batch, k, out_scores, out_indices, nullptr);
  });
}

extern "C" int msim_binary_score(msim_binary_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                                 int64_t dim, const char* reducer, const float* weights, int64_t weights_ndim,
                                 int64_t weights_dim0, int64_t weights_dim1, double temperature, double scale,
                                 int use_scale_vector, int use_token_scale, const float* scale_vector_override,
                                 const int64_t* candidates, int64_t num_candidates, float* out) {
  return guarded([&] {
    require_handle(h);
    check_binary_query(h, batch, query_tokens, dim);
    if (candidates) check_candidates(candidates, num_candidates, h->num_docs);
    const int red = parse_reducer(reducer);
    check_temperature(temperature);
    const std::vector<float> w =
        row_weights(reducer, weights, weights_ndim, weights_dim0, weights_dim1, batch, query_tokens);
    const int64_t targets = candidates ? num_candidates : h->num_docs;
    if (batch == 0 || targets == 0) return;
    select_device(h->device);
    const float* d_override = nullptr;
    if (scale_vector_override) {
      std::vector<float> v(scale_vector_override, scale_vector_override + h->num_docs);
      d_override = upload_vec(h->scale_override, v, "copy scale vector override to device");
    }
    const DocStreams s = binary_streams(h, scale, use_scale_vector, use_token_scale, d_override);
    float* d = binary_score_device(h, query, batch, query_tokens, dim, 3, false, s, red, w, (float)temperature,
                                   candidates, num_candidates);
    copy_scores_out(h->ws, out, d, sizeof(float) * batch * targets);
  });
}

namespace {

// Hamming MaxSim of sign-bit queries on the device: int32 [B, N] into
// h->iscores and (when d_fscores) float scores.
void hamming_device(msim_binary_docs* h, const uint8_t* d_qbits, int64_t batch, int64_t query_tokens,
                    float* d_fscores, int32_t* d_iscores, hipStream_t stream) {
  if (h->dim != 128) throw InvalidArgument("sign-query scoring currently requires dim=128");
  DocStreams s = binary_streams(h, 1.0, false, false, nullptr);
  QueryInput qi;
  qi.d_qbits = d_qbits;
  qi.limbs = 1;
  Targets t{};
  run_generic_score(h->ws, h->host_offsets, h->num_tokens, s, qi, kRedMax, 1.0f, batch, query_tokens, nullptr, t,
                    d_fscores, h->num_docs, d_iscores, stream);
}

const uint8_t* upload_qbits(msim_binary_docs* h, const uint8_t* qbits, int64_t rows) {
  h->ws.qbits.ensure((size_t)std::max<int64_t>(rows, 1) * 16, "hipMalloc sign query cache");
  if (rows) check_hip(hipMemcpy(h->ws.qbits.ptr, qbits, (size_t)rows * 16, hipMemcpyHostToDevice), "copy sign query");
  return h->ws.qbits.as<uint8_t>();
}

}  // namespace

extern "C" int msim_binary_hamming_batch(msim_binary_docs* h, const uint8_t* qbits, int64_t batch,
                                         int64_t query_tokens, int64_t dim, int32_t* out) {
  return guarded([&] {
    require_handle(h);
    check_binary_query(h, batch, query_tokens, dim);
    if (batch == 0 || h->num_docs == 0) return;
    select_device(h->device);
    const uint8_t* d_q = upload_qbits(h, qbits, batch * query_tokens);
    h->iscores.ensure(sizeof(int32_t) * batch * h->num_docs, "hipMalloc hamming scores");
    hamming_device(h, d_q, batch, query_tokens, nullptr, h->iscores.as<int32_t>(), nullptr);
    copy_scores_out(h->ws, out, h->iscores.ptr, sizeof(int32_t) * batch * h->num_docs);
  });
}

extern "C" int msim_binary_topk_hamming(msim_binary_docs* h, const uint8_t* qbits, int64_t batch,
                                        int64_t query_tokens, int64_t dim, int64_t k, float* out_scores,
                                        int64_t* out_indices) {
  return guarded([&] {
    require_handle(h);
    check_k(k, h->num_docs);
    check_binary_query(h, batch, query_tokens, dim);
    if (batch == 0) return;
    select_device(h->device);
    const uint8_t* d_q = upload_qbits(h, qbits, batch * query_tokens);
    h->scores.ensure(sizeof(float) * batch * h->num_docs, "hipMalloc score cache");
    hamming_device(h, d_q, batch, query_tokens, h->scores.as<float>(), nullptr, nullptr);
    copy_topk_out(h, h->scores.as<float>(), batch, k, out_scores, out_indices, nullptr);
  });
}

extern "C" int msim_binary_topk_hamming_async(msim_binary_docs* h, const uint8_t* d_qbits, int64_t batch,
                                              int64_t query_tokens, int64_t k, float* d_scores, int64_t* d_indices,
                                              void* stream) {
  return guarded([&] {
    require_handle(h);
    check_k(k, h->num_docs);
    require_shape(batch, query_tokens);
    if (batch == 0) return;
    select_device(h->device);
    h->scores.ensure(sizeof(float) * batch * h->num_docs, "hipMalloc score cache");
    hamming_device(h, d_qbits, batch, query_tokens, h->scores.as<float>(), nullptr, as_stream(stream));
    check_hip(launch_topk(h->scores.as<float>(), batch, h->num_docs, h->num_docs, k, nullptr, d_scores, d_indices,
                          as_stream(stream)),
              "launch topk selection kernel");
  });
}

// ----------------------------------------------------------------- cascades

namespace {

void check_cascade(int64_t k, int64_t m, int64_t num_docs) {
  if (k < 1 || k > m || m > num_docs)
    throw InvalidArgument("cascade sizes must satisfy 1 <= k <= candidates <= num_docs");
  if (m > kTopkMaxK || m > kSortMaxRow)
    throw NotSupported("cascade candidate budgets above 4096 are not supported by the device selector");
}

// Coarse scores of every document -> the top-M candidates of each batch row
// (score desc, document asc), put in document order -> fine scores of the
// candidates -> top-k, ties by document id (cascade.py:294-453), all on the
// device.  coarse(d_scores) and fine(d_candidate_ids, d_scores,
// tables_ready) enqueue the two scoring passes.  With one candidate per
// rescoring wave (`layout`, the rescoring pass's candidate_layout) the pass
// needs no tables; with more, the selector writes them itself, one launch
// fewer (tables_ready is then true).
template <typename Coarse, typename Fine>
void cascade_device(ScoreWorkspace& ws, int64_t batch, int64_t num_docs, int64_t k, int64_t m, Coarse coarse,
                    Fine fine, float* d_top_s, int64_t* d_top_i, hipStream_t stream, const CandidateLayout& layout,
                    const int64_t* d_offsets) {
  ws.coarse.ensure(sizeof(float) * batch * num_docs, "hipMalloc cascade coarse scores");
  coarse(ws.coarse.as<float>());
  ws.top_m_ids.ensure(sizeof(int64_t) * batch * m, "hipMalloc cascade candidates");
  bool tables_ready = false;
  if (num_docs <= kSortMaxRow) {
    // One candidate per rescoring wave needs no tables (the pass reads each
    // candidate's token range itself).
    const bool tables = layout.per_wave > 1;
    CandidateTables tab;
    if (tables) {
      ws.cand_info.ensure(sizeof(int64_t) * batch * layout.waves * kScoreInfoWords, "hipMalloc candidate wave table");
      ws.cand_tiles.ensure(sizeof(uint64_t) * batch * layout.waves * layout.cap, "hipMalloc candidate tile table");
      tab.d_offsets = d_offsets;
      tab.waves = layout.waves;
      tab.per_wave = layout.per_wave;
      tab.cap = layout.cap;
      tab.d_info = ws.cand_info.as<int64_t>();
      tab.d_tiles = ws.cand_tiles.as<uint64_t>();
    }
    check_hip(launch_select_topm(ws.coarse.as<float>(), batch, num_docs, num_docs, m, ws.top_m_ids.as<int64_t>(),
                                 stream, tables ? &tab : nullptr),
              "launch cascade candidate selection");
    tables_ready = tables;
  } else {
    ws.top_m_scores.ensure(sizeof(float) * batch * m, "hipMalloc cascade candidate scores");
    check_hip(launch_topk(ws.coarse.as<float>(), batch, num_docs, num_docs, m, nullptr, ws.top_m_scores.as<float>(),
                          ws.top_m_ids.as<int64_t>(), stream),
              "launch cascade candidate selection");
    check_hip(launch_sort_rows(ws.top_m_ids.as<int64_t>(), batch, m, stream), "launch candidate sort");
  }
  ws.fine.ensure(sizeof(float) * batch * m, "hipMalloc cascade fine scores");
  fine(ws.top_m_ids.as<int64_t>(), ws.fine.as<float>(), tables_ready);
  check_hip(launch_topk(ws.fine.as<float>(), batch, m, m, k, ws.top_m_ids.as<int64_t>(), d_top_s, d_top_i, stream),
            "launch cascade final selection");
}

}  // namespace

extern "C" int msim_int4_cascade_topk(msim_int4_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                                      int64_t dim, int64_t k, int64_t candidates, const char* reducer,
                                      const float* weights, int64_t weights_ndim, int64_t weights_dim0,
                                      int64_t weights_dim1, double temperature, float* out_scores,
                                      int64_t* out_indices) {
  return guarded([&] {
    require_handle(h);
    check_dim(dim, h->dim);
    require_shape(batch, query_tokens);
    check_cascade(k, candidates, h->num_docs);
    const int red = parse_reducer(reducer);
    check_temperature(temperature);
    const std::vector<float> w =
        row_weights(reducer, weights, weights_ndim, weights_dim0, weights_dim1, batch, query_tokens);
    if (!h->has_residual)
      throw InvalidArgument("residual int4 data was requested but is not loaded on this CUDA handle");
    if (batch == 0) return;
    select_device(h->device);
    const DocStreams prefix = int4_streams(h, false), fused = int4_streams(h, true);
    QueryInput qi;
    qi.d_query = stage_query(h->ws, query, batch * query_tokens, dim);
    qi.limbs = 3;
    const float* wp = w.empty() ? nullptr : w.data();
    const HostTopk out(h->ws, batch, k);
    if (candidates == h->num_docs) {
      // Every document is a candidate: full fused scoring (cascade.py:342-351).
      h->scores.ensure(sizeof(float) * batch * h->num_docs, "hipMalloc score cache");
      run_generic_score(h->ws, h->host_offsets, h->num_tokens, fused, qi, red, (float)temperature, batch,
                        query_tokens, wp, Targets{}, h->scores.as<float>(), h->num_docs, nullptr, nullptr);
      check_hip(launch_topk(h->scores.as<float>(), batch, h->num_docs, h->num_docs, k, nullptr, out.s, out.i,
                            nullptr),
                "launch topk selection kernel");
    } else {
      cascade_device(
          h->ws, batch, h->num_docs, k, candidates,
          [&](float* d) {
            run_generic_score(h->ws, h->host_offsets, h->num_tokens, prefix, qi, red, (float)temperature, batch,
                              query_tokens, wp, Targets{}, d, h->num_docs, nullptr, nullptr);
          },
          [&](const int64_t* ids, float* d, bool tables_ready) {
            Targets t;
            t.device = ids;
            t.count = candidates;
            t.per_row = true;
            t.d_offsets = h->offsets.as<int64_t>();
            t.max_doc_tiles = h->max_doc_tiles;
            t.tables_ready = tables_ready;
            QueryInput again = qi;
            again.quantized = true;
            run_generic_score(h->ws, h->host_offsets, h->num_tokens, fused, again, red, (float)temperature, batch,
                              query_tokens, wp, t, d, candidates, nullptr, nullptr);
          },
          out.s, out.i, nullptr,
          candidate_layout(batch, query_tokens, qi.limbs, candidates, h->max_doc_tiles, fused.chunks),
          h->offsets.as<int64_t>());
    }
    out.finish(out_scores, out_indices, nullptr);
  });
}

// ------------------------------------- binary prefix + int4 residual format

namespace {

DocStreams binres_streams(msim_binary_docs* h, bool fused) {
  if (h->dim != 128) throw InvalidArgument("binary residual scoring currently requires dim=128");
  if (!h->has_token_scale)
    throw InvalidArgument("binary residual scoring needs the prefix scales: call set_token_scale_vector first");
  if (fused && !h->has_residual)
    throw InvalidArgument("residual int4 data was requested but is not loaded on this CUDA handle");
  DocStreams s;
  s.doc = kDocSign;
  s.codes = h->packed.as<uint8_t>();
  s.tscale = h->token_scales.as<float>();
  s.tmul = 1.0f;
  if (fused) {
    s.residual = true;
    s.rcodes = h->residual_packed.as<uint8_t>();
    s.rtscale = h->residual_token_scales16.as<float>();
    s.rmul = (float)h->residual_scale;
  }
  return s;
}

// The prefix (sign) pass of a cascade on the int8-query scan kernel: the
// query rows are quantised once (the sign layout for this pass, the int4
// layout for the rescoring pass, which reads them back with from_alt), then
// score[b, n] = sum_q sigma_q max_t a_t (q8 . sign_t) in numpy's pairwise
// float64 order -- the prefix scores of the host format, bit for bit.  False
// (nothing done) when the scan does not apply: query rows of more than 128
// tokens, or token scales outside the one-fma epilogue's range.
bool binres_scan_prefix(msim_binary_docs* h, const float* d_query, int64_t batch, int64_t query_tokens, float* d_out,
                        hipStream_t stream) {
  if (!h->token_scales_fma || query_tokens <= 0 || query_tokens > kScanPassRows || h->num_docs == 0 ||
      h->num_tokens == 0)
    return false;
  const int64_t waves = std::max<int64_t>(1, std::min<int64_t>((int64_t)device_cu_count() * kScanWavesPerCu, h->num_docs));
  if (h->scan_partition_waves != waves) {
    std::vector<int64_t> info;
    std::vector<uint64_t> tiles;
    build_scan_tables(h->host_offsets.data(), h->num_docs, waves, false, info, tiles, h->scan_tile_stride,
                      h->num_scan_waves);
    upload_vec(h->scan_wave_info, info, "copy sign scan wave table to device");
    upload_vec(h->scan_tile_table, tiles, "copy sign scan tile table to device");
    h->scan_partition_waves = waves;
  }
  ScoreWorkspace& ws = h->ws;
  const int64_t rows = batch * query_tokens, rows_padded = ceil_div(rows, 16) * 16 + 128;
  ws.qpack.ensure((size_t)rows_padded * 128, "hipMalloc query limbs");
  ws.qpack_alt.ensure((size_t)rows_padded * 128, "hipMalloc query limbs (int4 layout)");
  ws.colmul.ensure(sizeof(float) * rows_padded, "hipMalloc query scales");
  ws.qsum.ensure(sizeof(int32_t) * rows_padded, "hipMalloc query limb sums");
  check_hip(launch_quantize_limbs(d_query, rows, rows_padded, 1, kDocSign, false, ws.qpack.as<int8_t>(),
                                  ws.colmul.as<float>(), ws.qsum.as<int32_t>(), stream, kDocInt4,
                                  ws.qpack_alt.as<int8_t>()),
            "launch query quantize kernel");
  ScanArgs a{};
  a.codes = h->packed.as<uint8_t>();
  a.token_scale16 = h->token_scales.as<float>();
  a.offsets = h->offsets.as<int64_t>();
  a.wave_info = h->scan_wave_info.as<int64_t>();
  a.tile_table = h->scan_tile_table.as<uint64_t>();
  a.tile_stride = h->scan_tile_stride;
  a.num_waves = h->num_scan_waves;
  a.q_row_order = 1;
  a.doc_sign = 1;
  a.query_tokens = (int32_t)query_tokens;
  a.scale = 1.0;
  a.score_stride = h->num_docs;
  a.num_docs = h->num_docs;
  const int64_t per_pass = std::max<int64_t>(1, kScanPassRows / query_tokens);
  for (int64_t b0 = 0; b0 < batch; b0 += per_pass) {
    const int64_t nb = std::min(per_pass, batch - b0), row0 = b0 * query_tokens;
    a.qpack = ws.qpack.as<int8_t>() + row0 * 128;
    a.qscale = ws.colmul.as<float>() + row0;
    a.qsum = ws.qsum.as<int32_t>() + row0;
    a.batch = (int32_t)nb;
    a.scores = d_out + b0 * h->num_docs;
    check_hip(launch_int8q_scan(a, kScanEpiFma, stream), "launch int8q sign scan kernel");
  }
  return true;
}

void binres_cascade(msim_binary_docs* h, const float* d_query, int64_t batch, int64_t query_tokens, int64_t k,
                    int64_t m, float* d_top_s, int64_t* d_top_i, hipStream_t stream) {
  const DocStreams prefix = binres_streams(h, false), fused = binres_streams(h, true);
  QueryInput qi;
  qi.d_query = d_query;
  qi.limbs = h->rescore_limbs;
  if (m == h->num_docs) {
    h->scores.ensure(sizeof(float) * batch * h->num_docs, "hipMalloc score cache");
    run_generic_score(h->ws, h->host_offsets, h->num_tokens, fused, qi, kRedMax, 1.0f, batch, query_tokens, nullptr,
                      Targets{}, h->scores.as<float>(), h->num_docs, nullptr, stream);
    check_hip(launch_topk(h->scores.as<float>(), batch, h->num_docs, h->num_docs, k, nullptr, d_top_s, d_top_i,
                          stream),
              "launch topk selection kernel");
    return;
  }
  // With the int8 query, one quantisation serves both passes: the prefix
  // pass's sign layout, and the int4 layout the fused pass reads (its sign
  // stream is unpacked in the int4 lane order).  With the fp32 query, the
  // rescoring pass quantises its three limbs itself (its buffers sized first,
  // so that no buffer the prefix pass reads is reallocated while in flight).
  QueryInput coarse_q = qi;
  coarse_q.limbs = 1;
  coarse_q.alt_int4 = true;
  QueryInput fine_q = qi;
  if (qi.limbs == 1) {
    fine_q.from_alt = true;
  } else {
    const int64_t rows_padded = ceil_div(batch * query_tokens, 16) * 16 + 128;
    h->ws.qpack.ensure((size_t)qi.limbs * rows_padded * 128, "hipMalloc query limbs");
    h->ws.qsum.ensure(sizeof(int32_t) * qi.limbs * rows_padded, "hipMalloc query limb sums");
  }
  cascade_device(
      h->ws, batch, h->num_docs, k, m,
      [&](float* d) {
        if (g_scan_prefix && binres_scan_prefix(h, d_query, batch, query_tokens, d, stream)) return;
        run_generic_score(h->ws, h->host_offsets, h->num_tokens, prefix, coarse_q, kRedMax, 1.0f, batch, query_tokens,
                          nullptr, Targets{}, d, h->num_docs, nullptr, stream);
      },
      [&](const int64_t* ids, float* d, bool tables_ready) {
        Targets t;
        t.device = ids;
        t.count = m;
        t.per_row = true;
        t.d_offsets = h->offsets.as<int64_t>();
        t.max_doc_tiles = h->max_doc_tiles;
        t.tables_ready = tables_ready;
        run_generic_score(h->ws, h->host_offsets, h->num_tokens, fused, fine_q, kRedMax, 1.0f, batch, query_tokens,
                          nullptr, t, d, m, nullptr, stream);
      },
      d_top_s, d_top_i, stream, candidate_layout(batch, query_tokens, qi.limbs, m, h->max_doc_tiles),
      h->offsets.as<int64_t>());
}

}  // namespace

extern "C" int msim_binary_set_residual(msim_binary_docs* h, const uint8_t* packed, int64_t num_tokens,
                                        int64_t row_bytes, double scale, const float* token_scales, int64_t count) {
  return guarded([&] {
    require_handle(h);
    if (h->dim != 128) throw InvalidArgument("binary residual data currently requires dim=128");
    if (num_tokens != h->num_tokens || row_bytes != h->dim / 2)
      throw InvalidArgument("residual packed data must have shape [num_doc_tokens, dim / 2]");
    if (!(scale > 0.0) || !std::isfinite(scale)) throw InvalidArgument("residual scale must be finite and > 0");
    if (count != h->num_tokens) throw InvalidArgument("residual token scale vector must have shape [num_doc_tokens]");
    validate_positive_scales(token_scales, count, "residual token scales must be finite and > 0");
    select_device(h->device);
    std::vector<uint8_t> codes(packed, packed + (size_t)num_tokens * (size_t)row_bytes);
    upload_vec(h->residual_packed, codes, "copy binary residual data to device");
    std::vector<float> s16(token_scales, token_scales + count);
    for (float& v : s16) v *= 0.0625f;
    upload_vec(h->residual_token_scales16, s16, "copy binary residual token scales to device");
    h->residual_scale = scale;
    h->has_residual = true;
  });
}

extern "C" int msim_binary_set_rescore_limbs(msim_binary_docs* h, int limbs) {
  return guarded([&] {
    require_handle(h);
    if (limbs != 1 && limbs != 3) throw InvalidArgument("rescore limbs must be 1 (int8 query) or 3 (fp32 query)");
    h->rescore_limbs = limbs;
  });
}

extern "C" int msim_binary_get_rescore_limbs(const msim_binary_docs* h, int* limbs) {
  return guarded([&] {
    require_handle(h);
    if (limbs == nullptr) throw InvalidArgument("limbs must not be null");
    *limbs = h->rescore_limbs;
  });
}

extern "C" int msim_binary_clear_residual(msim_binary_docs* h) {
  return guarded([&] {
    require_handle(h);
    h->has_residual = false;
  });
}

extern "C" int msim_binary_binres_score(msim_binary_docs* h, const float* query, int64_t batch,
                                        int64_t query_tokens, int64_t dim, int fused, const int64_t* candidates,
                                        int64_t num_candidates, float* out) {
  return guarded([&] {
    require_handle(h);
    check_binary_query(h, batch, query_tokens, dim);
    const DocStreams s = binres_streams(h, fused != 0);
    if (candidates) {
      if (num_candidates < 0) throw InvalidArgument("candidate_indices must have shape [batch, candidates]");
      check_candidates(candidates, batch * num_candidates, h->num_docs);
    }
    const int64_t targets = candidates ? num_candidates : h->num_docs;
    if (batch == 0 || targets == 0) return;
    select_device(h->device);
    QueryInput qi;
    qi.d_query = stage_query(h->ws, query, batch * query_tokens, dim);
    qi.limbs = fused ? h->rescore_limbs : 1;
    Targets t{candidates, num_candidates, candidates != nullptr};
    h->scores.ensure(sizeof(float) * batch * targets, "hipMalloc score cache");
    // Prefix scores of every document: the scan a cascade's prefix pass uses.
    const bool scanned = !fused && !candidates && g_scan_prefix &&
                         binres_scan_prefix(h, qi.d_query, batch, query_tokens, h->scores.as<float>(), nullptr);
    if (!scanned)
      run_generic_score(h->ws, h->host_offsets, h->num_tokens, s, qi, kRedMax, 1.0f, batch, query_tokens, nullptr, t,
                        h->scores.as<float>(), targets, nullptr, nullptr);
    copy_scores_out(h->ws, out, h->scores.ptr, sizeof(float) * batch * targets);
  });
}

extern "C" int msim_binary_binres_topk(msim_binary_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                                       int64_t dim, int64_t k, float* out_scores, int64_t* out_indices) {
  return guarded([&] {
    require_handle(h);
    check_binary_query(h, batch, query_tokens, dim);
    check_k(k, h->num_docs);
    const DocStreams s = binres_streams(h, true);
    if (batch == 0) return;
    select_device(h->device);
    QueryInput qi;
    qi.d_query = stage_query(h->ws, query, batch * query_tokens, dim);
    qi.limbs = h->rescore_limbs;
    h->scores.ensure(sizeof(float) * batch * h->num_docs, "hipMalloc score cache");
    run_generic_score(h->ws, h->host_offsets, h->num_tokens, s, qi, kRedMax, 1.0f, batch, query_tokens, nullptr,
                      Targets{}, h->scores.as<float>(), h->num_docs, nullptr, nullptr);
    const HostTopk out(h->ws, batch, k);
    check_hip(launch_topk(h->scores.as<float>(), batch, h->num_docs, h->num_docs, k, nullptr, out.s, out.i, nullptr),
              "launch topk selection kernel");
    out.finish(out_scores, out_indices, nullptr);
  });
}

extern "C" int msim_binary_cascade_topk(msim_binary_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                                        int64_t dim, int64_t k, int64_t candidates, float* out_scores,
                                        int64_t* out_indices) {
  return guarded([&] {
    require_handle(h);
    check_binary_query(h, batch, query_tokens, dim);
    check_cascade(k, candidates, h->num_docs);
    binres_streams(h, true);
    if (batch == 0) return;
    select_device(h->device);
    const float* d_query = stage_query(h->ws, query, batch * query_tokens, dim);
    const HostTopk out(h->ws, batch, k);
    binres_cascade(h, d_query, batch, query_tokens, k, candidates, out.s, out.i, nullptr);
    out.finish(out_scores, out_indices, nullptr);
  });
}

extern "C" int msim_binary_cascade_topk_async(msim_binary_docs* h, const float* d_query, int64_t batch,
                                              int64_t query_tokens, int64_t k, int64_t candidates, float* d_scores,
                                              int64_t* d_indices, void* stream) {
  return guarded([&] {
    require_handle(h);
    require_shape(batch, query_tokens);
    check_cascade(k, candidates, h->num_docs);
    binres_streams(h, true);
    if (batch == 0) return;
    select_device(h->device);
    binres_cascade(h, d_query, batch, query_tokens, k, candidates, d_scores, d_indices, as_stream(stream));
  });
}

// ------------------------------------------------- device-resident forms

extern "C" int msim_int4_score_async(msim_int4_docs* h, const float* d_query, int64_t batch, int64_t query_tokens,
                                     const char* reducer, const float* weights, int64_t weights_ndim,
                                     int64_t weights_dim0, int64_t weights_dim1, double temperature, int residual,
                                     float* d_out, void* stream) {
  return guarded([&] {
    require_handle(h);
    if (h->dim != 128) throw InvalidArgument("device-resident scoring currently requires dim=128");
    require_shape(batch, query_tokens);
    const int red = parse_reducer(reducer);
    check_temperature(temperature);
    const std::vector<float> w =
        row_weights(reducer, weights, weights_ndim, weights_dim0, weights_dim1, batch, query_tokens);
    if (batch == 0 || h->num_docs == 0) return;
    select_device(h->device);
    const DocStreams s = int4_streams(h, residual != 0);
    QueryInput qi;
    qi.d_query = d_query;
    qi.limbs = 3;
    run_generic_score(h->ws, h->host_offsets, h->num_tokens, s, qi, red, (float)temperature, batch, query_tokens,
                      w.empty() ? nullptr : w.data(), Targets{}, d_out, h->num_docs, nullptr, as_stream(stream));
  });
}

// ------------------------------------------- top-k under any reducer

extern "C" int msim_int4_topk_score(msim_int4_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                                    int64_t dim, int64_t k, const char* reducer, const float* weights,
                                    int64_t weights_ndim, int64_t weights_dim0, int64_t weights_dim1,
                                    double temperature, int residual, float* out_scores, int64_t* out_indices) {
  return guarded([&] {
    require_handle(h);
    check_k(k, h->num_docs);
    check_dim(dim, h->dim);
    require_shape(batch, query_tokens);
    const int red = parse_reducer(reducer);
    check_temperature(temperature);
    const std::vector<float> w =
        row_weights(reducer, weights, weights_ndim, weights_dim0, weights_dim1, batch, query_tokens);
    if (residual && !h->has_residual)
      throw InvalidArgument("residual int4 data was requested but is not loaded on this CUDA handle");
    if (batch == 0) return;
    select_device(h->device);
    float* d = int4_score_device(h, query, batch, query_tokens, dim, red, w, (float)temperature, nullptr, 0,
                                 residual != 0, nullptr);
    const HostTopk out(h->ws, batch, k);
    check_hip(launch_topk(d, batch, h->num_docs, h->num_docs, k, nullptr, out.s, out.i, nullptr),
              "launch topk selection kernel");
    out.finish(out_scores, out_indices, nullptr);
  });
}

extern "C" int msim_binary_topk_score(msim_binary_docs* h, const float* query, int64_t batch, int64_t query_tokens,
                                      int64_t dim, int64_t k, const char* reducer, const float* weights,
                                      int64_t weights_ndim, int64_t weights_dim0, int64_t weights_dim1,
                                      double temperature, double scale, int use_scale_vector, int use_token_scale,
                                      const float* scale_vector_override, float* out_scores, int64_t* out_indices) {
  return guarded([&] {
    require_handle(h);
    check_k(k, h->num_docs);
    check_binary_query(h, batch, query_tokens, dim);
    const int red = parse_reducer(reducer);
    check_temperature(temperature);
    const std::vector<float> w =
        row_weights(reducer, weights, weights_ndim, weights_dim0, weights_dim1, batch, query_tokens);
    if (batch == 0) return;
    select_device(h->device);
    const float* d_override = nullptr;
    if (scale_vector_override) {
      std::vector<float> v(scale_vector_override, scale_vector_override + h->num_docs);
      d_override = upload_vec(h->scale_override, v, "copy scale vector override to device");
    }
    const DocStreams s = binary_streams(h, scale, use_scale_vector, use_token_scale, d_override);
    float* d = binary_score_device(h, query, batch, query_tokens, dim, 3, false, s, red, w, (float)temperature,
                                   nullptr, 0);
    copy_topk_out(h, d, batch, k, out_scores, out_indices, nullptr);
  });
}
