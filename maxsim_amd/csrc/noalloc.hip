// noalloc.hip -- msim_int4_topk_int8q_noalloc: the int8-query search of
// msim_int4_topk_int8q_async with its scratch memory (quantised query, score
// rows of an unfused call, the fused selection's key rows, workgroup records
// and launch counter) in one fixed device array instead of handle workspaces, so
// a call allocates nothing.  For callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops).
//
// The array `scratch` is a file-scope __device__ object: every GPU the
// library runs on holds its own copy, at its own address, until the process
// ends, zero-initialised when the code object loads.  Host code never names
// it after set-up: the first call on a device looks its address up with
// hipGetSymbolAddress (with that device current) and keeps it per device.
// Every call on a GPU shares that GPU's array and leaves its contents
// behind; calls that overlap on one GPU (different streams, or different
// host threads) race on it.  The launch counter only grows, so entries left
// by earlier calls (of any handle) carry older tags than the current launch.
#include <mutex>

#include "capi_handles.hpp"

namespace msim {
namespace {

constexpr int64_t kNoallocMaxRows = 128;                     // batch * query_tokens per call
constexpr int64_t kNoallocQueryRows = kNoallocMaxRows + 128;  // padded rows the scan may read
constexpr int64_t kNoallocScoreFloats = kScanTailMaxRows * kScanTailRow;  // 32,768 scores
constexpr size_t kQpackOff = 0;
constexpr size_t kQscaleOff = kQpackOff + kNoallocQueryRows * 128;
constexpr size_t kQbiasOff = kQscaleOff + kNoallocQueryRows * 4;
constexpr size_t kScoresOff = kQbiasOff + kNoallocQueryRows * 4;  // score rows of an unfused call
constexpr size_t kKeysOff = kScoresOff + kNoallocScoreFloats * 4;  // fused: key rows
constexpr size_t kRecOff = kKeysOff + kScanTailMaxRows * kScanTailRow * 8;  // fused: workgroup records
constexpr size_t kEpochOff = kRecOff + kScanTailMaxRows * 3 * kScanTailBlocks * 8;  // fused: launch counter
constexpr size_t kScratchBytes = kEpochOff + 256;  // 526,592 bytes
static_assert(kScoresOff % 256 == 0 && kKeysOff % 256 == 0 && kRecOff % 256 == 0 && kEpochOff % 256 == 0,
              "aligned scratch regions");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
unsigned char* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's `scratch`, looked up at the first call on
// the device.
unsigned char* scratch_on(int device) {
  if (device < 0 || device >= kMaxDevices) throw RuntimeError("device ordinal out of range for the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr) throw RuntimeError("hipGetSymbolAddress(scratch) returned no address");
    g_scratch_ptr[device] = static_cast<unsigned char*>(ptr);
  }
  return g_scratch_ptr[device];
}

}  // namespace
}  // namespace msim

using namespace msim;

extern "C" int msim_int4_topk_int8q_noalloc(msim_int4_docs* h, const float* d_query, int64_t batch,
                                            int64_t query_tokens, int64_t k, float* d_scores,
                                            int64_t* d_indices, void* stream) {
  return guarded([&] {
    require_handle(h);
    if (k < 1 || k > h->num_docs) throw InvalidArgument("k must be between 1 and num_docs");
    if (h->dim != 128) throw InvalidArgument("int8 query scoring currently requires dim=128");
    require_shape(batch, query_tokens);
    if (batch == 0) return;
    const int64_t rows = batch * query_tokens;
    if (query_tokens == 0 || rows > kNoallocMaxRows)
      throw InvalidArgument("msim_int4_topk_int8q_noalloc takes 1 to 128 query rows (batch * query_tokens)");
    if (k > kScanTailMaxK) throw InvalidArgument("msim_int4_topk_int8q_noalloc takes k <= 32");
    const int64_t n = h->num_docs;
    const int mode = msim_get_fused_topk();
    const bool fused = mode != 0 && n >= kScanTailMinDocs && n <= kScanTailMaxDocs && batch <= kScanTailMaxRows &&
                       h->num_scan_waves <= (int64_t)kScanWavesPerGroup * kScanTailBlocks;
    if (!fused && batch * n > kNoallocScoreFloats)
      throw InvalidArgument(
          "msim_int4_topk_int8q_noalloc holds batch * num_docs <= 32768 scores unless the scan selects the top-k "
          "itself (256 <= num_docs <= 4096, batch <= 8)");
    if (!scan_tables_current(h))
      throw InvalidArgument(
          "the scan tables of this handle were built for other partition settings: make one "
          "msim_int4_topk_int8q_async call to rebuild them");
    check_hip(hipSetDevice(h->device), "hipSetDevice");
    const hipStream_t s = as_stream(stream);
    unsigned char* base = scratch_on(h->device);
    auto* qpack = reinterpret_cast<int8_t*>(base + kQpackOff);
    auto* qscale = reinterpret_cast<float*>(base + kQscaleOff);
    auto* qbias = reinterpret_cast<int32_t*>(base + kQbiasOff);
    auto* scores = reinterpret_cast<float*>(base + kScoresOff);
    const int64_t rows_padded = ((rows + 15) / 16) * 16 + 128;
    check_hip(launch_quantize_int8(d_query, rows, rows_padded, qpack, qscale, qbias, s, scan_pass_rows(query_tokens)),
              "launch int8 query quantize kernel");
    ScanArgs a{};
    scan_corpus_args(h, query_tokens, a);
    a.qpack = qpack;
    a.qscale = qscale;
    a.batch = (int32_t)batch;
    if (fused) {
      a.tail_keys = reinterpret_cast<uint64_t*>(base + kKeysOff);
      a.tail_rec = reinterpret_cast<uint64_t*>(base + kRecOff);
      a.tail_key_words = kScanTailMaxRows * kScanTailRow;
      a.topk_k = (int32_t)k;
      a.tail_cap = mode == 2 ? 0 : INT32_MAX;
      a.epoch = reinterpret_cast<uint32_t*>(base + kEpochOff);
      a.tail_wait_ticks = msim_get_fused_wait_ticks();
      a.top_scores = d_scores;
      a.top_ids = d_indices;
    }
    if (!fused) a.scores = scores;
    check_hip(launch_int8q_scan(a, scan_epilogue(h), s), "launch int8q scan kernel");
    if (!fused)
      check_hip(launch_topk(scores, batch, n, n, k, nullptr, d_scores, d_indices, s),
                "launch int8q topk selection kernel");
  });
}
