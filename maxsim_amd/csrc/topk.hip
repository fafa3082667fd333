// topk.hip -- stand-alone block top-k: one 1024-thread workgroup per score row.
// Selection algorithm and order: topk_block.hpp (reference order cu:1629-1692,
// _api.py:732-735).
#include "common.hpp"
#include "internal.hpp"
#include "topk_block.hpp"

namespace msim {

constexpr int kTopkThreads = 1024;

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float* __restrict__ scores,
                                                           int64_t n, int64_t row_stride, int32_t k,
                                                           const int64_t* __restrict__ id_map,
                                                           float* __restrict__ out_scores,
                                                           int64_t* __restrict__ out_ids) {
  __shared__ TopkSmem<kTopkThreads, kTopkMaxK> sm;
  const int64_t b = blockIdx.x;
  block_topk<kTopkThreads, 16, kTopkMaxK>(scores + b * row_stride, n, k,
                                          id_map ? id_map + b * n : nullptr, out_scores + b * k,
                                          out_ids + b * k, sm);
}

// ------------------------------------------------------------- small k
// k <= kSmallTopkMaxK and n <= THREADS * kSmallEPT: every element stays in
// registers as a 64-bit key (order-preserving score bits above the inverted
// position, so a larger key is a higher score or, on a tie, a lower
// position) and the k results come from k rounds of a block-wide maximum.
constexpr int kSmallTopkMaxK = 32;
constexpr int kSmallEPT = 16;

// Maximum of a 32-bit value over the wave (wave-uniform), DPP only.
__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Sorts a lane's E keys into descending order (odd-even transposition
// network, E rounds of independent compare-exchanges).
template <int E>
__device__ __forceinline__ void lane_sort_desc(uint64_t (&key)[E]) {
#pragma unroll
  for (int round = 0; round < E; ++round) {
#pragma unroll
    for (int i = round & 1; i + 1 < E; i += 2) {
      const uint64_t a = key[i], b = key[i + 1];
      key[i] = a > b ? a : b;
      key[i + 1] = a > b ? b : a;
    }
  }
}

// The k largest of the keys held by the wave (E per lane), largest first,
// into out[0..k) (lane 0 writes).  Keys of 0 are empty slots.  Each lane's
// keys are sorted first, so a round is one wave maximum over the lanes'
// heads plus a shift in the winning lane; only a tie on the score half
// needs the full 64-bit reduction.
template <int E>
__device__ __forceinline__ void wave_select(uint64_t (&key)[E], int k, uint64_t* out) {
  lane_sort_desc(key);
  for (int r = 0; r < k; ++r) {
    const uint64_t head = key[0];
    const uint32_t hs = (uint32_t)(head >> 32);
    const uint32_t top = wave_max_u32_dpp(hs);
    const uint64_t holders = __ballot(hs == top);
    uint64_t best;
    if (__popcll(holders) == 1) {
      const int owner = __ffsll((unsigned long long)holders) - 1;
      best = ((uint64_t)top << 32) | (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)head, owner);
    } else {
      best = wave_max_u64(head);
    }
    if (lane_id() == 0) out[r] = best;
    if (best != 0 && head == best) {  // the one lane holding it drops it
#pragma unroll
      for (int e = 0; e + 1 < E; ++e) key[e] = key[e + 1];
      key[E - 1] = 0u;
    }
  }
}

// One workgroup per row: each wave selects the k best of its kWave * kSmallEPT
// elements, then wave 0 selects the k best of those candidates.  No
// workgroup barrier inside the selection rounds.
template <int THREADS>
__global__ __launch_bounds__(THREADS) void topk_small_kernel(const float* __restrict__ scores, int64_t n,
                                                            int64_t row_stride, int32_t k,
                                                            const int64_t* __restrict__ id_map,
                                                            float* __restrict__ out_scores,
                                                            int64_t* __restrict__ out_ids) {
  constexpr int kWaves = THREADS / kWave;
  __shared__ uint64_t s_cand[kWaves * kSmallTopkMaxK];
  __shared__ uint64_t s_best[kSmallTopkMaxK];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int64_t b = blockIdx.x;
  const float* row = scores + b * row_stride;
  // Bounds-checked loads (positions past n read zero), all issued first.
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(row, (uint32_t)(n * 4));
  const int base = wave * kWave * kSmallEPT + lane;
  float v[kSmallEPT];
#pragma unroll
  for (int e = 0; e < kSmallEPT; ++e) v[e] = __uint_as_float(load_b32(rsrc, (base + e * kWave) * 4));
  uint64_t key[kSmallEPT];
#pragma unroll
  for (int e = 0; e < kSmallEPT; ++e) {
    const int i = base + e * kWave;
    key[e] = i < n ? ((uint64_t)score_key(v[e]) << 32) | (0xFFFFFFFFu - (uint32_t)i) : 0u;
  }
  wave_select(key, k, s_cand + wave * kSmallTopkMaxK);
  __syncthreads();
  // Merge the waves' sorted lists (one thread, k steps over kWaves heads).
  if (tid == 0) {
    int pos[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) pos[w] = 0;
    for (int r = 0; r < k; ++r) {
      uint64_t best = 0;
      int from = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const uint64_t h = pos[w] < k ? s_cand[w * kSmallTopkMaxK + pos[w]] : 0u;
        if (h > best) {
          best = h;
          from = w;
        }
      }
#pragma unroll
      for (int w = 0; w < kWaves; ++w) pos[w] += w == from ? 1 : 0;
      s_best[r] = best;
    }
  }
  __syncthreads();
  if (tid < k) {
    const int64_t pos = (int64_t)(0xFFFFFFFFu - (uint32_t)s_best[tid]);
    out_scores[b * k + tid] = row[pos];
    out_ids[b * k + tid] = id_map ? id_map[b * n + pos] : pos;
  }
}

// ------------------------------------------------------ threshold filter
// k <= kSmallTopkMaxK and n <= kFilterThreads * EPT: four waves, element i of
// the row in thread i % 256 (coalesced loads; the id map, when given, loaded
// beside the scores).  Keys are 64-bit, order-preserving score bits above
// 2^32 - 1 - position, so every key is distinct and a larger key is a higher
// score or, on a tie, a lower position.  In each wave, T_w = the k-th largest
// of the 64 lanes' maximum keys (a radix selection by ballot counts, no
// shuffles): k lanes of the wave hold a key >= T_w, so every key of the row's
// top k is >= T = max_w T_w.  At most k lanes per wave have a maximum >= T,
// so at most 4 * k * EPT keys pass the filter; they go to a list in LDS
// (one atomic per wave for its range, ballot offsets inside it) with their
// float bits and ids, and each one's rank is counted against the list.
// kCap is a multiple of eight.  The key of rank r < k is written to slot r.
constexpr int kFilterThreads = 256;
constexpr int kFilterWaves = kFilterThreads / kWave;

// The k-th largest of the wave's nonzero keys (wave-uniform), 0 when fewer
// than k lanes hold one.  The low 32 bits of every nonzero key are >= 2^32 -
// 4096 (positions below 4096), so those 20 bits of the result need no step.
__device__ __forceinline__ uint64_t wave_kth_largest_key(uint64_t x, int k) {
  if (__popcll(__ballot(x != 0)) < k) return 0;
  uint64_t t = 0;
#pragma unroll
  for (int bit = 63; bit >= 32; --bit) {
    const uint64_t c = t | (1ull << bit);
    t = __popcll(__ballot(x >= c)) >= k ? c : t;
  }
  t |= 0xFFFFF000ull;
#pragma unroll
  for (int bit = 11; bit >= 0; --bit) {
    const uint64_t c = t | (1ull << bit);
    t = __popcll(__ballot(x >= c)) >= k ? c : t;
  }
  return t;
}

template <int EPT>
__global__ __launch_bounds__(kFilterThreads) void topk_filter_kernel(const float* __restrict__ scores, int64_t n,
                                                                     int64_t row_stride, int32_t k,
                                                                     const int64_t* __restrict__ id_map,
                                                                     float* __restrict__ out_scores,
                                                                     int64_t* __restrict__ out_ids) {
  constexpr int kCap = kFilterWaves * kSmallTopkMaxK * EPT;
  static_assert(kCap % 8 == 0, "rank steps of eight keys");
  __shared__ uint64_t s_key[kCap];
  __shared__ int64_t s_id[kCap];
  __shared__ uint32_t s_raw[kCap];
  __shared__ uint64_t s_thr[kFilterWaves];
  __shared__ uint32_t s_count;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int64_t b = blockIdx.x;
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(scores + b * row_stride, (uint32_t)(n * 4));
  const __amdgpu_buffer_rsrc_t rid = make_rsrc(id_map ? id_map + b * n : nullptr, id_map ? (uint32_t)(n * 8) : 0u);
  uint32_t v[EPT];
  int64_t id[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) v[e] = load_b32(rsrc, (e * kFilterThreads + tid) * 4);
  if (id_map) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) id[e] = (int64_t)load_b64(rid, (e * kFilterThreads + tid) * 8);
  }
  if (tid == 0) s_count = 0;
  for (int i = tid; i < kCap; i += kFilterThreads) s_key[i] = 0u;
  uint64_t key[EPT], lmax = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int i = e * kFilterThreads + tid;
    key[e] = i < n ? ((uint64_t)score_key(__uint_as_float(v[e])) << 32) | (0xFFFFFFFFu - (uint32_t)i) : 0u;
    lmax = key[e] > lmax ? key[e] : lmax;
  }
  const uint64_t tw = wave_kth_largest_key(lmax, k);
  if (lane == 0) s_thr[wave] = tw;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int w = 0; w < kFilterWaves; ++w) t = s_thr[w] > t ? s_thr[w] : t;
  uint64_t mask[EPT];
  uint32_t cnt = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    mask[e] = __ballot(key[e] != 0 && key[e] >= t);
    cnt += (uint32_t)__popcll(mask[e]);
  }
  uint32_t base = 0;
  if (lane == 0 && cnt != 0) base = atomicAdd(&s_count, cnt);
  base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if ((mask[e] >> lane) & 1ull) {
      const uint32_t at =
          base + __builtin_amdgcn_mbcnt_hi((uint32_t)(mask[e] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask[e], 0u));
      s_key[at] = key[e];
      s_raw[at] = v[e];
      if (id_map) s_id[at] = id[e];
    }
    base += (uint32_t)__popcll(mask[e]);
  }
  __syncthreads();
  // Ranks, counted against the whole list (broadcast LDS reads, eight keys
  // per step; the zeroed tail pads the list to a multiple of eight).
  const int c = (int)s_count, c8 = (c + 7) & ~7;
  for (int i = tid; i < c; i += kFilterThreads) {
    const uint64_t x = s_key[i];
    int r = 0;
    for (int j = 0; j < c8; j += 8) {
      uint64_t y[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) y[u] = s_key[j + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) r += y[u] > x ? 1 : 0;
    }
    if (r < k) {
      out_scores[b * k + r] = __uint_as_float(s_raw[i]);
      out_ids[b * k + r] = id_map ? s_id[i] : (int64_t)(0xFFFFFFFFu - (uint32_t)x);
    }
  }
}

hipError_t launch_topk(const float* d_scores, int64_t batch, int64_t n, int64_t row_stride,
                       int64_t k, const int64_t* d_id_map, float* d_out_scores,
                       int64_t* d_out_ids, hipStream_t stream) {
  if (batch == 0 || k == 0) return hipSuccess;
  if (k > kTopkMaxK || k > n) return hipErrorInvalidValue;
  if (k <= kSmallTopkMaxK && n <= kFilterThreads * 16) {
    const dim3 grid((unsigned)batch), block(kFilterThreads);
    if (n <= kFilterThreads * 2)
      topk_filter_kernel<2><<<grid, block, 0, stream>>>(d_scores, n, row_stride, (int32_t)k, d_id_map, d_out_scores,
                                                        d_out_ids);
    else if (n <= kFilterThreads * 4)
      topk_filter_kernel<4><<<grid, block, 0, stream>>>(d_scores, n, row_stride, (int32_t)k, d_id_map, d_out_scores,
                                                        d_out_ids);
    else if (n <= kFilterThreads * 8)
      topk_filter_kernel<8><<<grid, block, 0, stream>>>(d_scores, n, row_stride, (int32_t)k, d_id_map, d_out_scores,
                                                        d_out_ids);
    else
      topk_filter_kernel<16><<<grid, block, 0, stream>>>(d_scores, n, row_stride, (int32_t)k, d_id_map, d_out_scores,
                                                         d_out_ids);
  } else if (k <= kSmallTopkMaxK && n <= 1024 * kSmallEPT) {
    topk_small_kernel<1024><<<dim3((unsigned)batch), dim3(1024), 0, stream>>>(
        d_scores, n, row_stride, (int32_t)k, d_id_map, d_out_scores, d_out_ids);
  } else {
    topk_kernel<<<dim3((unsigned)batch), dim3(kTopkThreads), 0, stream>>>(
        d_scores, n, row_stride, (int32_t)k, d_id_map, d_out_scores, d_out_ids);
  }
  return hipGetLastError();
}

}  // namespace msim
