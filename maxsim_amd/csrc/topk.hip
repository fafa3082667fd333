// topk.hip -- block-level top-k selection over score rows.
//
// Order restated from the reference: score descending, then document id
// ascending (cu:1629-1692 selection order; _api.py:732-735 lexsort).
//
// Design: one 1024-thread workgroup per row.  Scores map to order-preserving
// 32-bit keys; four 8-bit radix passes (LDS histograms) find the k-th largest
// key T.  Every key above T is kept, and among the keys equal to T the
// lowest positions are kept (a block prefix count over contiguous per-thread
// chunks gives position order).  The k survivors are ranked by counting
// (key desc, position asc) in LDS and written in order.  Work is O(n) per
// row plus O(k^2 / 1024) per thread for the final ranking.
#include "common.hpp"
#include "internal.hpp"

namespace msim {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / kWave;

__device__ __forceinline__ uint32_t score_key(float s) {
  if (s == 0.0f) s = 0.0f;  // -0 and +0 compare equal in the reference order
  const uint32_t u = __float_as_uint(s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Block-wide exclusive prefix sum of one value per thread.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_wave, uint32_t* total) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  uint32_t incl = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint32_t o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  if (lane == kWave - 1) s_wave[wave] = incl;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (int w = 0; w < kTopkWaves; ++w) {
      const uint32_t t = s_wave[w];
      s_wave[w] = run;
      run += t;
    }
    *total = run;
  }
  __syncthreads();
  return s_wave[wave] + incl - v;
}

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float* __restrict__ scores,
                                                           int64_t n, int64_t row_stride, int32_t k,
                                                           const int64_t* __restrict__ id_map,
                                                           float* __restrict__ out_scores,
                                                           int64_t* __restrict__ out_ids) {
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_wave[kTopkWaves];
  __shared__ uint32_t s_total;
  __shared__ uint32_t s_digit, s_kk, s_count;
  __shared__ uint32_t s_key[kTopkMaxK];
  __shared__ int32_t s_pos[kTopkMaxK];

  const int64_t b = blockIdx.x;
  const float* row = scores + b * row_stride;
  const int tid = threadIdx.x;
  const int64_t per = (n + kTopkThreads - 1) / kTopkThreads;
  const int64_t lo = min((int64_t)tid * per, n);
  const int64_t hi = min(lo + per, n);

  uint32_t prefix = 0, mask = 0, kk = (uint32_t)k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += kTopkThreads) s_hist[i] = 0;
    __syncthreads();
    for (int64_t i = lo; i < hi; ++i) {
      const uint32_t key = score_key(row[i]);
      if ((key & mask) == prefix) atomicAdd(&s_hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < kWave) {
      // Lane l owns digits 255-4l .. 252-4l (descending).
      const int lane = tid;
      uint32_t c[4];
      uint32_t local = 0;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        c[x] = s_hist[255 - 4 * lane - x];
        local += c[x];
      }
      uint32_t incl = local;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
      }
      uint32_t above = incl - local;  // elements with a larger digit
      if (above < kk && kk <= incl) {
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          if (above < kk && kk <= above + c[x]) {
            s_digit = (uint32_t)(255 - 4 * lane - x);
            s_kk = kk - above;
          }
          above += c[x];
        }
      }
    }
    __syncthreads();
    prefix |= s_digit << shift;
    mask |= 255u << shift;
    kk = s_kk;
    __syncthreads();
  }
  // prefix is the k-th largest key; kk of the keys equal to it are kept.
  uint32_t my_ties = 0;
  for (int64_t i = lo; i < hi; ++i) my_ties += score_key(row[i]) == prefix ? 1u : 0u;
  const uint32_t tie_base = block_exclusive_scan(my_ties, s_wave, &s_total);
  if (tid == 0) s_count = 0;
  for (int e = tid; e < k; e += kTopkThreads) {
    s_key[e] = 0;
    s_pos[e] = 0;
  }
  __syncthreads();
  uint32_t tie_rank = tie_base;
  for (int64_t i = lo; i < hi; ++i) {
    const uint32_t key = score_key(row[i]);
    bool keep = key > prefix;
    if (key == prefix) {
      keep = tie_rank < kk;
      ++tie_rank;
    }
    if (keep) {
      const uint32_t slot = atomicAdd(&s_count, 1u);
      if (slot < (uint32_t)k) {
        s_key[slot] = key;
        s_pos[slot] = (int32_t)i;
      }
    }
  }
  __syncthreads();
  for (int e = tid; e < k; e += kTopkThreads) {
    const uint32_t key = s_key[e];
    const int32_t pos = min(max(s_pos[e], 0), (int32_t)(n - 1));
    int rank = 0;
    for (int o = 0; o < k; ++o) {
      const uint32_t ok = s_key[o];
      rank += (ok > key || (ok == key && s_pos[o] < pos)) ? 1 : 0;
    }
    out_scores[b * k + rank] = row[pos];
    out_ids[b * k + rank] = id_map ? id_map[b * n + pos] : (int64_t)pos;
  }
}

hipError_t launch_topk(const float* d_scores, int64_t batch, int64_t n, int64_t row_stride,
                       int64_t k, const int64_t* d_id_map, float* d_out_scores,
                       int64_t* d_out_ids, hipStream_t stream) {
  if (batch == 0 || k == 0) return hipSuccess;
  if (k > kTopkMaxK || k > n) return hipErrorInvalidValue;
  topk_kernel<<<dim3((unsigned)batch), dim3(kTopkThreads), 0, stream>>>(
      d_scores, n, row_stride, (int32_t)k, d_id_map, d_out_scores, d_out_ids);
  return hipGetLastError();
}

}  // namespace msim
