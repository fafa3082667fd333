// cascade.hip -- device-side pieces of the coarse -> candidates -> rescoring
// cascade (reference: cascade_topk cascade.py:294-393, whose coarse
// selection, per-row candidate rescoring and stable top-k run on the host):
// the candidate lists stay on the device, are put in document order, and the
// rescoring kernel's tile tables are written from them on the device.
#include "common.hpp"
#include "internal.hpp"
#include "topk_block.hpp"

namespace msim {

namespace {

constexpr uint64_t kEntryStartMask = 0xFFFFFFFFFFull;

__device__ __forceinline__ uint64_t tile_entry(int64_t start, int64_t rows, bool last, bool empty, int64_t local) {
  return ((uint64_t)start & kEntryStartMask) | ((uint64_t)(rows - 1) << 40) | ((uint64_t)last << 45) |
         ((uint64_t)empty << 46) | ((uint64_t)local << 48);
}

// One thread per (group, wave): the wave's candidates [t0, t0 + n) with
// n <= per_wave, and their tiles at tiles[(g * waves + w) * cap ...]; the
// host sizes cap as per_wave * (largest document's tile count) + 1.
__global__ __launch_bounds__(256) void candidate_tables_kernel(const int64_t* __restrict__ cands, int64_t m,
                                                               int64_t groups, const int64_t* __restrict__ offsets,
                                                               int64_t waves, int64_t per_wave, int64_t cap,
                                                               int64_t* __restrict__ info,
                                                               uint64_t* __restrict__ tiles) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= groups * waves) return;
  const int64_t g = id / waves, w = id % waves;
  const int64_t t0 = min(w * per_wave, m);
  const int64_t n = min(per_wave, m - t0);
  const int64_t tab0 = id * cap;
  uint64_t* out = tiles + tab0;
  int64_t k = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t doc = cands[g * m + t0 + i];
    const int64_t s = offsets[doc], e = offsets[doc + 1];
    if (s == e) {
      out[k++] = tile_entry(0, 1, true, true, i);
      continue;
    }
    for (int64_t x = s; x < e; x += 16) out[k++] = tile_entry(x, min<int64_t>(16, e - x), x + 16 >= e, false, i);
  }
  out[k] = tile_entry(0, 1, false, false, 0);
  int64_t* row = info + id * kScoreInfoWords;
  row[0] = t0;
  row[1] = n;
  row[2] = k;
  row[3] = tab0;
}

// Ascending bitonic sort of s[0, pow2) in LDS by the whole block.
template <typename T>
__device__ void bitonic_sort(T* s, int pow2) {
  for (int size = 2; size <= pow2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < pow2; i += blockDim.x) {
        const int j = i ^ stride;
        if (j > i) {
          const bool up = (i & size) == 0;
          const T a = s[i], b = s[j];
          if ((a > b) == up) {
            s[i] = b;
            s[j] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Ascending sort of each row of n <= 4096 int64 values (bitonic, in LDS).
__global__ __launch_bounds__(1024) void sort_rows_kernel(int64_t* __restrict__ rows, int64_t n, int64_t pow2) {
  __shared__ int64_t s[kSortMaxRow];
  int64_t* row = rows + (int64_t)blockIdx.x * n;
  for (int64_t i = threadIdx.x; i < pow2; i += blockDim.x) s[i] = i < n ? row[i] : INT64_MAX;
  __syncthreads();
  bitonic_sort(s, (int)pow2);
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) row[i] = s[i];
}

// Per row of n <= 4096 scores: the m best by (score desc, position asc)
// (the order of _stable_topk, cascade.py:420-453), written as positions in
// ascending order.  One sort of (descending score key, position) pairs, then
// one sort of the m selected positions.
__global__ __launch_bounds__(1024) void select_topm_kernel(const float* __restrict__ scores, int64_t n,
                                                           int64_t stride, int64_t m, int pow2, int pow2m,
                                                           int64_t* __restrict__ out) {
  __shared__ uint64_t keys[kSortMaxRow];
  __shared__ uint32_t ids[kSortMaxRow];
  const float* row = scores + (int64_t)blockIdx.x * stride;
  for (int i = threadIdx.x; i < pow2; i += blockDim.x)
    keys[i] = i < n ? ((uint64_t)(~score_key(row[i])) << 32) | (uint32_t)i : ~0ull;
  __syncthreads();
  bitonic_sort(keys, pow2);
  for (int i = threadIdx.x; i < pow2m; i += blockDim.x) ids[i] = i < m ? (uint32_t)keys[i] : 0xFFFFFFFFu;
  __syncthreads();
  bitonic_sort(ids, pow2m);
  for (int i = threadIdx.x; i < m; i += blockDim.x) out[(int64_t)blockIdx.x * m + i] = ids[i];
}

}  // namespace

hipError_t launch_candidate_tables(const int64_t* d_cands, int64_t m, int64_t groups, const int64_t* d_offsets,
                                   int64_t waves, int64_t per_wave, int64_t cap, int64_t* d_info,
                                   uint64_t* d_tiles, hipStream_t stream) {
  const int64_t n = groups * waves;
  if (n <= 0) return hipSuccess;
  candidate_tables_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream>>>(
      d_cands, m, groups, d_offsets, waves, per_wave, cap, d_info, d_tiles);
  return hipGetLastError();
}

hipError_t launch_select_topm(const float* d_scores, int64_t batch, int64_t n, int64_t stride, int64_t m,
                              int64_t* d_out, hipStream_t stream) {
  if (batch <= 0 || m <= 0) return hipSuccess;
  if (n > kSortMaxRow || m > n) return hipErrorInvalidValue;
  int pow2 = 1, pow2m = 1;
  while (pow2 < n) pow2 <<= 1;
  while (pow2m < m) pow2m <<= 1;
  select_topm_kernel<<<dim3((unsigned)batch), dim3(1024), 0, stream>>>(d_scores, n, stride, m, pow2, pow2m, d_out);
  return hipGetLastError();
}

hipError_t launch_sort_rows(int64_t* d_rows, int64_t batch, int64_t n, hipStream_t stream) {
  if (batch <= 0 || n <= 1) return hipSuccess;
  if (n > kSortMaxRow) return hipErrorInvalidValue;
  int64_t pow2 = 1;
  while (pow2 < n) pow2 <<= 1;
  sort_rows_kernel<<<dim3((unsigned)batch), dim3(1024), 0, stream>>>(d_rows, n, pow2);
  return hipGetLastError();
}

}  // namespace msim
