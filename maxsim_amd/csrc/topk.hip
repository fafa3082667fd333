// topk.hip -- stand-alone block top-k: one 1024-thread workgroup per score row.
// Selection algorithm and order: topk_block.hpp (reference order cu:1629-1692,
// _api.py:732-735).
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
