// util.hip -- small device utilities (fills used instead of hipMemsetAsync so
// that every enqueued operation is a kernel and capturable in a HIP graph).
#include "capi_internal.hpp"
#include "common.hpp"

namespace msim {

__global__ void fill_f32_kernel(float* __restrict__ d, int64_t n, float value) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) d[i] = value;
}

hipError_t launch_fill_f32(float* d, int64_t n, float value, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  fill_f32_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(d, n, value);
  return hipGetLastError();
}

}  // namespace msim
