// capi_pack.cpp -- C ABI of the device int4 packer (pack.hip): the
// reference's pack_int4_symmetric (experimental.py:218-268) with its argument
// checks and error messages, on the GPU.
#include <cmath>
#include <cstring>

#include "capi_internal.hpp"

namespace msim {
hipError_t launch_int4_absmax(const float* d_x, int64_t num_tokens, int dim, uint32_t* d_work, int num_cus,
                              hipStream_t stream);
hipError_t launch_pack_int4(const float* d_x, int64_t num_tokens, int dim, bool token, double given_scale,
                            uint32_t* d_work, uint8_t* d_codes, float* d_token_scale, int8_t* d_values,
                            int num_cus, hipStream_t stream);
}

using namespace msim;

namespace {

constexpr const char* kNotFinite = "doc_embeddings must contain only finite values";

void check_shape(int64_t num_tokens, int dim) {
  if (num_tokens < 0) throw InvalidArgument("doc_embeddings must have shape [num_doc_tokens, dim]");
  if (dim <= 0) throw InvalidArgument("dim must be positive");
  if (dim % 2 != 0) throw InvalidArgument("dim must be divisible by 2 for int4 packing");
  if (dim % 8 != 0) throw InvalidArgument("dim must be divisible by 8");
}

// experimental.py:236-254, in the reference's order (after the finiteness check).
void check_scale_args(int token_granularity, double scale) {
  if (token_granularity != 0 && token_granularity != 1)
    throw InvalidArgument("scale_granularity must be 'tensor' or 'token'");
  if (token_granularity == 1 && scale != 0.0)
    throw InvalidArgument("scale cannot be provided when scale_granularity='token'");
  if (token_granularity == 0 && scale != 0.0 && !(std::isfinite(scale) && scale > 0.0))
    throw InvalidArgument("scale must be finite and > 0");
}

}  // namespace

extern "C" int msim_pack_int4_async(const float* d_x, int64_t num_tokens, int dim, int token_granularity,
                                    double scale, uint8_t* d_codes, float* d_token_scales, int8_t* d_values,
                                    uint32_t* d_work, void* stream) {
  return guarded([&] {
    check_shape(num_tokens, dim);
    check_scale_args(token_granularity, scale);
    if (d_work == nullptr) throw InvalidArgument("work must point to 2 device words");
    if (num_tokens > 0 && (d_x == nullptr || d_codes == nullptr || (token_granularity == 1 && d_token_scales == nullptr)))
      throw InvalidArgument("input and output pointers must not be NULL");
    if (reinterpret_cast<uintptr_t>(d_x) % 16 != 0 || (d_values && reinterpret_cast<uintptr_t>(d_values) % 2 != 0))
      throw InvalidArgument("embeddings must be 16-byte aligned (values 2-byte aligned)");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    check_hip(launch_fill_f32(reinterpret_cast<float*>(d_work), 2, 0.0f, s), "zero pack work words");
    // Tensor granularity: max |x| first (also flags non-finite values);
    // token granularity: the pack kernel flags them itself.
    if (token_granularity == 0)
      check_hip(launch_int4_absmax(d_x, num_tokens, dim, d_work, device_cu_count(), s), "launch int4 absmax kernel");
    check_hip(launch_pack_int4(d_x, num_tokens, dim, token_granularity == 1, scale, d_work, d_codes, d_token_scales,
                               d_values, device_cu_count(), s),
              "launch int4 pack kernels");
  });
}

extern "C" int msim_pack_int4(const float* x, int64_t num_tokens, int dim, int token_granularity, double scale,
                              uint8_t* codes, float* token_scales, int8_t* values, double* scale_out) {
  return guarded([&] {
    check_shape(num_tokens, dim);
    if (num_tokens > 0 && (x == nullptr || codes == nullptr)) throw InvalidArgument("input and output pointers must not be NULL");
    const size_t n = (size_t)num_tokens * (size_t)dim;
    DeviceBuffer dx, dcodes, dscales, dvalues, dwork;
    dwork.ensure(256, "hipMalloc pack work words");
    uint32_t work[2] = {0, 0};
    if (num_tokens > 0) {
      dx.ensure(n * sizeof(float), "hipMalloc pack input");
      check_hip(hipMemcpy(dx.ptr, x, n * sizeof(float), hipMemcpyHostToDevice), "copy embeddings to device");
      // Finiteness first (the reference checks it before the scale arguments).
      check_hip(launch_fill_f32(dwork.as<float>(), 2, 0.0f, nullptr), "zero pack work words");
      check_hip(launch_int4_absmax(dx.as<float>(), num_tokens, dim, dwork.as<uint32_t>(), device_cu_count(), nullptr),
                "launch int4 absmax kernel");
      check_hip(hipMemcpy(work, dwork.ptr, sizeof work, hipMemcpyDeviceToHost), "read pack work words");
      if (work[1] != 0) throw InvalidArgument(kNotFinite);
    }
    check_scale_args(token_granularity, scale);
    const bool token = token_granularity == 1;
    if (token && num_tokens > 0 && token_scales == nullptr) throw InvalidArgument("token_scales must not be NULL");
    double scale_value = 1.0;
    if (!token) {
      float peak = 0.0f;
      std::memcpy(&peak, &work[0], sizeof peak);
      scale_value = scale != 0.0 ? scale : (peak == 0.0f ? 1.0 : (double)peak / 7.0);
    }
    if (num_tokens > 0) {
      dcodes.ensure(n / 2, "hipMalloc pack codes");
      if (token) dscales.ensure((size_t)num_tokens * sizeof(float), "hipMalloc pack token scales");
      if (values) dvalues.ensure(n, "hipMalloc pack values");
      // The tensor scale computed on the host above is passed explicitly.
      check_hip(launch_pack_int4(dx.as<float>(), num_tokens, dim, token, token ? 0.0 : scale_value,
                                 dwork.as<uint32_t>(), dcodes.as<uint8_t>(), dscales.as<float>(),
                                 values ? dvalues.as<int8_t>() : nullptr, device_cu_count(), nullptr),
                "launch int4 pack kernels");
      check_hip(hipMemcpy(codes, dcodes.ptr, n / 2, hipMemcpyDeviceToHost), "copy codes to host");
      if (token)
        check_hip(hipMemcpy(token_scales, dscales.ptr, (size_t)num_tokens * sizeof(float), hipMemcpyDeviceToHost),
                  "copy token scales to host");
      if (values) check_hip(hipMemcpy(values, dvalues.ptr, n, hipMemcpyDeviceToHost), "copy values to host");
    }
    if (scale_out) *scale_out = scale_value;
  });
}
