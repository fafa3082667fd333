// capi_internal.hpp -- error plumbing and device buffers behind the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>

#include "../../include/maxsim_hip.h"
#include "internal.hpp"

namespace msim {

struct InvalidArgument : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct RuntimeError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct NotSupported : std::runtime_error {
  using std::runtime_error::runtime_error;
};

extern thread_local std::string g_last_error;
extern int g_docs_per_wave;
extern int g_hamming_fp4;  // sign-query scoring: fp4 Hamming kernel (1) or the int8 MFMA scorer (0)
extern int g_scan_prefix;  // binary-prefix cascades: prefix pass on the int8-query scan
extern uint64_t g_fused_wait_ticks;  // msim_set_fused_wait_ticks

void set_error(const std::string& msg);
void check_hip(hipError_t e, const char* what);
void validate_offsets(const int64_t* offsets, int64_t count, int64_t num_tokens);
void validate_positive_scales(const float* v, int64_t n, const char* msg);
int device_cu_count();
int32_t docs_per_wave_for(int64_t num_docs, int waves_per_cu);
hipStream_t as_stream(void* s);

// Run `fn`, translating exceptions into MSIM_* status codes and the
// thread-local message.
template <typename Fn>
int guarded(Fn&& fn) {
  try {
    fn();
    g_last_error.clear();
    return MSIM_OK;
  } catch (const InvalidArgument& e) {
    set_error(e.what());
    return MSIM_EINVAL;
  } catch (const NotSupported& e) {
    set_error(e.what());
    return MSIM_ENOTSUP;
  } catch (const std::bad_alloc&) {
    set_error("host allocation failed");
    return MSIM_ERUNTIME;
  } catch (const std::exception& e) {
    set_error(e.what());
    return MSIM_ERUNTIME;
  }
}

template <typename H>
void require_handle(const H* h) {
  if (h == nullptr) throw InvalidArgument("handle must not be NULL");
}

inline void require_shape(int64_t batch, int64_t query_tokens) {
  if (batch < 0 || query_tokens < 0) throw InvalidArgument("query must have shape [batch, query_tokens, dim]");
}

// A device allocation that only grows (the reference's ensure_device_capacity,
// cu:3057-3067) and is released with its owner.
struct DeviceBuffer {
  void* ptr = nullptr;
  size_t cap = 0;
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer();
  void ensure(size_t bytes, const char* what);
  void reset();
  template <typename T>
  T* as() const {
    return static_cast<T*>(ptr);
  }
};

// Pinned, coherent host memory that only grows.  The synchronous entry
// points stage the query and the results there: the kernels read the query
// and write top-k results across the host link themselves (a full score
// matrix comes back by one DMA copy), so no pageable staging copies remain.
struct HostBuffer {
  void* ptr = nullptr;
  size_t cap = 0;
  HostBuffer() = default;
  HostBuffer(const HostBuffer&) = delete;
  HostBuffer& operator=(const HostBuffer&) = delete;
  ~HostBuffer();
  void ensure(size_t bytes, const char* what);
  template <typename T>
  T* as() const {
    return static_cast<T*>(ptr);
  }
};

// util.hip
hipError_t launch_fill_f32(float* d, int64_t n, float value, hipStream_t stream);

}  // namespace msim
