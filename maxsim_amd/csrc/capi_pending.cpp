// capi_pending.cpp -- entry points declared in include/maxsim_hip.h whose
// kernels are not written yet; each reports MSIM_ENOTSUP.
#include "capi_internal.hpp"

using namespace msim;

#define MSIM_PENDING(name) \
  return guarded([&] { throw NotSupported(name " is not implemented yet"); })

extern "C" {
int msim_int4_maxsim_batch(msim_int4_docs*, const float*, int64_t, int64_t, int64_t, float*) { MSIM_PENDING("maxsim_batch"); }
int msim_int4_topk_batch(msim_int4_docs*, const float*, int64_t, int64_t, int64_t, int64_t, float*, int64_t*) { MSIM_PENDING("topk_batch"); }
int msim_int4_score(msim_int4_docs*, const float*, int64_t, int64_t, int64_t, const char*, const float*, int64_t, int64_t, int64_t, double, const int64_t*, int64_t, int, float*) { MSIM_PENDING("score_batch"); }
int msim_binary_create(const uint8_t*, int64_t, int64_t, const int64_t*, int64_t, int, msim_binary_docs**) { MSIM_PENDING("CudaPackedDocs"); }
int msim_binary_destroy(msim_binary_docs*) { return MSIM_OK; }
int msim_binary_set_scale_vector(msim_binary_docs*, const float*, int64_t) { MSIM_PENDING("set_scale_vector"); }
int msim_binary_clear_scale_vector(msim_binary_docs*) { MSIM_PENDING("clear_scale_vector"); }
int msim_binary_set_token_scale(msim_binary_docs*, const float*, int64_t) { MSIM_PENDING("set_token_scale_vector"); }
int msim_binary_clear_token_scale(msim_binary_docs*) { MSIM_PENDING("clear_token_scale_vector"); }
int msim_binary_get_props(const msim_binary_docs*, msim_binary_props*) { MSIM_PENDING("props"); }
int msim_binary_maxsim_batch(msim_binary_docs*, const float*, int64_t, int64_t, int64_t, double, int, int, float*) { MSIM_PENDING("maxsim_batch"); }
int msim_binary_topk_batch(msim_binary_docs*, const float*, int64_t, int64_t, int64_t, int64_t, double, int, int, float*, int64_t*) { MSIM_PENDING("topk_batch"); }
int msim_binary_score(msim_binary_docs*, const float*, int64_t, int64_t, int64_t, const char*, const float*, int64_t, int64_t, int64_t, double, double, int, int, const float*, const int64_t*, int64_t, float*) { MSIM_PENDING("score_batch"); }
int msim_binary_hamming_batch(msim_binary_docs*, const uint8_t*, int64_t, int64_t, int64_t, int32_t*) { MSIM_PENDING("hamming_batch"); }
int msim_binary_topk_hamming(msim_binary_docs*, const uint8_t*, int64_t, int64_t, int64_t, int64_t, float*, int64_t*) { MSIM_PENDING("topk_hamming"); }
int msim_binary_topk_hamming_async(msim_binary_docs*, const uint8_t*, int64_t, int64_t, int64_t, float*, int64_t*, void*) { MSIM_PENDING("topk_hamming_async"); }
}
