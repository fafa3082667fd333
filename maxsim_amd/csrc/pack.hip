// pack.hip -- symmetric int4 packing of fp32 embeddings on the device, for
// building int4 corpora without the host pass (reference: pack_int4_symmetric,
// experimental.py:218-268; nibble order _pack_signed_int4_values,
// experimental.py:604-609).
//
//   token granularity:  s_t = f32(max|x_t|) / f32(7), 0 -> 1; v = clip(rint(x / s_t), -7, 7)
//   tensor granularity: s = max|x| / 7 in float64 (0 -> 1) or the given scale;
//                       v = clip(rint(x / f32(s)), -7, 7)
//   byte i of a token = (v[2i] & 0xF) | (v[2i + 1] & 0xF) << 4
//
// Every division is IEEE single precision, correctly rounded, and rint rounds
// half to even, as NumPy's float32 arithmetic does, so the codes and scales
// equal the host packer's bit for bit.  HBM-bound byte work: 4 * dim bytes
// read, dim / 2 (+ dim values, + 4 scale) bytes written per token.
#include "common.hpp"
#include "internal.hpp"

namespace msim {

namespace {

constexpr uint32_t kExpMask = 0x7F800000u;

// |x| as order-preserving bits; non-finite values raise the flag.  The bits
// pass through an empty asm so that the exponent test stays an integer test:
// under -fno-honor-nans the compiler would otherwise fold it to |x| == inf
// and miss NaNs.
__device__ __forceinline__ uint32_t abs_bits(float x, uint32_t& bad) {
  uint32_t u = __float_as_uint(x);
  asm volatile("" : "+v"(u));
  u &= 0x7FFFFFFFu;
  bad |= (u & kExpMask) == kExpMask ? 1u : 0u;
  return u;
}

__device__ __forceinline__ int quant4(float x, float s) {
  const float r = rintf(__fdiv_rn(x, s));
  return r > 7.0f ? 7 : (r < -7.0f ? -7 : (int)r);
}

// Maximum |x| over n values (n a multiple of 4) into work[0] and the
// non-finite flag into work[1] (both zero before the launch).
__global__ __launch_bounds__(256) void absmax_kernel(const float4* __restrict__ x, int64_t n4,
                                                     uint32_t* __restrict__ work) {
  uint32_t m = 0, bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    const float4 v = x[i];
    m = max(m, max(max(abs_bits(v.x, bad), abs_bits(v.y, bad)), max(abs_bits(v.z, bad), abs_bits(v.w, bad))));
  }
  // Wave, then workgroup reduction: one pair of atomics per workgroup.
  __shared__ uint32_t s_m[4], s_bad[4];
  m = wave_reduce(m, [](uint32_t a, uint32_t b) { return max(a, b); });
  bad = wave_reduce(bad, [](uint32_t a, uint32_t b) { return a | b; });
  const int wave = threadIdx.x / kWave;
  if (lane_id() == 0) {
    s_m[wave] = m;
    s_bad[wave] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    m = max(max(s_m[0], s_m[1]), max(s_m[2], s_m[3]));
    bad = s_bad[0] | s_bad[1] | s_bad[2] | s_bad[3];
    if (m != 0) atomicMax(&work[0], m);
    if (bad != 0) atomicOr(&work[1], 1u);
  }
}

// One wave per token (grid-stride over tokens); lane l holds dims 2l, 2l + 1
// of each 128-dim chunk, so its byte is byte l of the chunk's 64.
template <bool kToken>
__global__ __launch_bounds__(256) void pack_int4_kernel(const float* __restrict__ x, int64_t num_tokens, int dim,
                                                        double given_scale, uint32_t* __restrict__ work,
                                                        uint8_t* __restrict__ codes, float* __restrict__ token_scale,
                                                        int8_t* __restrict__ values) {
  const int lane = lane_id();
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x / kWave);
  float s = 1.0f;
  if (!kToken) {
    if (given_scale > 0.0) {
      s = (float)given_scale;
    } else {
      const float peak = __uint_as_float(work[0]);
      s = peak == 0.0f ? 1.0f : (float)__ddiv_rn((double)peak, 7.0);
    }
  }
  uint32_t bad = 0;
  for (int64_t t = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave; t < num_tokens; t += waves) {
    const float* row = x + t * dim;
    if (kToken) {
      uint32_t m = 0;
      for (int c = 2 * lane; c < dim; c += 2 * kWave) {
        const float2 v = *reinterpret_cast<const float2*>(row + c);
        m = max(m, max(abs_bits(v.x, bad), abs_bits(v.y, bad)));
      }
      m = wave_reduce(m, [](uint32_t a, uint32_t b) { return max(a, b); });
      s = __fdiv_rn(__uint_as_float(m), 7.0f);
      if (s == 0.0f) s = 1.0f;
      if (lane == 0) token_scale[t] = s;
    }
    for (int c = 2 * lane; c < dim; c += 2 * kWave) {
      const float2 v = *reinterpret_cast<const float2*>(row + c);
      const int q0 = quant4(v.x, s), q1 = quant4(v.y, s);
      codes[t * (dim / 2) + c / 2] = (uint8_t)((q0 & 0xF) | ((q1 & 0xF) << 4));
      if (values) {
        const uint16_t pair = (uint16_t)((uint8_t)(int8_t)q0 | ((uint16_t)(uint8_t)(int8_t)q1 << 8));
        *reinterpret_cast<uint16_t*>(values + t * dim + c) = pair;
      }
    }
  }
  if (kToken) {
    bad = wave_reduce(bad, [](uint32_t a, uint32_t b) { return a | b; });
    if (lane == 0 && bad != 0) atomicOr(&work[1], 1u);
  }
}

// dim == 128: each wave takes 4 consecutive tokens per step and issues their
// four loads before any reduction, so that 2 KiB per wave are in flight.
constexpr int kPackTokens = 4;

template <bool kToken>
__global__ __launch_bounds__(256) void pack_int4_dim128_kernel(const float* __restrict__ x, int64_t num_tokens,
                                                               double given_scale, uint32_t* __restrict__ work,
                                                               uint8_t* __restrict__ codes,
                                                               float* __restrict__ token_scale,
                                                               int8_t* __restrict__ values) {
  const int lane = lane_id();
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x / kWave);
  float st = 1.0f;
  if (!kToken) {
    if (given_scale > 0.0) {
      st = (float)given_scale;
    } else {
      const float peak = __uint_as_float(work[0]);
      st = peak == 0.0f ? 1.0f : (float)__ddiv_rn((double)peak, 7.0);
    }
  }
  uint32_t bad = 0;
  for (int64_t t0 = ((int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave) * kPackTokens; t0 < num_tokens;
       t0 += waves * kPackTokens) {
    float2 v[kPackTokens];
#pragma unroll
    for (int j = 0; j < kPackTokens; ++j)
      v[j] = t0 + j < num_tokens ? reinterpret_cast<const float2*>(x + (t0 + j) * 128)[lane] : make_float2(0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < kPackTokens; ++j) {
      const int64_t t = t0 + j;
      if (t >= num_tokens) break;
      float s = st;
      if (kToken) {
        uint32_t m = max(abs_bits(v[j].x, bad), abs_bits(v[j].y, bad));
        m = wave_reduce(m, [](uint32_t a, uint32_t b) { return max(a, b); });
        s = __fdiv_rn(__uint_as_float(m), 7.0f);
        if (s == 0.0f) s = 1.0f;
        if (lane == 0) token_scale[t] = s;
      }
      const int q0 = quant4(v[j].x, s), q1 = quant4(v[j].y, s);
      codes[t * 64 + lane] = (uint8_t)((q0 & 0xF) | ((q1 & 0xF) << 4));
      if (values) {
        const uint16_t pair = (uint16_t)((uint8_t)(int8_t)q0 | ((uint16_t)(uint8_t)(int8_t)q1 << 8));
        reinterpret_cast<uint16_t*>(values + t * 128)[lane] = pair;
      }
    }
  }
  if (kToken) {
    bad = wave_reduce(bad, [](uint32_t a, uint32_t b) { return a | b; });
    if (lane == 0 && bad != 0) atomicOr(&work[1], 1u);
  }
}

}  // namespace

hipError_t launch_int4_absmax(const float* d_x, int64_t num_tokens, int dim, uint32_t* d_work, int num_cus,
                              hipStream_t stream) {
  if (num_tokens <= 0) return hipSuccess;
  if (dim <= 0 || dim % 8 != 0) return hipErrorInvalidValue;
  const int64_t n4 = num_tokens * dim / 4;
  const int64_t blocks = std::min<int64_t>((n4 + 255) / 256, (int64_t)std::max(1, num_cus) * 4);
  absmax_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(reinterpret_cast<const float4*>(d_x), n4, d_work);
  return hipGetLastError();
}

hipError_t launch_pack_int4(const float* d_x, int64_t num_tokens, int dim, bool token, double given_scale,
                            uint32_t* d_work, uint8_t* d_codes, float* d_token_scale, int8_t* d_values,
                            int num_cus, hipStream_t stream) {
  if (num_tokens <= 0) return hipSuccess;
  if (dim <= 0 || dim % 8 != 0 || d_codes == nullptr || (token && d_token_scale == nullptr))
    return hipErrorInvalidValue;
  if (dim == 128) {
    const int64_t blocks = std::min<int64_t>((num_tokens + 4 * kPackTokens - 1) / (4 * kPackTokens),
                                             (int64_t)std::max(1, num_cus) * 32);
    if (token)
      pack_int4_dim128_kernel<true><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(
          d_x, num_tokens, given_scale, d_work, d_codes, d_token_scale, d_values);
    else
      pack_int4_dim128_kernel<false><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(
          d_x, num_tokens, given_scale, d_work, d_codes, d_token_scale, d_values);
    return hipGetLastError();
  }
  const int64_t blocks = std::min<int64_t>((num_tokens + 3) / 4, (int64_t)std::max(1, num_cus) * 32);
  if (token)
    pack_int4_kernel<true><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(d_x, num_tokens, dim, given_scale, d_work,
                                                                             d_codes, d_token_scale, d_values);
  else
    pack_int4_kernel<false><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(d_x, num_tokens, dim, given_scale,
                                                                              d_work, d_codes, d_token_scale, d_values);
  return hipGetLastError();
}

}  // namespace msim
