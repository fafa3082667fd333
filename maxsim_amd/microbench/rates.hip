// rates.hip -- instruction-rate tests behind the scan's design choices, run
// by `bench.py --rates`: loops with no memory traffic, launched in the scan's
// shape (256-thread workgroups, 1 or 2 waves per SIMD on every CU), timed
// with HIP events.  Each test reports nanoseconds per unit per SIMD:
//   mfma         one v_mfma_i32_16x16x64_i8 (16 per unit, independent)
//   mfma_fmaN    one MFMA followed by N independent fp32 fmas that read the
//                other accumulator set (N = 2, 3, 4, 6)
//   scan_tile    the scan's 16-token tile: 16 MFMAs, the previous tile's
//                one-fma epilogue (32 fmas, 16 v_max3), the int4 unpack (12)
//                and the 4 per-tile epilogue constants
//   xor_bcnt     one 128-bit Hamming term per lane: 4 v_xor + 4 v_bcnt
//                (accumulating), 64 (query row, token) pairs per unit
//   mfma_sign    the same 64 pairs on the matrix core: int8 +-1 query bytes
//                against 0/1 sign bytes, 128 dims = 2 MFMAs per 16 x 16 pairs
#include <hip/hip_runtime.h>

#include <cstring>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float max3_op(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// 16 MFMAs per unit; NV fmas after each (0: MFMA alone).
template <int NV>
__global__ __launch_bounds__(256) void mfma_kernel(const v4i* __restrict__ in, float* __restrict__ out, int iters) {
  const int lane = threadIdx.x & 63;
  v4i a = in[lane], b[8], acc0[8], acc1[8];
  for (int j = 0; j < 8; ++j) {
    b[j] = in[64 * j + lane];
    acc0[j] = in[512 + 64 * j + lane];
    acc1[j] = in[1024 + 64 * j + lane];
  }
  float f[8];
  for (int k = 0; k < 8; ++k) f[k] = __int_as_float(in[1536 + lane][k & 3] & 0x3FFFFFFF);
  const float y = f[1] * 0.5f;
  auto unit = [&](v4i (&q)[8], const v4i (&p)[8]) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        q[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[j], h ? q[j] : p[j], 0, 0, 0);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          const int s = (h * 8 + j) * NV + v;
          f[s & 7] = __builtin_fmaf(__int_as_float(p[(s >> 2) & 7][s & 3]), y, f[s & 7]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
  };
  for (int i = 0; i < iters; i += 2) {
    unit(acc0, acc1);
    unit(acc1, acc0);
    a = a ^ i;
  }
  float s = 0.0f;
  for (int k = 0; k < 8; ++k) s += f[k];
  for (int j = 0; j < 8; ++j) s += (float)(acc0[j][0] + acc1[j][3]);
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// The scan's tile: MFMAs of the next tile interleaved with the epilogue of
// the previous one, two accumulator sets, C operand 2^23 (bits), the int4
// unpack and the per-tile constants c = -2^23 a.
__global__ __launch_bounds__(256) void scan_tile_kernel(const v4u* __restrict__ in, float* __restrict__ out, int iters) {
  constexpr int NT = 8;
  const int lane = threadIdx.x & 63;
  v4i blo[NT], bhi[NT], acc_a[NT], acc_b[NT];
  float m[NT];
  for (int j = 0; j < NT; ++j) {
    blo[j] = (v4i)in[2 * j * 64 + lane];
    bhi[j] = (v4i)in[(2 * j + 1) * 64 + lane];
    acc_a[j] = (v4i)in[1024 + j * 64 + lane];
    acc_b[j] = (v4i)in[1536 + j * 64 + lane];
    m[j] = -1e30f;
  }
  v4u w = in[lane], sv = in[64 + lane];
  v4i cmagic = {0x4B000000, 0x4B000000, 0x4B000000, 0x4B000000};
  asm volatile("" : "+v"(cmagic));
  float ea[4], ec[4];
  for (int r = 0; r < 4; ++r) {
    ea[r] = __uint_as_float(sv[r] & 0x3FFFFFFFu);
    ec[r] = ea[r] * -8388608.0f;
  }
  auto unit = [&](v4i (&acc_q)[NT], const v4i (&acc_p)[NT], int i) {
    const v4u wq = w;
    w = wq ^ (v4u){(unsigned)i, 1u, 2u, 3u};
    float a[4], c[4];
    for (int r = 0; r < 4; ++r) {
      a[r] = ea[r];
      c[r] = ec[r];
    }
    sv = sv ^ (unsigned)i;
    for (int r = 0; r < 4; ++r) {
      ea[r] = __uint_as_float(sv[r] & 0x3FFFFFFFu);
      ec[r] = ea[r] * -8388608.0f;
    }
    v4i lo, hi;
    for (int x = 0; x < 4; ++x) lo[x] = (int)((wq[x] << 4) & 0xF0F0F0F0u);
    __builtin_amdgcn_sched_barrier(0);
    auto epi = [&](int j, int h) {
      const float x0 = __builtin_fmaf(__int_as_float(acc_p[j][2 * h]), a[2 * h], c[2 * h]);
      const float x1 = __builtin_fmaf(__int_as_float(acc_p[j][2 * h + 1]), a[2 * h + 1], c[2 * h + 1]);
      m[j] = max3_op(m[j], x0, x1);
    };
    for (int j = 0; j < NT; ++j) {
      acc_q[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(lo, blo[j], cmagic, 0, 0, 0);
      epi(j, 0);
      if (j < 4) hi[j] = (int)(wq[j] & 0xF0F0F0F0u);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int j = 0; j < NT; ++j) {
      acc_q[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(hi, bhi[j], acc_q[j], 0, 0, 0);
      epi(j, 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int i = 0; i < iters; i += 2) {
    unit(acc_a, acc_b, i);
    unit(acc_b, acc_a, i + 1);
  }
  float s = 0.0f;
  for (int j = 0; j < NT; ++j) s += m[j] + (float)(acc_a[j][0] + acc_b[j][3]);
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// 128-bit Hamming terms on the VALU: per unit and lane, 8 independent
// (query row, token) pairs, each 4 XORs and 4 accumulating bit counts.
__global__ __launch_bounds__(256) void xor_bcnt_kernel(const v4u* __restrict__ in, float* __restrict__ out, int iters) {
  const int lane = threadIdx.x & 63;
  v4u q = in[lane], d[8];
  unsigned acc[8];
  for (int t = 0; t < 8; ++t) {
    d[t] = in[64 * (t + 1) + lane];
    acc[t] = 0u;
  }
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int x = 0; x < 4; ++x) acc[t] = __popc(q[x] ^ d[t][x]) + acc[t];  // v_xor, v_bcnt (adds)
    q = q ^ (unsigned)i;
  }
  unsigned s = 0;
  for (int t = 0; t < 8; ++t) s += acc[t];
  out[blockIdx.x * 256 + threadIdx.x] = (float)s;
}

// The same pairs on the matrix core: A = 16 tokens x 64 sign bytes (0/1),
// B = 64 dims x 16 query rows (+-1 bytes); 2 MFMAs per 128 dims, 8 query
// tiles per unit (16 tokens x 128 rows = 2048 pairs per 16 MFMAs).
__global__ __launch_bounds__(256) void mfma_sign_kernel(const v4i* __restrict__ in, float* __restrict__ out, int iters) {
  const int lane = threadIdx.x & 63;
  v4i a0 = in[lane] & 0x01010101, a1 = in[64 + lane] & 0x01010101, b[16], acc[8];
  for (int j = 0; j < 16; ++j) b[j] = in[128 + 64 * j + lane] | 0x01010101;
  for (int j = 0; j < 8; ++j) acc[j] = (v4i){0, 0, 0, 0};
  int best = 0;
  for (int i = 0; i < iters; ++i) {
    v4i r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b[2 * j], acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b[2 * j + 1], r[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = r[j];
    a0 = a0 ^ (i & 0x01010101);
  }
  for (int j = 0; j < 8; ++j) best += acc[j][0] + acc[j][3];
  out[blockIdx.x * 256 + threadIdx.x] = (float)best;
}

}  // namespace

// Runs test `name` with `waves_per_simd` (1 or 2) waves on every SIMD of
// `cus` compute units for `iters` units per wave; writes nanoseconds per
// unit per SIMD (see the file comment for each test's unit) and returns 0,
// or -1 for an unknown test or a HIP error.
extern "C" int msim_rate_test(const char* name, int cus, int waves_per_simd, int iters, double* ns_per_unit) {
  if (name == nullptr || ns_per_unit == nullptr || cus <= 0 || waves_per_simd < 1 || waves_per_simd > 2 || iters < 2)
    return -1;
  iters &= ~1;
  const int wgs = cus * waves_per_simd;  // 4 waves per workgroup: one per SIMD
  void* din = nullptr;
  float* dout = nullptr;
  if (hipMalloc(&din, 4096 * 16) != hipSuccess) return -1;
  if (hipMalloc(&dout, (size_t)wgs * 256 * 4) != hipSuccess) {
    (void)hipFree(din);
    return -1;
  }
  unsigned host[4096 * 4];
  for (unsigned i = 0; i < 4096 * 4; ++i) host[i] = (i * 2654435761u) & 0x3FFFFFFFu;
  int rc = hipMemcpy(din, host, sizeof(host), hipMemcpyHostToDevice) == hipSuccess ? 0 : -1;
  double units_per_wave = iters, mult = 1.0;
  auto launch = [&]() {
    const v4i* vi = static_cast<const v4i*>(din);
    const v4u* vu = static_cast<const v4u*>(din);
    if (!strcmp(name, "mfma")) mfma_kernel<0><<<wgs, 256>>>(vi, dout, iters);
    else if (!strcmp(name, "mfma_fma2")) mfma_kernel<2><<<wgs, 256>>>(vi, dout, iters);
    else if (!strcmp(name, "mfma_fma3")) mfma_kernel<3><<<wgs, 256>>>(vi, dout, iters);
    else if (!strcmp(name, "mfma_fma4")) mfma_kernel<4><<<wgs, 256>>>(vi, dout, iters);
    else if (!strcmp(name, "mfma_fma6")) mfma_kernel<6><<<wgs, 256>>>(vi, dout, iters);
    else if (!strcmp(name, "scan_tile")) scan_tile_kernel<<<wgs, 256>>>(vu, dout, iters);
    else if (!strcmp(name, "xor_bcnt")) xor_bcnt_kernel<<<wgs, 256>>>(vu, dout, iters);
    else if (!strcmp(name, "mfma_sign")) mfma_sign_kernel<<<wgs, 256>>>(vi, dout, iters);
    else return false;
    return true;
  };
  // Units: mfma*: per MFMA (16 per iteration); xor_bcnt: per pair (8 x 64
  // per iteration and wave); mfma_sign: per pair (2048 per iteration).
  if (!strncmp(name, "mfma_fma", 8) || !strcmp(name, "mfma")) mult = 16.0;
  else if (!strcmp(name, "xor_bcnt")) mult = 8.0 * 64.0;
  else if (!strcmp(name, "mfma_sign")) mult = 2048.0;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (rc == 0 && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)) rc = -1;
  if (rc == 0) {
    for (int w = 0; w < 2 && rc == 0; ++w)
      if (!launch()) rc = -1;
    if (rc == 0 && hipDeviceSynchronize() != hipSuccess) rc = -1;
  }
  constexpr int kReps = 5;
  if (rc == 0) {
    (void)hipEventRecord(e0, nullptr);
    for (int r = 0; r < kReps; ++r) launch();
    (void)hipEventRecord(e1, nullptr);
    float ms = 0.0f;
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess || hipGetLastError() != hipSuccess)
      rc = -1;
    else
      *ns_per_unit = (double)ms * 1e6 / kReps / (units_per_wave * mult * waves_per_simd);
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(din);
  (void)hipFree(dout);
  return rc;
}
