// common.hpp -- device helpers shared by the MI355X (gfx950) MaxSim kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace msim {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr float kNegInf = -__builtin_huge_valf();

// gfx9 buffer descriptor word 3 (raw byte addressing, bounds-checked by
// num_records: out-of-range lanes read zero instead of faulting).
constexpr int kBufferFlags = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_bytes, kBufferFlags);
}

// Cache-policy operand of a buffer load that reads the agent-coherent copy
// (the sc1 bit, as on an agent-scope atomic load).
constexpr int kCoherentLoadPolicy = 16;

__device__ __forceinline__ v4u load_b128(__amdgpu_buffer_rsrc_t r, int byte_offset) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, 0);
}

__device__ __forceinline__ uint64_t load_b64(__amdgpu_buffer_rsrc_t r, int byte_offset) {
  typedef unsigned v2u __attribute__((ext_vector_type(2)));
  const v2u v = __builtin_amdgcn_raw_buffer_load_b64(r, byte_offset, 0, 0);
  return ((uint64_t)v.y << 32) | v.x;
}

__device__ __forceinline__ uint64_t load_b64_coherent(__amdgpu_buffer_rsrc_t r, int byte_offset) {
  typedef unsigned v2u __attribute__((ext_vector_type(2)));
  const v2u v = __builtin_amdgcn_raw_buffer_load_b64(r, byte_offset, 0, kCoherentLoadPolicy);
  return ((uint64_t)v.y << 32) | v.x;
}

__device__ __forceinline__ unsigned load_b32(__amdgpu_buffer_rsrc_t r, int byte_offset) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, byte_offset, 0, 0);
}

// Buffer descriptor as an SGPR quad (for the inline-assembly loads below).
__device__ __forceinline__ v4i make_rsrc_words(const void* base, uint32_t num_bytes) {
  const uint64_t a = (uint64_t)base;
  return (v4i){(int)(uint32_t)a, (int)(uint32_t)(a >> 32) & 0xFFFF, (int)num_bytes, kBufferFlags};
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Buffer loads whose destination is LDS: lane l writes its 16 (4) bytes at
// LDS address lds + 16 l (4 l), lds being wave-uniform.  They are issued from
// inline assembly so that the compiler's conservative LDS-DMA tracking does
// not add a full vmcnt wait before every later LDS read; in exchange, the
// code must wait with vm_wait_lds<N>() (N = vector memory instructions
// issued after the load that may still be in flight) before reading the
// data.  M0 carries the LDS base (an SALU write of M0 needs one wait state
// before a load with the LDS destination reads it) and is restored afterwards.
__device__ __forceinline__ void lds_load_b128(v4i rsrc, uint32_t byte_offset, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(byte_offset), "s"(rsrc)
      : "memory");
}
__device__ __forceinline__ void lds_load_b32(v4i rsrc, uint32_t byte_offset, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dword %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(byte_offset), "s"(rsrc)
      : "memory");
}

// The same with a wave-uniform byte offset (soffset) added to every lane's
// voffset.  The buffer range check covers voffset only: the caller keeps
// soffset + voffset inside the buffer.
__device__ __forceinline__ void lds_load_b128_so(v4i rsrc, uint32_t voffset, uint32_t soffset, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(voffset), "s"(rsrc), "s"(soffset)
      : "memory");
}
__device__ __forceinline__ void lds_load_b32_so(v4i rsrc, uint32_t voffset, uint32_t soffset, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dword %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(voffset), "s"(rsrc), "s"(soffset)
      : "memory");
}

// A use of `v` at this point: the compiler completes its load here.
template <typename T>
__device__ __forceinline__ void use_here(const T& v) {
  asm volatile("" ::"v"(v));
}

template <int N>
__device__ __forceinline__ void vm_wait_lds() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Orders a later LDS-destination load into the slot these registers were
// read from after the read itself (the registers must hold the data first).
// Never issue loads with a register destination outside compiler tracking:
// the register allocator may copy such a register before the data lands.
template <typename A, typename B>
__device__ __forceinline__ void lds_read_done(const A& a, const B& b) {
  asm volatile("" ::"v"(a), "v"(b) : "memory");
}

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Mark a 64-bit value as wave-uniform so it lives in SGPRs (it must already be
// equal across the wave).
__device__ __forceinline__ int64_t wave_uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Read-only view in the constant address space: uniform loads through it
// become scalar loads (the data must not change during the kernel).
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* as_constant(const T* p) {
  return (const __attribute__((address_space(4))) T*)p;
}

// Order this wave's LDS accesses (no effect on global memory operations).
__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Workgroup barrier that orders LDS only: global stores still in flight are
// not waited for (__syncthreads would wait for them).
__device__ __forceinline__ void group_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Value of lane 4 * (l / 4) + I in every lane l (DPP quad permute).
template <int I>
__device__ __forceinline__ uint32_t quad_broadcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, I * 0x55, 0xF, 0xF, false);
}

// Wait states between a block of MFMAs and the first VALU reads of their
// results.  After v_mfma_i32_16x16x64_i8 the compiler's hazard model spaces a
// dependent VALU read 8 wait states behind the MFMA; on gfx950 reads at that
// distance returned the accumulator's earlier contents now and then
// (nondeterministic scores, depending on how the waves of a SIMD
// interleave).  24 more are added here, the scheduler kept from moving work
// across them.
__device__ __forceinline__ void mfma_results_fence() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
  __builtin_amdgcn_sched_barrier(0);
}

// Whole-wave reduction: DPP quad butterflies and row rotations by 4 and 8
// reduce each row of 16 lanes, then the four row results are combined from
// lanes 0, 16, 32 and 48.  The result is wave-uniform.
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
  static_assert(sizeof(T) == 4, "32-bit values");
  auto dpp = [](T x, auto ctrl) -> T {
    return __builtin_bit_cast(T, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), decltype(ctrl)::value, 0xF, 0xF, true));
  };
  v = op(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
  v = op(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
  v = op(v, dpp(v, std::integral_constant<int, 0x124>{}));  // row_ror:4
  v = op(v, dpp(v, std::integral_constant<int, 0x128>{}));  // row_ror:8
  const int x = __builtin_bit_cast(int, v);
  const T r0 = __builtin_bit_cast(T, __builtin_amdgcn_readlane(x, 0));
  const T r1 = __builtin_bit_cast(T, __builtin_amdgcn_readlane(x, 16));
  const T r2 = __builtin_bit_cast(T, __builtin_amdgcn_readlane(x, 32));
  const T r3 = __builtin_bit_cast(T, __builtin_amdgcn_readlane(x, 48));
  return op(op(r0, r1), op(r2, r3));
}

__device__ __forceinline__ float fmax3(float a, float b, float c) { return fmaxf(a, fmaxf(b, c)); }
// One v_max3_f32 (the compiler splits fmax chains into two-operand maxima to
// shorten dependencies; where issue slots are the limit, one instruction per
// three operands is better).  Operands are never NaN in these kernels.
__device__ __forceinline__ float max3_op(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// numpy's pairwise float64 reduction order over a[0..n) for 8 < n <= 128 is
// eight strided accumulators, combined ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)),
// then the n % 8 tail added sequentially; below 8 it is a plain sequential
// sum from 0.0; above 128 it splits at n/2 rounded down to a multiple of 8.
// pairwise_sum_serial evaluates that exact tree on one lane.  `get(i)`
// returns a[i] as double.
template <typename Get>
__device__ double pairwise_block(Get get, int64_t base, int64_t n) {
  if (n < 8) {
    double res = 0.0;
    for (int64_t i = 0; i < n; ++i) res = __dadd_rn(res, get(base + i));
    return res;
  }
  double r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = get(base + j);
  int64_t i = 8;
  for (; i < n - (n % 8); i += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = __dadd_rn(r[j], get(base + i + j));
  }
  double res = __dadd_rn(__dadd_rn(__dadd_rn(r[0], r[1]), __dadd_rn(r[2], r[3])),
                         __dadd_rn(__dadd_rn(r[4], r[5]), __dadd_rn(r[6], r[7])));
  for (; i < n; ++i) res = __dadd_rn(res, get(base + i));
  return res;
}

template <typename Get>
__device__ double pairwise_sum_serial(Get get, int64_t n) {
  if (n <= 128) return pairwise_block(get, 0, n);
  // Iterative post-order walk of numpy's split tree.
  struct Frame {
    int64_t base, n;
    int state;
    double left;
  };
  Frame stack[40];
  int top = 0;
  stack[0] = {0, n, 0, 0.0};
  double ret = 0.0;
  while (top >= 0) {
    Frame& f = stack[top];
    if (f.n <= 128) {
      ret = pairwise_block(get, f.base, f.n);
      --top;
      continue;
    }
    int64_t n2 = f.n / 2;
    n2 -= n2 % 8;
    if (f.state == 0) {
      f.state = 1;
      stack[top + 1] = {f.base, n2, 0, 0.0};
      ++top;
    } else if (f.state == 1) {
      f.left = ret;
      f.state = 2;
      stack[top + 1] = {f.base + n2, f.n - n2, 0, 0.0};
      ++top;
    } else {
      ret = __dadd_rn(f.left, ret);
      --top;
    }
  }
  return ret;
}

}  // namespace msim
