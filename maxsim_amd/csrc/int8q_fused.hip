// int8q_fused.hip -- one-launch int4 x int8-query MaxSim search on gfx950.
//
// Semantics restated from the reference: query quantisation
// tests/test_int4_int8q.py:11-14 (device form cu:1455-1492), token-scaled
// MaxSim cu:1569-1627 / tests/test_int4_int8q.py:15-26, top-k order
// cu:1629-1692.  Scores equal the C oracle bit for bit.
//
// One launch does the whole call:
//  1. every workgroup quantises the fp32 query rows (<= 128) into LDS in the
//     MFMA B-operand byte order (sigma = f32(max|q| / 127), rint(q / sigma));
//  2. each wave loads all query tiles into registers and walks its
//     documents (contiguous ranges balanced by 16-token tile count) as one
//     stream of 16-token tiles, keeping PREFETCH tiles of codes and token
//     scales in flight ahead of the MFMA work;
//  3. v_mfma_i32_16x16x64_i8 forms exact dots: each code byte's nibbles are
//     masked in place as int8 (hi = w & 0xF0, lo = (w << 4) & 0xF0), i.e.
//     sixteen times the signed value, so acc = 16 * dot; float(acc) times
//     (s_t / 16) rounds the same real number d * s_t as float(dot) * s_t;
//  4. per lane a running max over its four token rows; at a document end a
//     cross-lane max, then numpy's float64 pairwise sum over query tokens;
//  5. the last workgroup to finish (device-scope ticket) selects the top-k
//     of every batch row (topk_block.hpp) and resets the ticket.
#include "common.hpp"
#include "internal.hpp"
#include "topk_block.hpp"

namespace msim {

constexpr int kPrefetch = 3;
constexpr int kTailEPT = 16;  // tail keys per thread kept in registers (4096 docs at 256 threads)

template <int THREADS>
struct FusedSmem {
  static constexpr int kWaves = THREADS / kWave;
  union {
    struct {
      int8_t q[128 * 128];
      float qscale[128];
      float rowmax[kWaves][128];
    } s;
    TopkSmem<THREADS, kFusedMaxK> t;
  } u;
  uint32_t is_last;
};

// rint(f32(v / s)) with v / s in [-127, 127].  r = f32(v * f32(1/s)) is within
// 2^-15 of the correctly rounded quotient q (|r - q| <= 127 * 2^-23 + 2^-18),
// so both round to the same integer unless r lies within 2^-15 of a half
// integer; only then is the exact quotient formed.
__device__ __forceinline__ int quantize_code(float v, float s, float inv) {
  const float r = v * inv;
  const float f = floorf(r);
  if (fabsf(r - f - 0.5f) <= 3.0517578125e-05f) return (int)rintf(__fdiv_rn(v, s));
  return (int)rintf(r);
}

// Quantise query rows [0, rows) into sm.q (B order) and sm.qscale; rows up to
// 128 are zero-filled.  Each row is split over 128 / E threads of E dims.
template <int THREADS>
__device__ __forceinline__ void quantize_rows_to_lds(const float* __restrict__ query, int rows,
                                                     FusedSmem<THREADS>& sm) {
  constexpr int E = 128 * 128 / THREADS;  // dims per thread (16, 32 or 64)
  constexpr int kSegs = 128 / E;          // threads per row
  const int tid = threadIdx.x;
  const int r = tid / kSegs, seg = tid % kSegs;
  float x[E];
  if (r < rows) {
    const float4* src = reinterpret_cast<const float4*>(query + (int64_t)r * 128 + E * seg);
#pragma unroll
    for (int v = 0; v < E / 4; ++v) {
      const float4 f = src[v];
      x[4 * v + 0] = f.x;
      x[4 * v + 1] = f.y;
      x[4 * v + 2] = f.z;
      x[4 * v + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] = 0.0f;
  }
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < E; ++i) m = fmaxf(m, fabsf(x[i]));
#pragma unroll
  for (int off = 1; off < kSegs; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
  const float s = m == 0.0f ? 1.0f : __fdiv_rn(m, 127.0f);
  const float inv = __frcp_rn(s);
  // Chunk of 16 dims d0..d0+15: even dims -> bytes 32g + io + i', odd dims ->
  // bytes 32g + 16 + io + i' (g = d0 / 32, io = (d0 % 32) / 2, i' = 0..7).
#pragma unroll
  for (int ch = 0; ch < E / 16; ++ch) {
    const int d0 = E * seg + 16 * ch;
    const int g = d0 / 32, io = (d0 % 32) / 2;
#pragma unroll
    for (int parity = 0; parity < 2; ++parity) {
      uint32_t wd[2];
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = x[16 * ch + 2 * (4 * w + j) + parity];
          const int q = max(-127, min(127, quantize_code(v, s, inv)));
          word |= (uint32_t)(q & 0xFF) << (8 * j);
        }
        wd[w] = word;
      }
      *reinterpret_cast<uint2*>(sm.u.s.q + r * 128 + 32 * g + 16 * parity + io) = make_uint2(wd[0], wd[1]);
    }
  }
  if (seg == 0) sm.u.s.qscale[r] = r < rows ? s : 0.0f;
}

// Scores are stored with agent-scope atomic stores: they are written through
// to the coherence point, so the last workgroup can read them without an
// L2-wide writeback or invalidate.
__device__ __forceinline__ void store_score(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// out[b * stride] = f32(pairwise_f64(max[b,q] * sigma[b,q]) * scale), b < batch.
__device__ __forceinline__ void finish_doc_scores(const float* rowmax, const float* qscale,
                                                  int batch, int query_tokens, double scale,
                                                  float* __restrict__ out, int64_t stride) {
  const int lane = lane_id();
  auto prod = [&](int r) -> double { return (double)rowmax[r] * (double)qscale[r]; };
  if (query_tokens < 8) {
    for (int b = lane; b < batch; b += kWave) {
      double res = 0.0;
      for (int q = 0; q < query_tokens; ++q) res = __dadd_rn(res, prod(b * query_tokens + q));
      store_score(out + (int64_t)b * stride, (float)(res * scale));
    }
    return;
  }
  const int body = query_tokens - (query_tokens % 8);
  for (int b0 = 0; b0 < batch; b0 += kWave / 8) {
    const int b = b0 + (lane >> 3), k = lane & 7;
    const bool valid = b < batch;
    const int base = b * query_tokens;
    double r = valid ? prod(base + k) : 0.0;
    for (int i = 8 + k; i < body; i += 8) r = valid ? __dadd_rn(r, prod(base + i)) : r;
    double o = __shfl_xor(r, 1);
    if ((k & 1) == 0) r = __dadd_rn(r, o);
    o = __shfl_xor(r, 2);
    if ((k & 3) == 0) r = __dadd_rn(r, o);
    o = __shfl_xor(r, 4);
    if (k == 0) r = __dadd_rn(r, o);
    if (k == 0 && valid) {
      for (int i = body; i < query_tokens; ++i) r = __dadd_rn(r, prod(base + i));
      store_score(out + (int64_t)b * stride, (float)(r * scale));
    }
  }
}

template <int NT, bool kTS, int THREADS>
__global__ __launch_bounds__(THREADS) void int8q_search_kernel(
    FusedArgs p, const uint8_t* __restrict__ codes_ptr, const float* __restrict__ token_scale_ptr,
    const int64_t* __restrict__ offsets_ptr, const int64_t* __restrict__ wave_docs_ptr,
    const float* __restrict__ query, float* __restrict__ scores, float* __restrict__ top_scores,
    int64_t* __restrict__ top_ids, uint32_t* __restrict__ counter) {
  constexpr int kFusedWaves = THREADS / kWave;
  __shared__ FusedSmem<THREADS> sm;
  const auto offsets = as_constant(offsets_ptr);
  const auto wave_docs = as_constant(wave_docs_ptr);
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_uniform(tid / kWave);
  const int g = lane >> 4, c = lane & 15;
  const int rows = p.batch * p.query_tokens;

  quantize_rows_to_lds(query, rows, sm);
  __syncthreads();

  v4i blo[NT], bhi[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int8_t* src = sm.u.s.q + (16 * j + c) * 128 + 32 * g;
    blo[j] = *reinterpret_cast<const v4i*>(src);
    bhi[j] = *reinterpret_cast<const v4i*>(src + 16);
  }

  const int64_t gw = (int64_t)blockIdx.x * kFusedWaves + wave;
  int64_t d0 = 0, d1 = 0;
  if (gw < p.num_waves) {
    d0 = wave_docs[gw];
    d1 = wave_docs[gw + 1];
  }
  d0 = wave_uniform64(d0);
  d1 = wave_uniform64(d1);
  float* rowmax = sm.u.s.rowmax[wave];

  if (d0 < d1) {
    const int64_t T0 = offsets[d0];
    const int64_t T1 = offsets[d1];
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(codes_ptr + T0 * 64, (uint32_t)((T1 - T0) * 64));
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(kTS ? (const void*)(token_scale_ptr + T0) : (const void*)codes_ptr,
                  kTS ? (uint32_t)((T1 - T0) * 4) : 0u);

    // Load cursor: next tile to fetch.  Compute cursor: next tile to score.
    int64_t ld_doc = d0;
    while (ld_doc < d1 && offsets[ld_doc + 1] == offsets[ld_doc]) ++ld_doc;
    int64_t ld_t = ld_doc < d1 ? offsets[ld_doc] : T1;
    int64_t ld_end = ld_doc < d1 ? offsets[ld_doc + 1] : T1;

    v4u raw[kPrefetch], sc[kPrefetch];
    auto issue = [&](v4u& rbuf, v4u& sbuf) {
      // Past the last tile the offset is out of range and the load reads zero.
      const uint32_t rel = ld_doc < d1 ? (uint32_t)(ld_t - T0) : 0x3FFFFF0u;
      rbuf = load_b128(rc, (int)((rel + (uint32_t)c) * 64u + 16u * (uint32_t)g));
      if (kTS) sbuf = load_b128(rs, (int)((rel + 4u * (uint32_t)g) * 4u));
      if (ld_doc < d1) {
        ld_t += 16;
        if (ld_t >= ld_end) {
          ++ld_doc;
          while (ld_doc < d1 && offsets[ld_doc + 1] == offsets[ld_doc]) ++ld_doc;
          if (ld_doc < d1) {
            ld_t = offsets[ld_doc];
            ld_end = offsets[ld_doc + 1];
          }
        }
      }
    };
#pragma unroll
    for (int s = 0; s < kPrefetch; ++s) issue(raw[s], sc[s]);

    int64_t cp_doc = d0;
    // Empty documents score 0.
    auto skip_empty = [&]() {
      while (cp_doc < d1 && offsets[cp_doc + 1] == offsets[cp_doc]) {
        for (int b = lane; b < p.batch; b += kWave) store_score(scores + (int64_t)b * p.score_stride + cp_doc, 0.0f);
        ++cp_doc;
      }
    };
    skip_empty();
    int64_t cp_t = cp_doc < d1 ? offsets[cp_doc] : T1;
    int64_t cp_end = cp_doc < d1 ? offsets[cp_doc + 1] : T1;
    int64_t ntiles = 0;
    for (int64_t d = d0; d < d1; ++d) ntiles += (offsets[d + 1] - offsets[d] + 15) >> 4;
    float m[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) m[j] = kNegInf;

    // One tile: consume slot s, refill it PREFETCH tiles ahead, score, and
    // finish the document when its last tile is done.
    auto step = [&](v4u& rbuf, v4u& sbuf) {
      const v4u w = rbuf;
      float s0 = 0.0625f, s1 = 0.0625f, s2 = 0.0625f, s3 = 0.0625f;
      if (kTS) {
        s0 = __uint_as_float(sbuf.x) * 0.0625f;
        s1 = __uint_as_float(sbuf.y) * 0.0625f;
        s2 = __uint_as_float(sbuf.z) * 0.0625f;
        s3 = __uint_as_float(sbuf.w) * 0.0625f;
      }
      v4i lo, hi;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        hi[x] = (int)(w[x] & 0xF0F0F0F0u);
        lo[x] = (int)((w[x] << 4) & 0xF0F0F0F0u);
      }
      issue(rbuf, sbuf);
      const int64_t rem = cp_end - cp_t;
      const int row0 = 4 * g;
      // Query tiles in groups of kGroup: MFMAs of a group, then its epilogue
      // (bounds the live accumulators).
      constexpr int kGroup = NT < 4 ? NT : 4;
#pragma unroll
      for (int j0 = 0; j0 < NT; j0 += kGroup) {
        v4i acc[kGroup];
#pragma unroll
        for (int jj = 0; jj < kGroup; ++jj) {
          if (j0 + jj < NT) {
            acc[jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(lo, blo[j0 + jj], (v4i){0, 0, 0, 0}, 0, 0, 0);
            acc[jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(hi, bhi[j0 + jj], acc[jj], 0, 0, 0);
          }
        }
#pragma unroll
        for (int jj = 0; jj < kGroup; ++jj) {
          if (j0 + jj < NT) {
            float x0 = (float)acc[jj][0] * s0;
            float x1 = (float)acc[jj][1] * s1;
            float x2 = (float)acc[jj][2] * s2;
            float x3 = (float)acc[jj][3] * s3;
            if (rem < 16) {
              x0 = row0 + 0 < rem ? x0 : kNegInf;
              x1 = row0 + 1 < rem ? x1 : kNegInf;
              x2 = row0 + 2 < rem ? x2 : kNegInf;
              x3 = row0 + 3 < rem ? x3 : kNegInf;
            }
            m[j0 + jj] = fmaxf(fmaxf(m[j0 + jj], fmaxf(fmaxf(x0, x1), x2)), x3);
          }
        }
      }
      cp_t += 16;
      if (cp_t >= cp_end) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          m[j] = fmaxf(m[j], __shfl_xor(m[j], 16));
          m[j] = fmaxf(m[j], __shfl_xor(m[j], 32));
        }
        if (g == 0) {
#pragma unroll
          for (int j = 0; j < NT; ++j) rowmax[16 * j + c] = m[j];
        }
        wave_sync_lds();
        finish_doc_scores(rowmax, sm.u.s.qscale, p.batch, p.query_tokens, p.scale, scores + cp_doc,
                          p.score_stride);
        wave_sync_lds();
#pragma unroll
        for (int j = 0; j < NT; ++j) m[j] = kNegInf;
        ++cp_doc;
        skip_empty();
        if (cp_doc < d1) {
          cp_t = offsets[cp_doc];
          cp_end = offsets[cp_doc + 1];
        }
      }
    };

    int64_t i = 0;
    for (; i + kPrefetch <= ntiles; i += kPrefetch) {
#pragma unroll
      for (int s = 0; s < kPrefetch; ++s) step(raw[s], sc[s]);
    }
#pragma unroll
    for (int s = 0; s < kPrefetch - 1; ++s)
      if (i + s < ntiles) step(raw[s], sc[s]);
    // Trailing empty documents were written by the last finish's skip_empty.
  } else if (gw < p.num_waves) {
    for (int64_t doc = d0; doc < d1; ++doc)
      for (int b = lane; b < p.batch; b += kWave) store_score(scores + (int64_t)b * p.score_stride + doc, 0.0f);
  }

  if (p.k <= 0) return;
  // Last-workgroup top-k.  Every thread waits until its score stores have
  // completed (they are write-through), then one thread takes a ticket; the
  // workgroup holding the last ticket selects from coherent loads.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const uint32_t ticket = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm.is_last = ticket == gridDim.x - 1 ? 1u : 0u;
  }
  __syncthreads();
  if (sm.is_last == 0) return;
  for (int b = 0; b < p.batch; ++b)
    block_topk<THREADS, kTailEPT, kFusedMaxK, true>(scores + (int64_t)b * p.score_stride, p.num_docs, p.k,
                                              nullptr, top_scores + (int64_t)b * p.k,
                                              top_ids + (int64_t)b * p.k, sm.u.t);
  __syncthreads();
  if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kFusedThreads = 256;

template <bool kTS>
static void launch_fused_nt(const FusedArgs& a, int nt, int64_t blocks, hipStream_t stream) {
  const dim3 grid((unsigned)blocks), block(kFusedThreads);
  switch (nt) {
#define MSIM_FUSED_CASE(N)                                                                  \
  int8q_search_kernel<N, kTS, kFusedThreads><<<grid, block, 0, stream>>>(                   \
      a, a.codes, a.token_scale, a.offsets, a.wave_docs, a.query, a.scores, a.top_scores,   \
      a.top_ids, a.counter)
    case 1: MSIM_FUSED_CASE(1); break;
    case 2: MSIM_FUSED_CASE(2); break;
    case 3: MSIM_FUSED_CASE(3); break;
    case 4: MSIM_FUSED_CASE(4); break;
    case 5: MSIM_FUSED_CASE(5); break;
    case 6: MSIM_FUSED_CASE(6); break;
    case 7: MSIM_FUSED_CASE(7); break;
    default: MSIM_FUSED_CASE(8); break;
#undef MSIM_FUSED_CASE
  }
}

int fused_waves_per_block() { return kFusedThreads / kWave; }

hipError_t launch_int8q_search(const FusedArgs& args, bool token_scale, hipStream_t stream) {
  const int rows = args.batch * args.query_tokens;
  if (rows <= 0 || rows > 128 || args.num_waves <= 0) return hipErrorInvalidValue;
  if (args.k > kFusedMaxK) return hipErrorInvalidValue;
  const int nt = (rows + 15) / 16;
  const int waves_per_block = kFusedThreads / kWave;
  const int64_t blocks = (args.num_waves + waves_per_block - 1) / waves_per_block;
  if (token_scale) launch_fused_nt<true>(args, nt, blocks, stream);
  else launch_fused_nt<false>(args, nt, blocks, stream);
  return hipGetLastError();
}

}  // namespace msim
