// int8q.hip -- per-token int4 documents x int8-quantised queries on gfx950 MFMA.
//
// Semantics restated from the reference: query quantisation
// tests/test_int4_int8q.py:11-14 (device form cu:1455-1492) and the
// token-scaled MaxSim cu:1569-1627 / tests/test_int4_int8q.py:15-26.
//
// Design (MI355X): one wave walks whole documents.  A 16-token tile of the
// document is the MFMA A operand (16 rows x 128 dims, int4 nibbles widened
// to int8 in registers), every query row is a B column held in registers
// for the life of the wave, so each code byte read from HBM feeds all
// B*Q <= 128 query rows.  v_mfma_i32_16x16x64_i8 accumulates exact int32
// dot products; the epilogue scales by the token scale (scale before max),
// keeps a per-lane running max and finishes each document with a
// cross-lane max and numpy's float64 pairwise sum over query tokens.
#include <algorithm>

#include "common.hpp"
#include "internal.hpp"

namespace msim {

// ---------------------------------------------------------------- quantise

// One wave per query row of 128 dims: sigma = f32(max|q| / 127) (0 -> 1),
// q8 = clip(rint(q / sigma), -127, 127) with a correctly rounded divide.
// bias = -8 * sum(q8) undoes the +8 offset the row-pass kernel's nibble
// unpack adds to every document code.  Two layouts of the codes (the MFMA B
// operands):
//  * row order (pass_rows == 0; the row-pass kernel): row r at r * 128, where
//    for lane group g = 0..3 bytes [32g, 32g+16) hold dims 32g+2i (i = 0..15)
//    and bytes [32g+16, 32g+32) dims 32g+2i+1 -- the low and high nibbles of
//    the document bytes 16g..16g+15;
//  * lane order (pass_rows > 0; the scan): the rows of scan pass p (rows
//    [p * pass_rows, (p + 1) * pass_rows)) fill a region of TP = ceil(pass_rows
//    / 16) tiles of 2 KiB; in tile j the 16 bytes lane (g, c) holds -- row 16j
//    + c, dims 32g+2i (half 0) or 32g+2i+1 (half 1) -- sit at (2j + half) *
//    1024 + (16g + c) * 16, so a wave reads each half-tile as one linear
//    1 KiB run.  Slots of no row hold zeros.
// Items t < rows_padded also write qscale[t] / qbias[t] (0 past `rows`).
__global__ __launch_bounds__(256) void quantize_query_int8_kernel(
    const float* __restrict__ query, int64_t rows, int64_t rows_padded, int64_t pass_rows, int64_t items,
    int8_t* __restrict__ qpack, float* __restrict__ qscale, int32_t* __restrict__ qbias) {
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (t >= items) return;
  const int g = lane >> 4, i = lane & 15;
  int64_t row = t;
  int8_t *dst0 = nullptr, *dst1 = nullptr;  // byte destinations of dims 2 * lane and 2 * lane + 1
  bool valid = t < rows;
  if (pass_rows > 0) {
    const int64_t tp = (pass_rows + 15) / 16;
    const int64_t slots = ((rows + pass_rows - 1) / pass_rows) * tp * 16;
    if (t < slots) {
      const int64_t pass = t / (tp * 16), rl = t % (tp * 16);
      row = pass * pass_rows + rl;
      valid = rl < pass_rows && row < rows;
      int8_t* tile = qpack + (pass * tp + rl / 16) * 2048 + (16 * g + rl % 16) * 16 + i;
      dst0 = tile;
      dst1 = tile + 1024;
    } else {
      valid = false;
    }
    if (t >= rows && t < rows_padded && lane == 0) {
      qscale[t] = 0.0f;
      qbias[t] = 0;
    }
  } else if (t < rows_padded) {
    dst0 = qpack + t * 128 + 32 * g + i;
    dst1 = dst0 + 16;
    if (!valid && lane == 0) {
      qscale[t] = 0.0f;
      qbias[t] = 0;
    }
  }
  if (!valid) {
    if (dst0 != nullptr) {
      *dst0 = 0;
      *dst1 = 0;
    }
    return;
  }
  const float2 v = reinterpret_cast<const float2*>(query + row * 128)[lane];
  const float m = wave_reduce(fmaxf(fabsf(v.x), fabsf(v.y)), [](float x, float y) { return fmaxf(x, y); });
  const float s = m == 0.0f ? 1.0f : __fdiv_rn(m, 127.0f);
  const int a = max(-127, min(127, (int)rintf(__fdiv_rn(v.x, s))));
  const int b = max(-127, min(127, (int)rintf(__fdiv_rn(v.y, s))));
  const int sum = wave_reduce(a + b, [](int x, int y) { return x + y; });
  *dst0 = (int8_t)a;
  *dst1 = (int8_t)b;
  if (lane == 0) {
    qscale[row] = s;
    qbias[row] = -8 * sum;
  }
}

// ------------------------------------------------------------------ score

// Per-wave scratch for the per-row maxima of one document.
constexpr int kRowsPerPass = 128;

__device__ __forceinline__ void wave_lds_sync() { wave_sync_lds(); }

// Finish one document: out[b] = f32(pairwise_f64(max[b,q] * sigma[b,q]) * scale)
// for the `batch` rows held in `rowmax` (query_tokens per batch row).
__device__ __forceinline__ void finish_doc(const float* rowmax, const float* __restrict__ qscale,
                                           int batch, int query_tokens, double scale,
                                           float* __restrict__ out, int64_t out_stride) {
  const int lane = lane_id();
  auto prod = [&](int r) -> double { return (double)rowmax[r] * (double)qscale[r]; };
  if (query_tokens < 8) {
    for (int b = lane; b < batch; b += kWave) {
      double res = 0.0;
      for (int q = 0; q < query_tokens; ++q) res = __dadd_rn(res, prod(b * query_tokens + q));
      out[(int64_t)b * out_stride] = (float)(res * scale);
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
      out[(int64_t)b * out_stride] = (float)(r * scale);
    }
  }
}

// NT: number of 16-row query tiles held in registers (rows = 16 * NT <= 128).
// kTokenScale: per-token document scales (int4_per_token) vs tensor scale.
// kFinish: finish documents in-kernel (rows hold whole batch rows); otherwise
// write the per-row maxima to rowmax_out[row * num_docs + doc].
template <int NT, bool kTokenScale, bool kFinish>
__global__ __launch_bounds__(256) void int8q_maxsim_kernel(Int8qArgs p) {
  __shared__ float s_rowmax[4][kRowsPerPass];
  const int lane = lane_id();
  const int wave = wave_uniform(threadIdx.x / kWave);
  const int g = lane >> 4, c = lane & 15;
  const int64_t gwave = (int64_t)blockIdx.x * (blockDim.x / kWave) + wave;
  const int64_t doc_begin = gwave * p.docs_per_wave;
  if (doc_begin >= p.num_docs) return;
  const int64_t doc_end = min(doc_begin + (int64_t)p.docs_per_wave, p.num_docs);

  // Query tiles: lane (g, c) holds row 16j + c, dims of lane group g.
  v4i blo[NT], bhi[NT];
  int bias[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const v4i* src = reinterpret_cast<const v4i*>(p.qpack + (int64_t)(16 * j + c) * 128 + 32 * g);
    blo[j] = src[0];
    bhi[j] = src[1];
    bias[j] = p.qbias[16 * j + c];
  }

  float* rowmax = s_rowmax[wave];

  for (int64_t doc = doc_begin; doc < doc_end; ++doc) {
    const int64_t start = p.offsets[doc];
    const int64_t end = p.offsets[doc + 1];
    if (start == end) {
      if (kFinish) {
        for (int b = lane; b < p.batch; b += kWave) p.out[(int64_t)b * p.out_stride + doc] = 0.0f;
      } else if (g == 0) {
#pragma unroll
        for (int j = 0; j < NT; ++j)
          if (16 * j + c < p.rows_valid) p.rowmax_out[(int64_t)(16 * j + c) * p.num_docs + doc] = kNegInf;
      }
      continue;
    }
    // Buffer descriptors rebased on this document: byte offsets stay small
    // for any corpus size, and rows past the document end read as zero.
    const int64_t len = end - start;
    const __amdgpu_buffer_rsrc_t codes = make_rsrc(p.codes + start * 64, (uint32_t)(len * 64));
    const __amdgpu_buffer_rsrc_t scales =
        make_rsrc(kTokenScale ? (const void*)(p.token_scale + start) : (const void*)p.codes,
                  kTokenScale ? (uint32_t)(len * 4) : 0u);
    float m[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) m[j] = kNegInf;

    for (int64_t t0 = 0; t0 < len; t0 += 16) {
      const uint32_t code_off = (uint32_t)(t0 + c) * 64u + 16u * (uint32_t)g;
      const v4u raw = load_b128(codes, (int)code_off);
      float s0 = 1.0f, s1 = 1.0f, s2 = 1.0f, s3 = 1.0f;
      if (kTokenScale) {
        const v4u sv = load_b128(scales, (int)((uint32_t)(t0 + 4 * g) * 4u));
        s0 = __uint_as_float(sv.x);
        s1 = __uint_as_float(sv.y);
        s2 = __uint_as_float(sv.z);
        s3 = __uint_as_float(sv.w);
      }
      // Offset-binary unpack: nibble ^ 8 = value + 8 in [1, 15]; the query
      // bias -8 * sum(q8) in the accumulator removes the offset exactly.
      v4i lo, hi;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const unsigned w = raw[x] ^ 0x88888888u;
        lo[x] = (int)(w & 0x0F0F0F0Fu);
        hi[x] = (int)((w >> 4) & 0x0F0F0F0Fu);
      }
      const int64_t rem = len - t0;  // valid rows in this tile (>= 1)
      const int row0 = 4 * g;
      v4i accs[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j)
        accs[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(lo, blo[j], (v4i){bias[j], bias[j], bias[j], bias[j]}, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < NT; ++j) accs[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(hi, bhi[j], accs[j], 0, 0, 0);
      mfma_results_fence();
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const v4i acc = accs[j];
        float x0 = (float)acc[0], x1 = (float)acc[1], x2 = (float)acc[2], x3 = (float)acc[3];
        if (kTokenScale) {
          x0 = x0 * s0;
          x1 = x1 * s1;
          x2 = x2 * s2;
          x3 = x3 * s3;
        }
        if (rem < 16) {
          x0 = row0 + 0 < rem ? x0 : kNegInf;
          x1 = row0 + 1 < rem ? x1 : kNegInf;
          x2 = row0 + 2 < rem ? x2 : kNegInf;
          x3 = row0 + 3 < rem ? x3 : kNegInf;
        }
        m[j] = fmax3(m[j], x0, x1);
        m[j] = fmax3(m[j], x2, x3);
      }
    }

    // Max across the four lane groups: lane c of every group then holds the
    // document max of query row 16j + c.
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      m[j] = fmaxf(m[j], __shfl_xor(m[j], 16));
      m[j] = fmaxf(m[j], __shfl_xor(m[j], 32));
    }
    if (kFinish) {
      if (g == 0) {
#pragma unroll
        for (int j = 0; j < NT; ++j) rowmax[16 * j + c] = m[j];
      }
      wave_lds_sync();
      finish_doc(rowmax, p.qscale, p.batch, p.query_tokens, p.scale, p.out + doc, p.out_stride);
      wave_lds_sync();
    } else if (g == 0) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
        if (16 * j + c < p.rows_valid) p.rowmax_out[(int64_t)(16 * j + c) * p.num_docs + doc] = m[j];
    }
  }
}

// Finish kernel for query_tokens > 128: one wave per (batch row, doc).
__global__ __launch_bounds__(256) void int8q_finish_kernel(const float* __restrict__ rowmax,
                                                           const float* __restrict__ qscale,
                                                           int64_t batch, int64_t query_tokens,
                                                           int64_t num_docs, double scale,
                                                           const int64_t* __restrict__ offsets,
                                                           float* __restrict__ out) {
  const int64_t item = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (item >= batch * num_docs) return;
  if (lane_id() != 0) return;
  const int64_t b = item / num_docs, doc = item % num_docs;
  if (offsets[doc] == offsets[doc + 1]) {
    out[b * num_docs + doc] = 0.0f;
    return;
  }
  const float* rm = rowmax + (b * query_tokens) * num_docs + doc;
  const float* qs = qscale + b * query_tokens;
  auto get = [&](int64_t q) -> double { return (double)rm[q * num_docs] * (double)qs[q]; };
  out[b * num_docs + doc] = (float)(pairwise_sum_serial(get, query_tokens) * scale);
}

// ------------------------------------------------------------------ launch

int64_t scan_qpack_bytes(int64_t rows, int64_t pass_rows) {
  if (rows <= 0 || pass_rows <= 0) return 0;
  return ((rows + pass_rows - 1) / pass_rows) * ((pass_rows + 15) / 16) * 2048;
}

hipError_t launch_quantize_int8(const float* d_query, int64_t rows, int64_t rows_padded,
                                int8_t* d_qpack, float* d_qscale, int32_t* d_qbias,
                                hipStream_t stream, int64_t pass_rows) {
  const int64_t slots = scan_qpack_bytes(rows, pass_rows) / 128;  // 16 rows per 2 KiB tile
  const int64_t items = std::max<int64_t>(rows_padded, slots);
  const int64_t blocks = (items + 3) / 4;
  if (blocks == 0) return hipSuccess;
  quantize_query_int8_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(
      d_query, rows, rows_padded, pass_rows, items, d_qpack, d_qscale, d_qbias);
  return hipGetLastError();
}

template <int NT, bool kTS, bool kFin>
static void launch_nt(const Int8qArgs& a, int64_t blocks, hipStream_t stream) {
  int8q_maxsim_kernel<NT, kTS, kFin><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(a);
}

template <bool kTS, bool kFin>
static void launch_ts(const Int8qArgs& a, int nt, int64_t blocks, hipStream_t stream) {
  switch (nt) {
    case 1: launch_nt<1, kTS, kFin>(a, blocks, stream); break;
    case 2: launch_nt<2, kTS, kFin>(a, blocks, stream); break;
    case 3: launch_nt<3, kTS, kFin>(a, blocks, stream); break;
    case 4: launch_nt<4, kTS, kFin>(a, blocks, stream); break;
    case 5: launch_nt<5, kTS, kFin>(a, blocks, stream); break;
    case 6: launch_nt<6, kTS, kFin>(a, blocks, stream); break;
    case 7: launch_nt<7, kTS, kFin>(a, blocks, stream); break;
    default: launch_nt<8, kTS, kFin>(a, blocks, stream); break;
  }
}

hipError_t launch_int8q_maxsim(const Int8qArgs& args, int rows_in_pass, bool token_scale,
                               bool finish, hipStream_t stream) {
  if (args.num_docs == 0) return hipSuccess;
  const int nt = (rows_in_pass + 15) / 16;
  const int64_t waves = (args.num_docs + args.docs_per_wave - 1) / args.docs_per_wave;
  const int64_t blocks = (waves + 3) / 4;
  if (token_scale) {
    if (finish) launch_ts<true, true>(args, nt, blocks, stream);
    else launch_ts<true, false>(args, nt, blocks, stream);
  } else {
    if (finish) launch_ts<false, true>(args, nt, blocks, stream);
    else launch_ts<false, false>(args, nt, blocks, stream);
  }
  return hipGetLastError();
}

hipError_t launch_int8q_finish(const float* d_rowmax, const float* d_qscale, int64_t batch,
                               int64_t query_tokens, int64_t num_docs, double scale,
                               const int64_t* d_offsets, float* d_out, hipStream_t stream) {
  const int64_t items = batch * num_docs;
  if (items == 0) return hipSuccess;
  const int64_t blocks = (items + 3) / 4;
  int8q_finish_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(
      d_rowmax, d_qscale, batch, query_tokens, num_docs, scale, d_offsets, d_out);
  return hipGetLastError();
}

}  // namespace msim
