// cascade.hip -- device-side pieces of the coarse -> candidates -> rescoring
// cascade (reference: cascade_topk cascade.py:294-393, whose coarse
// selection, per-row candidate rescoring and stable top-k run on the host):
// the candidate lists stay on the device, are put in document order, and the
// rescoring kernel's tile tables are written from them on the device.
#include "common.hpp"
#include "internal.hpp"
#include "topk_block.hpp"

namespace msim {

namespace {

__device__ __forceinline__ uint64_t tile_entry(int64_t start, int64_t rows, bool last, bool empty, int64_t local) {
  return score_tile_entry(start, rows, last, empty, local);
}

// Tables of wave w of group g: its candidates [t0, t0 + n) of the group's m
// (n <= per_wave; cand(i) gives the group's i-th document), their tiles at
// tiles[(g * waves + w) * cap ...]; the host sizes cap as per_wave *
// (largest document's tile count) + 1.
template <typename Cand>
__device__ void candidate_wave_tables(Cand cand, int64_t m, int64_t g, const int64_t* __restrict__ offsets,
                                      int64_t waves, int64_t w, int64_t per_wave, int64_t cap,
                                      int64_t* __restrict__ info, uint64_t* __restrict__ tiles) {
  const int64_t id = g * waves + w;
  const int64_t t0 = min(w * per_wave, m);
  const int64_t n = min(per_wave, m - t0);
  const int64_t tab0 = id * cap;
  uint64_t* out = tiles + tab0;
  int64_t k = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t doc = cand(t0 + i);
    const int64_t s = offsets[doc], e = offsets[doc + 1];
    if (s == e) {
      out[k++] = tile_entry(0, 1, true, true, i);
      continue;
    }
    for (int64_t x = s; x < e; x += 16) out[k++] = tile_entry(x, min<int64_t>(16, e - x), x + 16 >= e, false, i);
  }
  out[k] = tile_entry(0, 1, false, false, 0);
  int64_t* row = info + id * kScoreInfoWords;
  row[0] = t0;
  row[1] = n;
  row[2] = k;
  row[3] = tab0;
}

// One thread per (group, wave).
__global__ __launch_bounds__(256) void candidate_tables_kernel(const int64_t* __restrict__ cands, int64_t m,
                                                               int64_t groups, const int64_t* __restrict__ offsets,
                                                               int64_t waves, int64_t per_wave, int64_t cap,
                                                               int64_t* __restrict__ info,
                                                               uint64_t* __restrict__ tiles) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= groups * waves) return;
  const int64_t g = id / waves;
  candidate_wave_tables([&](int64_t i) { return cands[g * m + i]; }, m, g, offsets, waves, id % waves, per_wave, cap,
                        info, tiles);
}

// Ascending bitonic sort of s[0, pow2) in LDS by the whole block.
template <typename T>
__device__ void bitonic_sort(T* s, int pow2) {
  for (int size = 2; size <= pow2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < pow2; i += blockDim.x) {
        const int j = i ^ stride;
        if (j > i) {
          const bool up = (i & size) == 0;
          const T a = s[i], b = s[j];
          if ((a > b) == up) {
            s[i] = b;
            s[j] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Ascending sort of each row of n <= 4096 int64 values (bitonic, in LDS).
__global__ __launch_bounds__(1024) void sort_rows_kernel(int64_t* __restrict__ rows, int64_t n, int64_t pow2) {
  __shared__ int64_t s[kSortMaxRow];
  int64_t* row = rows + (int64_t)blockIdx.x * n;
  for (int64_t i = threadIdx.x; i < pow2; i += blockDim.x) s[i] = i < n ? row[i] : INT64_MAX;
  __syncthreads();
  bitonic_sort(s, (int)pow2);
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) row[i] = s[i];
}

// Block-wide exclusive prefix sum of one value per thread (1024 threads):
// wave scans by shuffles, then the wave totals.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_wave, uint32_t& total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  uint32_t x = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == kWave - 1) s_wave[wave] = x;
  __syncthreads();
  uint32_t before = 0, all = 0;
  for (int w = 0; w < (int)(blockDim.x / kWave); ++w) {
    const uint32_t t = s_wave[w];
    before += w < wave ? t : 0u;
    all += t;
  }
  __syncthreads();
  total = all;
  return before + x - v;
}

// Per row of n <= 4096 scores: the m best by (score desc, position asc)
// (the order of _stable_topk, cascade.py:420-453), written as positions in
// ascending order.  Radix selection of the m-th largest order-preserving
// score key, 8 bits per round, then a stable compaction: keys above it, and
// the first `need` keys equal to it in position order.
__global__ __launch_bounds__(1024) void select_topm_kernel(const float* __restrict__ scores, int64_t n,
                                                           int64_t stride, int64_t m, int64_t* __restrict__ out,
                                                           CandidateTables tab) {
  constexpr int E = kSortMaxRow / 1024;  // positions 4 t .. 4 t + 3 of thread t
  __shared__ uint32_t s_hist[4][256];
  __shared__ uint32_t s_sel[kSortMaxRow];  // the selected positions, for the tables
  __shared__ uint32_t s_wave[16];
  __shared__ uint32_t s_or[16], s_and[16];
  const int tid = threadIdx.x, lane = tid % kWave;
  const float* row = scores + (int64_t)blockIdx.x * stride;
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(row, (uint32_t)(n * 4));
  uint32_t key[E];
  bool valid[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = E * tid + e;
    valid[e] = i < n;
    key[e] = score_key(__uint_as_float(load_b32(rsrc, i * 4)));
  }
  // The bits every key of the row shares are fixed first: scores of one
  // query lie in a narrow range, so their top bits agree, and a radix digit
  // over them would send every key to one histogram bin (serialised LDS
  // atomics).  The rounds then take 8 bits at a time from the highest bit
  // that varies.
  uint32_t kor = 0u, kand = ~0u;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (valid[e]) {
      kor |= key[e];
      kand &= key[e];
    }
  for (int i = tid; i < 4 * 256; i += blockDim.x) (&s_hist[0][0])[i] = 0u;
  kor = wave_reduce(kor, [](uint32_t a, uint32_t b) { return a | b; });
  kand = wave_reduce(kand, [](uint32_t a, uint32_t b) { return a & b; });
  if (lane == 0) {
    s_or[tid / kWave] = kor;
    s_and[tid / kWave] = kand;
  }
  __syncthreads();
  kor = 0u;
  kand = ~0u;
  for (int w = 0; w < (int)(blockDim.x / kWave); ++w) {
    kor |= s_or[w];
    kand &= s_and[w];
  }
  const uint32_t diff = kor ^ kand;
  const int top = diff == 0u ? -1 : 31 - __clz(diff);  // highest varying bit
  uint32_t mask = top >= 31 ? 0u : ~0u << (top + 1);
  uint32_t prefix = kand & mask, need = (uint32_t)m;
  // One histogram per round (at most four rounds of 8 bits), all zeroed
  // before the reduction's barrier above, and every wave finds the digit
  // itself from the histogram: one barrier per round.
  int round = 0;
  for (int hi = top; hi >= 0; hi -= 8, ++round) {
    const int shift = hi >= 7 ? hi - 7 : 0;
    const uint32_t dmask = (hi - shift == 31 ? ~0u : (2u << (hi - shift)) - 1u);  // digit of bits shift..hi
    uint32_t* hist = s_hist[round];
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (valid[e] && (key[e] & mask) == prefix) atomicAdd(&hist[(key[e] >> shift) & dmask], 1u);
    __syncthreads();
    // Lane l holds digits 4l .. 4l + 3; suffix sums over the lanes from the
    // top digit down find the digit where the count reaches `need` (exactly
    // one lane finds it).
    uint32_t c[4], local = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = hist[4 * lane + j];
      local += c[j];
    }
    uint32_t suffix = local;  // inclusive: lanes >= this one
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const uint32_t y = __shfl_down(suffix, d);
      if (lane + d < kWave) suffix += y;
    }
    uint32_t above = suffix - local;  // digits of higher lanes
    uint32_t digit = 0, above_digit = 0;
    bool found = false;
#pragma unroll
    for (int j = 3; j >= 0; --j) {
      if (above < need && above + c[j] >= need) {
        digit = (uint32_t)(4 * lane + j);
        above_digit = above;
        found = true;
      }
      above += c[j];
    }
    const int src = (int)__builtin_ctzll(__ballot(found));
    prefix |= (uint32_t)__builtin_amdgcn_readlane((int)digit, src) << shift;
    mask |= dmask << shift;
    need -= (uint32_t)__builtin_amdgcn_readlane((int)above_digit, src);
  }
  // Stable compaction in position order.
  uint32_t eq = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) eq += (valid[e] && key[e] == prefix) ? 1u : 0u;
  uint32_t total;
  uint32_t tie_rank = block_exclusive_scan(eq, s_wave, total);
  uint32_t sel = 0;
  bool take[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const bool tie = valid[e] && key[e] == prefix;
    take[e] = valid[e] && (key[e] > prefix || (tie && tie_rank < need));
    tie_rank += tie ? 1u : 0u;
    sel += take[e] ? 1u : 0u;
  }
  uint32_t rank = block_exclusive_scan(sel, s_wave, total);
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (take[e]) {
      out[(int64_t)blockIdx.x * m + rank] = E * tid + e;
      s_sel[rank] = (uint32_t)(E * tid + e);
      ++rank;
    }
  (void)lane;
  if (tab.d_info == nullptr) return;
  // The rescoring pass's tables of this row (group), from the positions in
  // LDS: one thread per wave of the pass.
  __syncthreads();
  for (int64_t w = tid; w < tab.waves; w += blockDim.x)
    candidate_wave_tables([&](int64_t i) { return (int64_t)s_sel[i]; }, m, (int64_t)blockIdx.x, tab.d_offsets,
                          tab.waves, w, tab.per_wave, tab.cap, tab.d_info, tab.d_tiles);
}

}  // namespace

hipError_t launch_candidate_tables(const int64_t* d_cands, int64_t m, int64_t groups, const int64_t* d_offsets,
                                   int64_t waves, int64_t per_wave, int64_t cap, int64_t* d_info,
                                   uint64_t* d_tiles, hipStream_t stream) {
  const int64_t n = groups * waves;
  if (n <= 0) return hipSuccess;
  candidate_tables_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream>>>(
      d_cands, m, groups, d_offsets, waves, per_wave, cap, d_info, d_tiles);
  return hipGetLastError();
}

hipError_t launch_select_topm(const float* d_scores, int64_t batch, int64_t n, int64_t stride, int64_t m,
                              int64_t* d_out, hipStream_t stream, const CandidateTables* tables) {
  if (batch <= 0 || m <= 0) return hipSuccess;
  if (n > kSortMaxRow || m > n) return hipErrorInvalidValue;
  const CandidateTables tab = tables ? *tables : CandidateTables{};
  if (tab.d_info && (tab.d_tiles == nullptr || tab.d_offsets == nullptr || tab.waves <= 0 || tab.per_wave <= 0 ||
                     tab.waves * tab.per_wave < m))
    return hipErrorInvalidValue;
  select_topm_kernel<<<dim3((unsigned)batch), dim3(1024), 0, stream>>>(d_scores, n, stride, m, d_out, tab);
  return hipGetLastError();
}

hipError_t launch_sort_rows(int64_t* d_rows, int64_t batch, int64_t n, hipStream_t stream) {
  if (batch <= 0 || n <= 1) return hipSuccess;
  if (n > kSortMaxRow) return hipErrorInvalidValue;
  int64_t pow2 = 1;
  while (pow2 < n) pow2 <<= 1;
  sort_rows_kernel<<<dim3((unsigned)batch), dim3(1024), 0, stream>>>(d_rows, n, pow2);
  return hipGetLastError();
}

}  // namespace msim
