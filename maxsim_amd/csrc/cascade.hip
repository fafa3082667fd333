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
// (n <= per_wave; range(i) gives the token range [start, end) of the group's
// i-th document), their tiles at tiles[(g * waves + w) * cap ...]; the host
// sizes cap as per_wave * (largest document's tile count) + 1.
template <typename Range>
__device__ void candidate_wave_tables(Range range, int64_t m, int64_t g, int64_t waves, int64_t w, int64_t per_wave,
                                      int64_t cap, int64_t* __restrict__ info, uint64_t* __restrict__ tiles) {
  const int64_t id = g * waves + w;
  const int64_t t0 = min(w * per_wave, m);
  const int64_t n = min(per_wave, m - t0);
  const int64_t tab0 = id * cap;
  uint64_t* out = tiles + tab0;
  int64_t k = 0;
  for (int64_t i = 0; i < n; ++i) {
    int64_t s, e;
    range(t0 + i, s, e);
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
  candidate_wave_tables(
      [&](int64_t i, int64_t& b, int64_t& e) {
        const int64_t doc = cands[g * m + i];
        b = offsets[doc];
        e = offsets[doc + 1];
      },
      m, g, waves, id % waves, per_wave, cap, info, tiles);
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

// Sum over each row of 16 lanes, in every lane of the row (DPP quad
// butterflies, then rotations by 4 and 8).
__device__ __forceinline__ uint32_t row_sum16(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true);   // quad_perm [1,0,3,2]
  v += (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
  v += (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, true);  // row_ror:4
  v += (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true);  // row_ror:8
  return v;
}

// Per row of n <= 4096 scores: the m best by (score desc, position asc)
// (the order of _stable_topk, cascade.py:420-453), written as positions in
// ascending order.  Keys are 44 bits, the order-preserving score key above
// 4095 - position: distinct, and larger for a better element.  Radix
// selection of the m-th largest key, 11 bits per round, starting below the
// bits every key of the row shares (scores of one query lie in a narrow
// range, so their top bits agree, and a digit over them would put every key
// in one bin).  A round's histogram counts reversed digits (2047 - digit) in
// 64 groups of 32 (one atomic per key; a pad word after each group keeps
// reads across groups free of bank conflicts); after a barrier each wave
// sums four groups, and after a second one every wave finds the digit itself
// from two wave scans: the group where the running count reaches `need`,
// then the digit inside it.  The rounds stop once the digit's count is what is still needed
// (distinct keys guarantee it once every bit is fixed); the selected keys are
// then those whose fixed bits are at least the prefix.  Positions are
// written in ascending order from ballot counts per (slot, wave), one scan
// over their 64 counts; with tables requested, the selected documents' token
// ranges (loaded with the scores) stay in LDS for the rescoring pass's
// tables.
__global__ __launch_bounds__(1024) void select_topm_kernel(const float* __restrict__ scores, int64_t n,
                                                           int64_t stride, int64_t m, int64_t* __restrict__ out,
                                                           CandidateTables tab) {
  constexpr int kThreads = 1024, kWaves = kThreads / kWave;
  constexpr int E = kSortMaxRow / kThreads;  // positions e * 1024 + t of thread t
  constexpr int kBits = 11, kBins = 1 << kBits, kGroupBins = kBins / kWave, kRounds = 4;
  constexpr int kGroupStride = kGroupBins + 1;  // one pad word per group: conflict-free reads across groups
  static_assert(E * kWaves == kWave, "one lane per (slot, wave) count");
  static_assert(kRounds * kBits >= 44 && kGroupBins == 32 && 4 * kWaves == kWave, "44-bit keys, 64 groups of 32");
  __shared__ uint32_t s_hist[kRounds][kWave * kGroupStride];
  __shared__ uint32_t s_group[kRounds][kWave];
  __shared__ uint32_t s_or[kWaves], s_and[kWaves];
  __shared__ uint32_t s_cnt[E * kWaves];
  __shared__ int64_t s_beg[kSortMaxRow];
  __shared__ uint32_t s_len[kSortMaxRow];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const bool tables = tab.d_info != nullptr;
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(scores + (int64_t)blockIdx.x * stride, (uint32_t)(n * 4));
  const __amdgpu_buffer_rsrc_t roff = make_rsrc(tables ? tab.d_offsets : nullptr, tables ? (uint32_t)((n + 1) * 8) : 0u);
  uint32_t v[E];
  int64_t beg[E], end[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = load_b32(rsrc, (e * kThreads + tid) * 4);
  if (tables) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      beg[e] = (int64_t)load_b64(roff, (e * kThreads + tid) * 8);
      end[e] = (int64_t)load_b64(roff, (e * kThreads + tid + 1) * 8);
    }
  }
  for (int i = tid; i < kRounds * kWave * kGroupStride; i += kThreads) (&s_hist[0][0])[i] = 0u;
  if (tid < kRounds * kWave) (&s_group[0][0])[tid] = 0u;
  uint64_t key[E];
  bool valid[E];
  uint32_t kor = 0u, kand = ~0u;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int p = e * kThreads + tid;
    const uint32_t sk = score_key(__uint_as_float(v[e]));
    valid[e] = p < n;
    key[e] = ((uint64_t)sk << 12) | (uint32_t)(kSortMaxRow - 1 - p);
    if (valid[e]) {
      kor |= sk;
      kand &= sk;
    }
  }
  kor = wave_reduce(kor, [](uint32_t a, uint32_t b) { return a | b; });
  kand = wave_reduce(kand, [](uint32_t a, uint32_t b) { return a & b; });
  if (lane == 0) {
    s_or[wave] = kor;
    s_and[wave] = kand;
  }
  __syncthreads();
  kor = 0u;
  kand = ~0u;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    kor |= s_or[w];
    kand &= s_and[w];
  }
  const uint32_t diff = kor ^ kand;
  const int top = diff != 0u ? 12 + (31 - __clz(diff)) : 11;  // highest bit in which keys may differ
  constexpr uint64_t kKeyMask = (1ull << 44) - 1ull;
  uint64_t mask = (~0ull << (top + 1)) & kKeyMask;
  uint64_t prefix = ((uint64_t)kand << 12) & mask;
  uint32_t need = (uint32_t)m;
  if (m < n) {
    for (int r = 0, hi = top;; ++r, hi -= kBits) {
      const int shift = hi >= kBits - 1 ? hi - (kBits - 1) : 0;
      const uint32_t dbits = (2u << (hi - shift)) - 1u;
      uint32_t* hist = s_hist[r];
      uint32_t* grp = s_group[r];
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (valid[e] && (key[e] & mask) == prefix) {
          const uint32_t rd = (uint32_t)(kBins - 1) - ((uint32_t)(key[e] >> shift) & dbits);
          atomicAdd(&hist[rd + rd / kGroupBins], 1u);
        }
      __syncthreads();
      {  // group totals: wave w sums groups 4 w .. 4 w + 3, two bins per lane
        const int gq = 4 * wave + lane / 16, j0 = 2 * (lane % 16);
        const uint32_t part = row_sum16(hist[gq * kGroupStride + j0] + hist[gq * kGroupStride + j0 + 1]);
        if (lane % 16 == 0) grp[gq] = part;
      }
      __syncthreads();
      const uint32_t gc = grp[lane];
      const uint32_t gincl = wave_inclusive_scan(gc);
      const int g = min((int)__builtin_ctzll(__ballot(gincl >= need)), kWave - 1);
      const uint32_t gabove = (uint32_t)__builtin_amdgcn_readlane((int)(gincl - gc), g);
      const uint32_t dc = lane < kGroupBins ? hist[g * kGroupStride + lane] : 0u;
      const uint32_t dincl = wave_inclusive_scan(dc) + gabove;
      const int j = min((int)__builtin_ctzll(__ballot(dincl >= need)), kGroupBins - 1);
      const uint32_t cnt = (uint32_t)__builtin_amdgcn_readlane((int)dc, j);
      const uint32_t above = (uint32_t)__builtin_amdgcn_readlane((int)dincl, j) - cnt;
      const uint32_t digit = (uint32_t)(kBins - 1) - (uint32_t)(g * kGroupBins + j);
      prefix |= (uint64_t)digit << shift;
      mask |= (uint64_t)dbits << shift;
      need -= above;
      if (cnt == need || shift == 0) break;
    }
  }
  // Stable compaction in position order.
  bool take[E];
  uint64_t bal[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    take[e] = valid[e] && (key[e] & mask) >= prefix;
    bal[e] = __ballot(take[e]);
  }
  uint32_t mine = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) mine = lane == e ? (uint32_t)__popcll(bal[e]) : mine;
  if (lane < E) s_cnt[lane * kWaves + wave] = mine;
  __syncthreads();
  const uint32_t c = s_cnt[lane];
  const uint32_t excl = wave_inclusive_scan(c) - c;
  int64_t* orow = out + (int64_t)blockIdx.x * m;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (take[e]) {
      const uint32_t r = (uint32_t)__builtin_amdgcn_readlane((int)excl, e * kWaves + wave) +
                         __builtin_amdgcn_mbcnt_hi((uint32_t)(bal[e] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal[e], 0u));
      const int p = e * kThreads + tid;
      orow[r] = p;
      if (tables) {
        s_beg[r] = beg[e];
        s_len[r] = (uint32_t)(end[e] - beg[e]);
      }
    }
  if (!tables) return;
  // The rescoring pass's tables of this row (group), from the token ranges in
  // LDS: one thread per wave of the pass.
  __syncthreads();
  for (int64_t w = tid; w < tab.waves; w += kThreads)
    candidate_wave_tables(
        [&](int64_t i, int64_t& b, int64_t& e) {
          b = s_beg[i];
          e = b + s_len[i];
        },
        m, (int64_t)blockIdx.x, tab.waves, w, tab.per_wave, tab.cap, tab.d_info, tab.d_tiles);
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
