// topk_block.hpp -- top-k of one score row by a workgroup or by one wave,
// shared by the stand-alone top-k kernel and the fused search kernels' tail.
//
// Order restated from the reference: score descending, then position
// ascending (cu:1629-1692 selection order; _api.py:732-735 lexsort).
//
// Scores map to order-preserving 32-bit keys (-0 folded onto +0 so the two
// tie).  A min/max pre-pass finds the highest bit in which the keys differ;
// radix passes of 8 bits from there down (histograms in LDS, one per wave so
// atomics from different waves never collide) find the k-th largest key T.
// Every key above T survives, and among keys equal to T the lowest positions
// survive (a prefix count over contiguous per-thread chunks gives position
// order).  The k survivors are ranked by counting (key desc, position asc)
// and written in order.  Keys stay in registers when a thread's chunk fits
// EPT elements; otherwise each pass re-reads them.
#pragma once

#include "common.hpp"

namespace msim {

__device__ __forceinline__ uint32_t score_key(float s) {
  if (s == 0.0f) s = 0.0f;
  const uint32_t u = __float_as_uint(s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off));
  return v;
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, off));
  return v;
}

__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)v, off);
    if (lane >= off) v += o;
  }
  return v;
}

// Digit search over a 256-bin histogram held as `parts` partial histograms of
// 256 bins each (summed here); run by one full wave.  Returns via *digit and
// *kk_out the digit holding the kk-th largest element and the rank inside it.
__device__ __forceinline__ void find_digit(const uint32_t* hist, int parts, uint32_t kk,
                                           uint32_t* digit, uint32_t* kk_out) {
  const int lane = lane_id();
  uint32_t c[4];
  uint32_t local = 0;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    uint32_t sum = 0;
    for (int p = 0; p < parts; ++p) sum += hist[p * 256 + 255 - 4 * lane - x];
    c[x] = sum;
    local += sum;
  }
  const uint32_t incl = wave_inclusive_scan(local);
  uint32_t above = incl - local;
  if (above < kk && kk <= incl) {
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      if (above < kk && kk <= above + c[x]) {
        *digit = (uint32_t)(255 - 4 * lane - x);
        *kk_out = kk - above;
      }
      above += c[x];
    }
  }
}

// Number of radix passes and the shift of the first one for keys in [lo, hi].
__device__ __forceinline__ int first_shift(uint32_t lo, uint32_t hi) {
  const uint32_t diff = lo ^ hi;
  if (diff == 0) return -1;
  const int top = 31 - __clz((int)diff);  // highest differing bit
  return top >= 7 ? top - 7 : 0;
}

template <int THREADS, int MAXK>
struct TopkSmem {
  uint32_t hist[THREADS / kWave][256];
  uint32_t wave_sum[THREADS / kWave];
  uint32_t wave_min[THREADS / kWave], wave_max[THREADS / kWave];
  uint32_t digit, kk;
  uint32_t count;
  uint32_t key[MAXK];
  int32_t pos[MAXK];
};

// Exclusive prefix sum of one value per thread over the workgroup.
template <int THREADS>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_sum) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const uint32_t incl = wave_inclusive_scan(v);
  if (lane == kWave - 1) wave_sum[wave] = incl;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (int w = 0; w < THREADS / kWave; ++w) {
      const uint32_t t = wave_sum[w];
      wave_sum[w] = run;
      run += t;
    }
  }
  __syncthreads();
  const uint32_t r = wave_sum[wave] + incl - v;
  __syncthreads();
  return r;
}

// Load a score written by other workgroups of the same launch: an
// agent-scope atomic load reads the coherent copy (no L2-wide invalidate).
template <bool kCoherent>
__device__ __forceinline__ float load_score(const float* p) {
  if (kCoherent) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *p;
}

// Rank the k survivors held in key/pos and write them in order.
template <bool kCoherent>
__device__ __forceinline__ void rank_and_write(const uint32_t* skey, const int32_t* spos, int k,
                                               int first, int stride, const float* __restrict__ row,
                                               int64_t n, const int64_t* __restrict__ id_map,
                                               float* __restrict__ out_scores,
                                               int64_t* __restrict__ out_ids) {
  for (int e = first; e < k; e += stride) {
    const uint32_t key = skey[e];
    const int32_t pos = min(max(spos[e], 0), (int32_t)(n - 1));
    int rank = 0;
    for (int o = 0; o < k; ++o) {
      const uint32_t ok = skey[o];
      rank += (ok > key || (ok == key && spos[o] < pos)) ? 1 : 0;
    }
    out_scores[rank] = load_score<kCoherent>(row + pos);
    out_ids[rank] = id_map ? id_map[pos] : (int64_t)pos;
  }
}

// ------------------------------------------------------------ workgroup form
// All THREADS threads must call this together.  1 <= k <= min(n, MAXK).
template <int THREADS, int EPT, int MAXK, bool kCoherent = false>
__device__ void block_topk(const float* __restrict__ row, int64_t n, int k,
                           const int64_t* __restrict__ id_map, float* __restrict__ out_scores,
                           int64_t* __restrict__ out_ids, TopkSmem<THREADS, MAXK>& sm) {
  constexpr int kWaves = THREADS / kWave;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int64_t per = (n + THREADS - 1) / THREADS;
  const int64_t lo = min((int64_t)tid * per, n);
  const int64_t hi = min(lo + per, n);
  const int cnt = (int)(hi - lo);
  const bool cached = per <= EPT;
  uint32_t keys[EPT];
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
  if (cached) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      keys[e] = e < cnt ? score_key(load_score<kCoherent>(row + lo + e)) : 0u;
      if (e < cnt) {
        kmin = min(kmin, keys[e]);
        kmax = max(kmax, keys[e]);
      }
    }
  } else {
    for (int64_t i = lo; i < hi; ++i) {
      const uint32_t key = score_key(load_score<kCoherent>(row + i));
      kmin = min(kmin, key);
      kmax = max(kmax, key);
    }
  }
  kmin = wave_min_u32(kmin);
  kmax = wave_max_u32(kmax);
  if (lane_id() == 0) {
    sm.wave_min[wave] = kmin;
    sm.wave_max[wave] = kmax;
  }
  __syncthreads();
  kmin = 0xFFFFFFFFu;
  kmax = 0u;
  for (int w = 0; w < kWaves; ++w) {
    kmin = min(kmin, sm.wave_min[w]);
    kmax = max(kmax, sm.wave_max[w]);
  }
  const int shift0 = first_shift(kmin, kmax);

  // Bits above shift0 + 7 are equal for every key; passes cover 8 bits each,
  // the last one clamped to shift 0 (its high bits repeat fixed ones).
  uint32_t mask = shift0 < 0 ? 0xFFFFFFFFu : (shift0 + 8 >= 32 ? 0u : ~((2u << (shift0 + 7)) - 1u));
  uint32_t prefix = kmax & mask;
  uint32_t kk = (uint32_t)k;
  for (int shift = shift0; shift >= 0;) {
    uint32_t* myhist = sm.hist[wave];
    for (int i = lane_id(); i < 256; i += kWave) myhist[i] = 0;
    __syncthreads();
    if (cached) {
#pragma unroll
      for (int e = 0; e < EPT; ++e)
        if (e < cnt && (keys[e] & mask) == prefix) atomicAdd(&myhist[(keys[e] >> shift) & 255u], 1u);
    } else {
      for (int64_t i = lo; i < hi; ++i) {
        const uint32_t key = score_key(load_score<kCoherent>(row + i));
        if ((key & mask) == prefix) atomicAdd(&myhist[(key >> shift) & 255u], 1u);
      }
    }
    __syncthreads();
    if (tid < kWave) find_digit(&sm.hist[0][0], kWaves, kk, &sm.digit, &sm.kk);
    __syncthreads();
    prefix |= sm.digit << shift;
    mask |= 255u << shift;
    kk = sm.kk;
    __syncthreads();
    if (shift == 0) break;
    shift = shift > 8 ? shift - 8 : 0;
  }

  uint32_t my_ties = 0;
  if (cached) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) my_ties += (e < cnt && keys[e] == prefix) ? 1u : 0u;
  } else {
    for (int64_t i = lo; i < hi; ++i) my_ties += score_key(load_score<kCoherent>(row + i)) == prefix ? 1u : 0u;
  }
  uint32_t tie_rank = block_exclusive_scan<THREADS>(my_ties, sm.wave_sum);
  if (tid == 0) sm.count = 0;
  for (int e = tid; e < k; e += THREADS) {
    sm.key[e] = 0;
    sm.pos[e] = 0;
  }
  __syncthreads();
  auto consider = [&](uint32_t key, int64_t i) {
    bool keep = key > prefix;
    if (key == prefix) {
      keep = tie_rank < kk;
      ++tie_rank;
    }
    if (keep) {
      const uint32_t slot = atomicAdd(&sm.count, 1u);
      if (slot < (uint32_t)k) {
        sm.key[slot] = key;
        sm.pos[slot] = (int32_t)i;
      }
    }
  };
  if (cached) {
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (e < cnt) consider(keys[e], lo + e);
  } else {
    for (int64_t i = lo; i < hi; ++i) consider(score_key(load_score<kCoherent>(row + i)), i);
  }
  __syncthreads();
  rank_and_write<kCoherent>(sm.key, sm.pos, k, tid, THREADS, row, n, id_map, out_scores, out_ids);
  __syncthreads();
}

// ----------------------------------------------------------------- wave form
// One wave selects the top-k of a row of n <= 64 * EPT scores.  Survivors go
// to skey/spos (k entries, wave-private LDS).  1 <= k <= n.
template <int EPT>
__device__ void wave_topk(const float* __restrict__ row, int64_t n, int k,
                          const int64_t* __restrict__ id_map, float* __restrict__ out_scores,
                          int64_t* __restrict__ out_ids, uint32_t* hist, uint32_t* skey,
                          int32_t* spos) {
  const int lane = lane_id();
  const int64_t per = (n + kWave - 1) / kWave;
  const int64_t lo = min((int64_t)lane * per, n);
  const int cnt = (int)(min(lo + per, n) - lo);
  uint32_t keys[EPT];
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    keys[e] = e < cnt ? score_key(load_score<false>(row + lo + e)) : 0u;
    if (e < cnt) {
      kmin = min(kmin, keys[e]);
      kmax = max(kmax, keys[e]);
    }
  }
  kmin = wave_min_u32(kmin);
  kmax = wave_max_u32(kmax);
  const int shift0 = first_shift(kmin, kmax);
  uint32_t mask = shift0 < 0 ? 0xFFFFFFFFu : (shift0 + 8 >= 32 ? 0u : ~((2u << (shift0 + 7)) - 1u));
  uint32_t prefix = kmax & mask;
  uint32_t kk = (uint32_t)k;
  for (int shift = shift0; shift >= 0;) {
    for (int i = lane; i < 256; i += kWave) hist[i] = 0;
    wave_sync_lds();
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (e < cnt && (keys[e] & mask) == prefix) atomicAdd(&hist[(keys[e] >> shift) & 255u], 1u);
    wave_sync_lds();
    uint32_t c[4];
    uint32_t local = 0;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      c[x] = hist[255 - 4 * lane - x];
      local += c[x];
    }
    const uint32_t incl = wave_inclusive_scan(local);
    uint32_t above = incl - local;
    uint32_t found = 0, d = 0, r = 0;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      if (above < kk && kk <= above + c[x]) {
        found = 1;
        d = (uint32_t)(255 - 4 * lane - x);
        r = kk - above;
      }
      above += c[x];
    }
    // Exactly one lane holds the digit: broadcast it.
    const unsigned long long who = __ballot(found);
    const int src = who ? __ffsll(who) - 1 : 0;
    prefix |= (uint32_t)__shfl((int)d, src) << shift;
    mask |= 255u << shift;
    kk = (uint32_t)__shfl((int)r, src);
    wave_sync_lds();
    if (shift == 0) break;
    shift = shift > 8 ? shift - 8 : 0;
  }

  // Survivors: keys above the threshold, then the first kk ties by position.
  uint32_t my_ties = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) my_ties += (e < cnt && keys[e] == prefix) ? 1u : 0u;
  const uint32_t tie_base = wave_inclusive_scan(my_ties) - my_ties;
  uint32_t tr = tie_base, mine = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if (e < cnt) {
      if (keys[e] > prefix) {
        ++mine;
      } else if (keys[e] == prefix) {
        if (tr < kk) ++mine;
        ++tr;
      }
    }
  }
  uint32_t slot = wave_inclusive_scan(mine) - mine;
  tr = tie_base;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if (e < cnt) {
      bool keep = keys[e] > prefix;
      if (keys[e] == prefix) {
        keep = tr < kk;
        ++tr;
      }
      if (keep && slot < (uint32_t)k) {
        skey[slot] = keys[e];
        spos[slot] = (int32_t)(lo + e);
        ++slot;
      }
    }
  }
  wave_sync_lds();
  rank_and_write<false>(skey, spos, k, lane, kWave, row, n, id_map, out_scores, out_ids);
  wave_sync_lds();
}

}  // namespace msim
