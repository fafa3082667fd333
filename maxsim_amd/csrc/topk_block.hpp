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

// Integer operations only, so the key of every bit pattern (NaNs included)
// is independent of floating-point compile flags.
__device__ __forceinline__ uint32_t score_key(float s) {
  uint32_t u = __float_as_uint(s);
  if (u == 0x80000000u) u = 0u;  // -0 ties +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, CTRL, 0xF, 0xF, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, true);
  return ((uint64_t)hi << 32) | lo;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_update_u64(uint64_t old, uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)old, (int)(uint32_t)v, CTRL, ROW_MASK, 0xF, false);
  const uint32_t hi =
      (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(old >> 32), (int)(uint32_t)(v >> 32), CTRL, ROW_MASK, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}

// Maximum over the wave, wave-uniform: DPP butterflies and rotations within
// rows of 16 lanes, row broadcasts 15 and 31 into lane 63, then readlane.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  uint64_t o = dpp_u64<0xB1>(v);  // quad_perm [1,0,3,2]
  v = v > o ? v : o;
  o = dpp_u64<0x4E>(v);  // quad_perm [2,3,0,1]
  v = v > o ? v : o;
  o = dpp_u64<0x124>(v);  // row_ror:4
  v = v > o ? v : o;
  o = dpp_u64<0x128>(v);  // row_ror:8
  v = v > o ? v : o;
  o = dpp_update_u64<0x142, 0xA>(v, v);  // row_bcast:15 into rows 1 and 3
  v = v > o ? v : o;
  o = dpp_update_u64<0x143, 0xC>(v, v);  // row_bcast:31 into rows 2 and 3
  v = v > o ? v : o;
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
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

// Inclusive prefix sum over the wave: DPP row shifts by 1, 2, 4 and 8 (zero
// filled at row starts) sum within each row of 16 lanes, then row_bcast:15
// adds the last lane of rows 0 / 2 to rows 1 / 3 and row_bcast:31 the last
// lane of row 1 to rows 2 and 3.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
  auto shr = [](uint32_t x, auto ctrl) -> uint32_t {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, decltype(ctrl)::value, 0xF, 0xF, true);
  };
  v += shr(v, std::integral_constant<int, 0x111>{});  // row_shr:1
  v += shr(v, std::integral_constant<int, 0x112>{});  // row_shr:2
  v += shr(v, std::integral_constant<int, 0x114>{});  // row_shr:4
  v += shr(v, std::integral_constant<int, 0x118>{});  // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15, rows 1 and 3
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31, rows 2 and 3
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

// ----------------------------------------------------------------- tail form
// The int8-query scan's fused selection (int8q_scan.hip): workgroup 0 of the
// launch, once its own documents are done, selects each batch row's top-k,
// one wave per row, from what every workgroup wrote with agent-scope atomic
// stores, read back with coherent loads:
//  * keys [n]: every document's 64-bit full key at its position (the scan's
//    wave order; positions per workgroup are contiguous, block_pos);
//  * rec [3][kTailBlocks]: per workgroup (block) its largest and second largest
//    full keys (none: key 0) and, above the tag, the third largest's 32-bit
//    score key.
// Every entry carries the launch's tag (rec[2]: its low 32 bits, full keys:
// their low kTailTagBits bits, tail_key_tag), and the selection reads an
// entry again until it carries the tag: stores of other workgroups are in
// flight, not missing, so the wait is short.  A wait longer than the
// caller's budget (wait_ticks of s_memrealtime; 0 = no read at all) gives up:
// id -1 and a NaN score in every output slot of the row, and one is added to
// *status, so that the host can tell a given-up row from a result.
//
// Keys: tail_key maps a float's bits to a 32-bit order-preserving key (u ^
// 2^31 for sign bit 0, -u otherwise, so -0 ties +0; every finite float's key
// is >= 2^23, so 0 is below every score); the full key puts 4095 - id, a -0
// flag and the tag below it, so a larger full key is a higher score or, on a
// tie, a lower document id (the reference order; ids are distinct, so flag
// and tag never decide).
//
// Selection: lane l holds the records of blocks l, l + 64, ...; T, the k-th
// largest of the 64 lane maxima (ties counted; each lane counts the maxima at
// least its own), is at most the row's k-th largest score key, because k
// lanes hold a block maximum >= T, each a different document's key.  So
// every key of the top-k is >= T and lies in a block whose maximum is >= T.
// A block whose third score key is below T has all its keys >= T in its
// record; a deeper one has its keys loaded (eight lanes per block, two keys
// each, a second round trip).  The keys >= T are appended to a candidate
// list in LDS and each one's rank counted against the whole list (broadcast
// LDS reads).  More than kTailHotMax deep blocks, a deep one of more than
// kTailBlockKeys documents, more candidates than the list holds, or cap = 0
// fall back to k rounds of a wave maximum over the whole row.  Every step
// after the last record's poll is a fixed sequence of independent
// instructions: one wave selects, and a chain of dependent ones would cost
// it several cycles each.
constexpr int kTailBlocks = 512;                            // workgroups at most
constexpr int kTailBlocksPerLane = kTailBlocks / kWave;     // 8
constexpr int kTailHotMax = 48;                             // hot blocks of the fast path at most
constexpr int kTailBlockKeys = 16;                          // documents per deep block at most
constexpr int kTailMaxDocs = 4096;                          // ids below 2^12
constexpr int kTailTagBits = 19;
constexpr uint32_t kTailTagMask = (1u << kTailTagBits) - 1u;
static_assert(kTailTagMask == kScanTailKeyPeriod, "the scan zeroes the key rows at the key-tag period");
// LDS of the selecting wave: candidates (at most kTailCandMax, then eight
// zero keys, then a spare slot for the stores of lanes without a
// candidate), then the list of deep blocks (kTailHotMax entries and a spare).
constexpr int kTailCandMax = kTailHotMax * kTailBlockKeys;
constexpr int kTailSpare = kTailCandMax + 8;
constexpr int kTailLdsBytes = (kTailCandMax + 9) * 8 + (kTailHotMax + 1) * 4;

__device__ __forceinline__ uint32_t tail_key(uint32_t u) {
  const uint32_t s = (uint32_t)((int32_t)u >> 31);
  return (u ^ (s | 0x80000000u)) - s;
}

// The float of a tail key (+0 for the key of +0 and -0).
__device__ __forceinline__ float tail_key_score(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : (0u - k));
}

// The key tag of a launch tag: never 0, so zeroed entries never carry it.
__device__ __forceinline__ uint32_t tail_key_tag(uint32_t tag) { return tag % kTailTagMask + 1u; }

// Full key of score s of document id < kTailMaxDocs, tagged.
__device__ __forceinline__ uint64_t tail_full_key(float s, uint32_t id, uint32_t tag) {
  const uint32_t u = __float_as_uint(s);
  const uint32_t lo = (((uint32_t)(kTailMaxDocs - 1) - id) << (kTailTagBits + 1)) |
                      ((u == 0x80000000u ? 1u : 0u) << kTailTagBits) | tail_key_tag(tag);
  return ((uint64_t)tail_key(u) << 32) | lo;
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int src) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), src) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, src);
}

// The score and document id of a full key.
__device__ __forceinline__ void tail_write(uint64_t key, float* out_s, int64_t* out_i) {
  const uint32_t lo = (uint32_t)key;
  *out_s = ((lo >> kTailTagBits) & 1u) ? -0.0f : tail_key_score((uint32_t)(key >> 32));
  *out_i = (int64_t)((uint32_t)(kTailMaxDocs - 1) - (lo >> (kTailTagBits + 1)));
}

// Start position and document count of workgroups lane + 64 j (count 0
// past nblocks): static per corpus, so the scan loads them early.
__device__ __forceinline__ void tail_block_ranges(const int64_t* bpos, int nblocks, int (&bs)[kTailBlocksPerLane],
                                                  int (&len)[kTailBlocksPerLane]) {
  const int lane = lane_id();
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(bpos, (uint32_t)(nblocks + 1) * 8u);
#pragma unroll
  for (int j = 0; j < kTailBlocksPerLane; ++j) {
    const int blk = lane + kWave * j;
    bs[j] = (int)load_b64(rp, blk * 8);
    len[j] = (int)load_b64(rp, blk * 8 + 8);
  }
#pragma unroll
  for (int j = 0; j < kTailBlocksPerLane; ++j) len[j] = lane + kWave * j < nblocks ? len[j] - bs[j] : 0;
}

// Inlined into the calling kernel, whose main-loop registers are dead by
// then (a call would save the callee-saved registers it uses to scratch).
// `lds_arg`: wave-private LDS of kTailLdsBytes.  1 <= k <= min(n, 64),
// n <= kTailMaxDocs, nblocks <= kTailBlocks; bs / len from tail_block_ranges.
// Returns false when it gave up (the row holds id -1 / NaN).
__device__ __forceinline__ bool tail_topk(const uint64_t* keys_arg, const uint64_t* rec_arg, int nblocks_arg,
                                          int n_arg, int k_arg, int cap_arg, uint32_t tag_arg, uint64_t* lds_arg,
                                          const int (&bs)[kTailBlocksPerLane], const int (&len)[kTailBlocksPerLane],
                                          float* out_s_arg, int64_t* out_i_arg, uint64_t wait_ticks,
                                          uint32_t* status) {
  const uint64_t* keys = reinterpret_cast<const uint64_t*>(wave_uniform64(reinterpret_cast<int64_t>(keys_arg)));
  const uint64_t* rec = reinterpret_cast<const uint64_t*>(wave_uniform64(reinterpret_cast<int64_t>(rec_arg)));
  float* out_s = reinterpret_cast<float*>(wave_uniform64(reinterpret_cast<int64_t>(out_s_arg)));
  int64_t* out_i = reinterpret_cast<int64_t*>(wave_uniform64(reinterpret_cast<int64_t>(out_i_arg)));
  const int nblocks = wave_uniform(nblocks_arg), n = wave_uniform(n_arg), k = wave_uniform(k_arg);
  const int cap = wave_uniform(cap_arg);
  const uint32_t tag = (uint32_t)wave_uniform((int)tag_arg), ktag = tail_key_tag(tag);
  // `lds_arg` points into LDS: address it as LDS (ds_* instructions).
  typedef __attribute__((address_space(3))) uint64_t lds_u64;
  typedef __attribute__((address_space(3))) uint32_t lds_u32;
  lds_u64* cand = (lds_u64*)lds_arg;
  lds_u32* deep_list = (lds_u32*)(cand + kTailSpare + 1);
  const int lane = lane_id();
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(keys, (uint32_t)n * 8u);
  const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
  auto expired = [&]() { return __builtin_amdgcn_s_memrealtime() - t_start > wait_ticks; };
  auto give_up = [&]() {
    if (lane < k) {
      out_s[lane] = __uint_as_float(0x7FC00000u);  // quiet NaN by its bits (device code is built without NaN semantics)
      out_i[lane] = -1;
    }
    if (lane == 0) __hip_atomic_fetch_add(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if (wait_ticks == 0) {
    give_up();
    return false;
  }
  auto rank_below = [&](uint64_t mask) -> int {  // set bits of mask below this lane
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
  };
  auto key_current = [&](uint64_t x) { return ((uint32_t)x & kTailTagMask) == ktag; };

  // T of the lane maxima lmax: the largest lane maximum that k lane maxima
  // reach (ties counted).  Each lane counts the lane maxima at least its own
  // (broadcast reads of all 64 from LDS, independent compares); T is the
  // largest maximum whose count reaches k.  T >= 1, so blocks without
  // documents (maximum 0) are never hot.
  lds_u32* lm = (lds_u32*)cand;
  auto threshold = [&](uint32_t lmax) -> uint32_t {
    lm[lane] = lmax;
    wave_sync_lds();
    int ge0 = 0, ge1 = 0;
#pragma unroll
    for (int j = 0; j < kWave; j += 8) {
      const v4u q0 = *(const __attribute__((address_space(3))) v4u*)(lm + j);
      const v4u q1 = *(const __attribute__((address_space(3))) v4u*)(lm + j + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ge0 += q0[e] >= lmax ? 1 : 0;
        ge1 += q1[e] >= lmax ? 1 : 0;
      }
    }
    const uint32_t tt = max(wave_reduce(ge0 + ge1 >= k ? lmax : 0u, [](uint32_t x, uint32_t y) { return max(x, y); }), 1u);
    wave_sync_lds();
    return tt;
  };

  // Round trip 1: the records (out of range: 0; a block without documents
  // still writes one), read until every word carries the tag.  Once at
  // most half the lanes still wait, T is computed ahead from the current
  // records (stale words count as 0) while the next poll is in flight, each
  // time the lane maxima changed: they only grow, and if none that changed
  // since ends at or above that T, the final T is the same (the lane maxima
  // at or above it are the same multiset).
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(rec, (uint32_t)(3 * kTailBlocks * 8));
  uint64_t w0[kTailBlocksPerLane], w1[kTailBlocksPerLane];
  uint32_t third[kTailBlocksPerLane];
  uint64_t ra[kTailBlocksPerLane], rb[kTailBlocksPerLane], rc[kTailBlocksPerLane];
  auto issue_poll = [&]() {
#pragma unroll
    for (int j = 0; j < kTailBlocksPerLane; ++j) {
      const int blk = lane + kWave * j;
      ra[j] = load_b64_coherent(rr, blk * 8);
      rb[j] = load_b64_coherent(rr, (kTailBlocks + blk) * 8);
      rc[j] = load_b64_coherent(rr, (2 * kTailBlocks + blk) * 8);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  uint32_t t_ahead = 0, lmax_ahead = 0;  // t_ahead 0: none computed
  issue_poll();
  for (;;) {
    uint32_t stale = 0;
#pragma unroll
    for (int j = 0; j < kTailBlocksPerLane; ++j) {
      const bool in = lane + kWave * j < nblocks;
      w0[j] = in ? ra[j] : 0ull;
      w1[j] = in ? rb[j] : 0ull;
      third[j] = in ? (uint32_t)(rc[j] >> 32) : 0u;
      stale |= (uint32_t)in & ((uint32_t)!key_current(ra[j]) | (uint32_t)!key_current(rb[j]) |
                               (uint32_t)((uint32_t)rc[j] != tag));
    }
    const uint64_t stale_lanes = __ballot(stale != 0);
    if (stale_lanes == 0) break;
    if (expired()) {
      give_up();
      return false;
    }
    // Poll gently while many workgroups are still scanning (the polls take
    // issue slots from the scan waves sharing this CU), then closely, and
    // compute T ahead when the current records changed it may.  A poll
    // takes 1-2 us to return while the scan streams, and the last third of
    // the records lands within the last 1.5 us, so even the gentle pause is
    // short (8 x 64 clocks; 32 x 64 left the last poll before the end
    // seeing 100-250 stale records and cost 0.3 us per launch).
    const int nstale = __popcll(stale_lanes);
    uint32_t lf = 0;
#pragma unroll
    for (int j = 0; j < kTailBlocksPerLane; ++j) lf = max(lf, key_current(w0[j]) ? (uint32_t)(w0[j] >> 32) : 0u);
    const bool ahead = nstale <= 32 && (t_ahead == 0 || __ballot(lf != lmax_ahead) != 0);
    if (nstale > 32) __builtin_amdgcn_s_sleep(8);
    else if (!ahead && nstale > 4) __builtin_amdgcn_s_sleep(8);
    else if (!ahead) __builtin_amdgcn_s_sleep(1);
    issue_poll();
    if (ahead) {  // while the poll is in flight
      lmax_ahead = lf;
      t_ahead = threshold(lf);
    }
  }
  uint32_t lmax = 0;
#pragma unroll
  for (int j = 0; j < kTailBlocksPerLane; ++j) lmax = max(lmax, (uint32_t)(w0[j] >> 32));
  const bool ahead_holds = t_ahead != 0 && __ballot(lmax != lmax_ahead && lmax >= t_ahead) == 0;
  const uint32_t t = ahead_holds ? t_ahead : threshold(lmax);
  // Per lane: its deep blocks (a third key >= T: all their keys are loaded;
  // bit j of dmask) and the record keys >= T of its other blocks (bits 2j,
  // 2j + 1 of cmask).  One scan gives every lane its offsets; each lane then
  // writes its 16 record keys and 8 block ranges unconditionally, those it
  // does not hold to a spare slot (no branches: one wave runs this, and a
  // branch costs it far more than a store).
  uint32_t dmask = 0, cmask = 0, wide = 0;
#pragma unroll
  for (int j = 0; j < kTailBlocksPerLane; ++j) {
    const uint32_t d = third[j] >= t ? 1u : 0u;
    dmask |= d << j;
    wide |= d & (len[j] > kTailBlockKeys ? 1u : 0u);
    cmask |= ((d ^ 1u) & ((uint32_t)(w0[j] >> 32) >= t ? 1u : 0u)) << (2 * j);
    cmask |= ((d ^ 1u) & ((uint32_t)(w1[j] >> 32) >= t ? 1u : 0u)) << (2 * j + 1);
  }
  const uint32_t lc = (uint32_t)__popc(cmask), ld = (uint32_t)__popc(dmask);
  const uint32_t incl = wave_inclusive_scan((lc << 16) | ld);
  const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
  const int ndeep = (int)(tot & 0xFFFFu);
  int ncand = (int)(tot >> 16);
  const bool fast = cap > 0 && ndeep <= kTailHotMax && __ballot(wide != 0) == 0 &&
                    ncand + kTailBlockKeys * ndeep <= kTailCandMax;
  if (fast) {
    const uint32_t cbase = (incl >> 16) - lc, dbase = (incl & 0xFFFFu) - ld;
#pragma unroll
    for (int slot = 0; slot < 2 * kTailBlocksPerLane; ++slot) {
      const uint64_t key = (slot & 1) ? w1[slot >> 1] : w0[slot >> 1];
      const uint32_t at = cbase + (uint32_t)__popc(cmask & ((1u << slot) - 1u));
      cand[((cmask >> slot) & 1u) ? at : (uint32_t)kTailSpare] = key;
    }
    if (ndeep > 0) {
#pragma unroll
      for (int j = 0; j < kTailBlocksPerLane; ++j) {
        const uint32_t at = dbase + (uint32_t)__popc(dmask & ((1u << j) - 1u));
        deep_list[((dmask >> j) & 1u) ? at : (uint32_t)kTailHotMax] = ((uint32_t)bs[j] << 8) | (uint32_t)len[j];
      }
    }
  }
  if (fast) {
    if (ndeep > 0) {
      wave_sync_lds();
      // Round trip 2: eight lanes per deep block, two keys each (past the
      // block's count: out of range, key 0), all rounds issued together,
      // read until every key carries the tag.
      constexpr int kRounds = (kTailHotMax + 7) / 8;
      const int sub = 2 * (lane & 7);
      int start[kRounds], cnt[kRounds];
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        const int h = 8 * r + (lane >> 3);
        const uint32_t hb = h < ndeep ? (uint32_t)deep_list[h] : 0u;
        start[r] = (int)(hb >> 8) + sub;
        cnt[r] = (int)(hb & 255u) - sub;
      }
      uint64_t x[2 * kRounds];
      for (;;) {
        uint32_t st = 0;
#pragma unroll
        for (int r = 0; r < kRounds; ++r) {
          if (8 * r >= ndeep) break;
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            x[2 * r + e] = load_b64_coherent(rk, e < cnt[r] ? (start[r] + e) * 8 : n * 8);
            st |= (uint32_t)(e < cnt[r]) & (uint32_t)!key_current(x[2 * r + e]);
          }
        }
        if (__ballot(st != 0) == 0) break;
        if (expired()) {
          give_up();
          return false;
        }
        __builtin_amdgcn_s_sleep(1);
      }
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        if (8 * r >= ndeep) break;
        const uint64_t x0 = x[2 * r], x1 = x[2 * r + 1];
        const bool c0 = (uint32_t)(x0 >> 32) >= t, c1 = (uint32_t)(x1 >> 32) >= t;
        const uint64_t m0 = __ballot(c0), m1 = __ballot(c1);
        if (c0) cand[ncand + rank_below(m0)] = x0;
        if (c1) cand[ncand + __popcll(m0) + rank_below(m1)] = x1;
        ncand += __popcll(m0) + __popcll(m1);
      }
    }
    // Rank of each candidate: the candidates above it (distinct full keys),
    // counted over the list eight at a time (zero keys pad it).
    if (lane < 8) cand[ncand + lane] = 0ull;
    wave_sync_lds();
    for (int i0 = 0; i0 < ncand; i0 += kWave) {
      const int i = i0 + lane;
      const uint64_t y = i < ncand ? (uint64_t)cand[i] : ~0ull;
      int r = 0;
      for (int j = 0; j < ncand; j += 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) r += (uint64_t)cand[j + e] > y ? 1 : 0;
      }
      if (i < ncand && r < k) tail_write(y, out_s + r, out_i + r);
    }
    wave_sync_lds();
    return true;
  }
  // Fallback: wait until every key of the row carries the tag, then k
  // rounds over the row (read again each round): the largest full key below
  // the previous round's.
  const int chunks = (n + 2 * kWave - 1) / (2 * kWave);
  for (;;) {
    bool stale = false;
#pragma unroll 1
    for (int i = 0; i < chunks; ++i) {
      const int p = 2 * (i * kWave + lane);
      const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rk, p * 8, 0, kCoherentLoadPolicy);
      stale = stale || (p < n && (v[0] & kTailTagMask) != ktag) || (p + 1 < n && (v[2] & kTailTagMask) != ktag);
    }
    if (__ballot(stale) == 0) break;
    if (expired()) {
      give_up();
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  uint64_t prev = ~0ull;
  for (int r = 0; r < k; ++r) {
    uint64_t best = 0;
#pragma unroll 1
    for (int i = 0; i < chunks; ++i) {
      const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rk, (i * kWave + lane) * 16, 0, kCoherentLoadPolicy);
      const uint64_t a = ((uint64_t)v[1] << 32) | v[0], b = ((uint64_t)v[3] << 32) | v[2];
      best = (a < prev && a > best) ? a : best;
      best = (b < prev && b > best) ? b : best;
    }
    const uint64_t top = wave_max_u64(best);
    if (lane == 0) tail_write(top, out_s + r, out_i + r);
    prev = top;
  }
  return true;
}

}  // namespace msim
