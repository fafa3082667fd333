// int8q_scan.hip -- int4 documents x int8-quantised queries: full-corpus scan
// on gfx950 MFMA.
//
// Semantics restated from the reference: token-scaled MaxSim cu:1569-1627 /
// tests/test_int4_int8q.py:15-26 (scale before max, empty doc -> 0), with the
// query rows already quantised by quantize_query_int8_kernel (int8q.hip).
// Scores equal the C oracle bit for bit.
//
// Work split: every wave owns a contiguous range of documents (balanced by
// 16-token tiles on the host, see ScanArgs) and walks its non-empty
// documents as one stream of 16-token tiles.  The four waves of a workgroup
// are independent (no barriers).
//  * a document of len >= 16 tokens is covered by ceil(len / 16) tiles whose
//    last one is shifted back to end at the document end (it re-reads up to
//    15 tokens: max is idempotent), so every tile has 16 valid rows; only
//    documents shorter than 16 tokens need row masking;
//  * kPrefetch tiles of codes and token scales are in flight per wave,
//    loaded global -> LDS into a per-wave ring and read back one tile ahead
//    of use; every global load is issued without compiler tracking and
//    waited for explicitly (common.hpp), so the steady state has exactly one
//    vmcnt wait per tile;
//  * the query tiles (B operands, <= 128 rows) live in registers for the
//    life of the wave; v_mfma_i32_16x16x64_i8 forms exact dots with each code
//    byte's nibbles masked in place as int8 (hi = w & 0xF0, lo = (w << 4) &
//    0xF0), i.e. sixteen times the signed value, so acc = 16 * dot and
//    float(acc) * (s_t / 16) rounds the same real number as float(dot) * s_t;
//  * per tile: 16 MFMAs, then the VALU epilogue (scale, running max); the
//    two waves of a SIMD overlap one's MFMAs with the other's VALU work;
//  * at a document end: cross-lane max over the four lane groups and numpy's
//    float64 pairwise sum over query tokens; for 32-token queries entirely
//    in registers (permlane swaps scatter batch row b to lane group b, DPP
//    moves order the pairwise sum), otherwise through LDS;
//  * fused selection (ScanArgs::topk_k > 0): scores are stored write-through
//    as tagged keys, each workgroup's largest key per batch row likewise;
//    workgroup 0, once its own documents are done, waits until what it reads
//    carries the launch's tag and selects each batch row's top-k
//    (topk_block.hpp, tail form), one wave per row, in its own LDS.
#include "common.hpp"
#include "internal.hpp"
#include "topk_block.hpp"

namespace msim {

constexpr int kScanThreads = 256;
constexpr int kScanWaves = kScanThreads / kWave;
constexpr int kPrefetch = kScanPrefetch;  // tiles in flight per wave
static_assert(kPrefetch >= 2, "ring of at least two tiles");
static_assert(kScanTailBlocks == kTailBlocks && kScanTailMaxDocs <= kScanTailRow && kScanTailMaxDocs <= kTailMaxDocs,
              "fused selection sizes");
static_assert(kScanTailMaxRows <= kScanThreads, "one thread per batch row writes the block maxima");
static_assert(kPrefetch * kWave * 16 >= kTailLdsBytes, "a wave's tile ring holds the selection's candidates");
static_assert(kScanTailMaxK <= 32, "fused selection k: the selection's list holds 32 keys");

// Maximum over the four lane groups (lanes l, l ^ 16, l ^ 32, l ^ 48).
__device__ __forceinline__ float max_over_groups(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}

// Reduce-scatter of eight per-lane tile maxima over the four lane groups:
// group g ends with the maxima of tiles 2g (t0) and 2g + 1 (t1).  A
// permlane32 swap of (m[a], m[a + 4]) leaves tile a in lanes 0..31 and tile
// a + 4 in lanes 32..63, each reduced over the two halves; a permlane16 swap
// of (x[a], x[a + 2]) then reduces over the two rows of each half.  Tiles
// past NT are -inf.
template <int NT>
__device__ __forceinline__ void max_scatter_groups(const float (&m)[NT], float& t0, float& t1) {
  auto mm = [&](int j) { return j < NT ? m[j] : kNegInf; };
  auto swap_max = [](float a, float b, auto swap) {
    const auto r = swap(__float_as_uint(a), __float_as_uint(b));
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  };
  auto sw32 = [](uint32_t a, uint32_t b) { return __builtin_amdgcn_permlane32_swap(a, b, false, false); };
  auto sw16 = [](uint32_t a, uint32_t b) { return __builtin_amdgcn_permlane16_swap(a, b, false, false); };
  float x[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) x[a] = swap_max(mm(a), mm(a + 4), sw32);
  t0 = swap_max(x[0], x[2], sw16);
  t1 = swap_max(x[1], x[3], sw16);
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  return __builtin_bit_cast(double, dpp_u64<CTRL>(__builtin_bit_cast(uint64_t, v)));
}

// emit(b, f32(pairwise_f64(max[b,q] * sigma[b,q]) * scale)) for b < batch.
// rows = batch * query_tokens <= 128, so query_tokens < 8 means batch <= 128
// (lanes b and b + 64) and query_tokens >= 8 means batch <= 16 (two rounds of
// eight lanes per batch row).  Each path emits at most twice per lane.
template <class Emit>
static __device__ __forceinline__ void scan_finish_doc(const float* rowmax, const float* qs, int batch,
                                                       int query_tokens, double scale, Emit emit) {
  const int lane = lane_id();
  auto prod = [&](int r) -> double { return (double)rowmax[r] * (double)qs[r]; };
  if (query_tokens < 8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int b = lane + kWave * h;
      double res = 0.0;
      if (b < batch) {
        for (int q = 0; q < query_tokens; ++q) res = __dadd_rn(res, prod(b * query_tokens + q));
        emit(b, (float)(res * scale));
      }
    }
    return;
  }
  const int body = query_tokens - (query_tokens % 8);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (8 * h >= batch) break;
    const int b = 8 * h + (lane >> 3), k = lane & 7;
    const bool valid = b < batch;
    const int base = valid ? b * query_tokens : 0;
    double r = prod(base + k);
    for (int i = 8 + k; i < body; i += 8) r = __dadd_rn(r, prod(base + i));
    double o = __shfl_xor(r, 1);
    if ((k & 1) == 0) r = __dadd_rn(r, o);
    o = __shfl_xor(r, 2);
    if ((k & 3) == 0) r = __dadd_rn(r, o);
    o = __shfl_xor(r, 4);
    if (k == 0) r = __dadd_rn(r, o);
    if (k == 0 && valid) {
      for (int i = body; i < query_tokens; ++i) r = __dadd_rn(r, prod(base + i));
      emit(b, (float)(r * scale));
    }
  }
}

// Two waves per SIMD (eight per CU): at most 256 VGPRs per wave.
#define MSIM_SCAN_OCCUPANCY __attribute__((amdgpu_waves_per_eu(2, 2)))

// Epilogue constants of one tile: per accumulator row r (the lane's token
// 4g + r) the factor a[r] and, for kScanEpiFma, the addend c[r].
struct TileEpi {
  float a[4], c[4];
};

// A dispatch's identity, as the fused selection's give-up mark stores it:
// its packet index in its queue (the dispatch id, + 1 so that a zeroed mark
// names no dispatch) and the queue's address.
struct LaunchMark {
  uint32_t w[4];
};
// The dispatch id has no clang builtin: the LLVM intrinsic by name.
extern "C" __device__ uint64_t msim_dispatch_id() __asm("llvm.amdgcn.dispatch.id");
__device__ __forceinline__ LaunchMark launch_mark() {
  const uint64_t d = msim_dispatch_id() + 1u;
  const uint64_t q = reinterpret_cast<uint64_t>(__builtin_amdgcn_queue_ptr());
  return {{(uint32_t)d, (uint32_t)(d >> 32), (uint32_t)q, (uint32_t)(q >> 32)}};
}

// Bits of 2^23 as an int32: the C operand of a kScanEpiFma tile's first MFMAs.
constexpr int kMagic = 0x4B000000;
constexpr int kMaskedAcc = -(1 << 30);  // C operand of masked rows (|16 * dot| < 2^21)

template <int NT, int EPI, bool kTail, bool kSign = false>
__global__ __launch_bounds__(kScanThreads) MSIM_SCAN_OCCUPANCY void int8q_scan_kernel(
    ScanArgs p, const uint8_t* __restrict__ codes, const float* __restrict__ token_scale16,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ wave_info_ptr,
    const uint64_t* __restrict__ tile_table, const int8_t* __restrict__ qpack,
    const float* __restrict__ qscale, float* __restrict__ scores) {
  constexpr bool kTS = EPI != kScanEpiIntMax;
  // LDS: the workgroup's copy of the query tiles; per wave the tile ring
  // (codes as 64 lanes x 16 B, token scales as 64 lanes x 4 B per slot), the
  // per-row maxima of the document being finished and the query scales.
  constexpr int kQueryParts = (NT + 1) / 2;  // 1 KiB half-tiles per wave
  __shared__ __attribute__((aligned(16))) v4u s_query[kQueryParts * kScanWaves * kWave];
  __shared__ __attribute__((aligned(16))) v4u s_codes[kScanWaves][kPrefetch][kWave];
  __shared__ __attribute__((aligned(16))) uint32_t s_scales[kScanWaves][kPrefetch][kWave];
  __shared__ float s_rowmax[kScanWaves][128];
  __shared__ float s_qscale[kScanWaves][128];
  const int lane = lane_id();
  const int wave = wave_uniform(threadIdx.x / kWave);
  const int g = lane >> 4, c = lane & 15;
  // The host pads the wave table to whole workgroups (padding waves have no
  // tiles), so every wave reaches the barrier below.
  const int64_t gw = (int64_t)blockIdx.x * kScanWaves + wave;

  const auto info = as_constant(wave_info_ptr) + gw * kWaveInfoWords;
  const int64_t d0 = info[0];
  const int64_t T0 = info[2], T1 = info[3];
  const int ntiles = (int)info[4];
  const auto tt = as_constant(tile_table) + gw * p.tile_stride;  // no wait on `info`
  const int nempty = (int)info[6];
  const int64_t e0 = info[7];
  constexpr bool fused = kTail;  // p.topk_k > 0 exactly when kTail
  float* rowmax = s_rowmax[wave];
  float* qs = s_qscale[wave];
  // Fused selection: documents take positions pos0, pos0 + 1, ... (the
  // wave's empty documents, then the others in tile order); per batch row
  // the three largest full keys of the wave's documents (0: none).
  __shared__ uint64_t s_top[kScanWaves][kScanTailMaxRows][3];
  const int pos0 = (int)info[5];
  int nfin = 0;
  uint32_t tag = 0;  // the launch's tag (fused), read below
  if (fused && lane < kScanTailMaxRows * 3) (&s_top[wave][0][0])[lane] = 0ull;
  // Score v of document doc for batch row b, at position pos; `rank` also
  // enters it in the wave's top three of row b (one lane per row at a time).
  auto emit = [&](int b, int64_t doc, int pos, float v, bool rank = true) {
    if constexpr (fused) {
      const uint64_t key = tail_full_key(v, (uint32_t)doc, tag);
      __hip_atomic_store(p.tail_keys + (int64_t)b * kScanTailRow + pos, key, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (rank) {
        uint64_t* t3 = s_top[wave][b];
        const uint64_t a0 = t3[0], a1 = t3[1], a2 = t3[2];
        t3[0] = max(a0, key);
        t3[1] = max(a1, min(a0, key));
        t3[2] = max(a2, min(a1, key));
      }
    } else {
      scores[(int64_t)b * p.score_stride + doc] = v;
    }
  };

  // Global loads, all with an LDS destination (untracked by the compiler,
  // waited for explicitly), in this order: the workgroup's query tiles (each
  // wave a quarter of the 1 KiB half-tiles, lane order), this wave's query
  // scales, the wave's first kStartTiles tiles.
  {
    const v4i rqp = make_rsrc_words(qpack, (uint32_t)(NT * 2048));
    const uint32_t q_lds = wave_uniform((int)lds_address(s_query));
#pragma unroll
    for (int i = 0; i < kQueryParts; ++i) {
      const uint32_t half = (uint32_t)(i * kScanWaves + wave), part = half * kWave;
      // Lane order: the half-tile is one linear 1 KiB run.  Row order (128
      // bytes per row): lane (g, c) takes row 16 (half / 2) + c, bytes
      // 32g + 16 (half % 2) .. + 16.
      const uint32_t src = p.q_row_order ? ((16u * (half >> 1) + (uint32_t)c) * 128u + 32u * (uint32_t)g + 16u * (half & 1u))
                                         : (part + (uint32_t)lane) * 16u;
      lds_load_b128(rqp, src, (uint32_t)wave_uniform((int)(q_lds + part * 16u)));
    }
    const v4i rq = make_rsrc_words(qscale, (uint32_t)(16 * NT * 4));
    const uint32_t qs_lds = wave_uniform((int)lds_address(qs));
    lds_load_b32(rq, 4u * (uint32_t)lane, qs_lds);
    lds_load_b32(rq, 4u * (uint32_t)(lane + kWave), qs_lds + 4 * kWave);
    // Fused: the launch counter and the give-up mark (words 0 .. 5 of
    // epoch) into words 0 .. 5 of the row-maxima buffer; the other lanes
    // read past the 24-byte range: 0.  One load instruction over one cache
    // line: the words come from one snapshot of the line.
    if (fused) lds_load_b32(make_rsrc_words(p.epoch, 24u), 4u * (uint32_t)lane, wave_uniform((int)lds_address(rowmax)));
    // Sign documents: the query rows' code sums into the row-maxima buffer.
    if (kSign) {
      const v4i rsum = make_rsrc_words(p.qsum, (uint32_t)(16 * NT * 4));
      const uint32_t rm_lds = wave_uniform((int)lds_address(rowmax));
      lds_load_b32(rsum, 4u * (uint32_t)lane, rm_lds);
      lds_load_b32(rsum, 4u * (uint32_t)(lane + kWave), rm_lds + 4 * kWave);
    }
  }

  // Descriptors over the wave's tokens and the kScanPadTokens zero rows that
  // follow the corpus (tile starts are wave-relative and below T1 - T0, so
  // every tile's 16 rows lie in that range).
  constexpr int kTokenBytes = kSign ? 16 : 64;
  const v4i rc = make_rsrc_words(codes + T0 * kTokenBytes, (uint32_t)((T1 - T0 + kScanPadTokens) * kTokenBytes));
  const v4i rs = make_rsrc_words(kTS ? (const void*)(token_scale16 + T0) : (const void*)codes,
                                 kTS ? (uint32_t)((T1 - T0 + kScanPadTokens) * 4) : 0u);
  const uint32_t ring_codes = wave_uniform((int)lds_address(&s_codes[wave][0][0]));
  const uint32_t ring_scales = wave_uniform((int)lds_address(&s_scales[wave][0][0]));

  // Tile i of the wave starts at token tt[i] (low 32 bits, relative to T0):
  // documents of len >= 16 are covered by tiles at s, s + 16, ..., with the
  // last one at e - 16.  Lane (g, c) fetches the 16 code bytes of token
  // t + c for dims [32g, 32g + 32) and the (pre-divided by 16) scale of
  // token t + c; a lane then reads the four scales of its accumulator rows
  // 4g..4g+3 as one 16-byte LDS read.  The tile's byte offset is the loads'
  // scalar offset, the lane's part a constant VGPR.  Tile x goes to ring
  // slot x % kPrefetch.  The wave starts with kStartTiles tiles in flight
  // and fills the ring over its first kRampStages steps, three tiles each
  // (every wave asking for its whole ring at the start takes about 1.8 us
  // to issue, the first tile then lands 0.4 us later); from then on every
  // step issues exactly kOps loads, so the tile read next is complete once
  // vmcnt <= (kPrefetch - 1) * kOps.
  constexpr int kOps = kTS ? 2 : 1;
  constexpr int kRingWait = (kPrefetch - 1) * kOps;
  constexpr int kStartTiles = 2, kRampStages = 3;
  static_assert(kStartTiles + 2 * kRampStages == kPrefetch, "after the ramp the ring runs kPrefetch tiles ahead");
  const uint32_t voff_codes = kSign ? 16u * (uint32_t)c + 4u * (uint32_t)g : 64u * (uint32_t)c + 16u * (uint32_t)g;
  const uint32_t voff_scales = 4u * (uint32_t)c;
  auto load_tile = [&](int slot_, uint32_t t) {
    const uint32_t tu = (uint32_t)wave_uniform((int)t);
    if (kSign) lds_load_b32_so(rc, voff_codes, tu * 16u, ring_codes + slot_ * kWave * 16);
    else lds_load_b128_so(rc, voff_codes, tu * 64u, ring_codes + slot_ * kWave * 16);
    if (kTS) lds_load_b32_so(rs, voff_scales, tu * 4u, ring_scales + slot_ * kWave * 4);
  };
#pragma unroll
  for (int s = 0; s < kStartTiles; ++s) load_tile(s, (uint32_t)tt[s]);
  // First tokens of the ramp's tiles kStartTiles .. kStartTiles + 3
  // kRampStages - 1 (the table has at least kScanMinStride entries per wave).
  static_assert(kStartTiles + 3 * kRampStages <= kScanMinStride, "ramp entries inside the wave's table row");
  uint32_t ramp_tok[3 * kRampStages];
#pragma unroll
  for (int x = 0; x < 3 * kRampStages; ++x) ramp_tok[x] = (uint32_t)tt[kStartTiles + x];

  // The query tiles (and scales) are complete once at most kStartTiles *
  // kOps loads are outstanding; the barrier publishes all four quarters.
  vm_wait_lds<kStartTiles * kOps>();
  __builtin_amdgcn_s_barrier();
  if (fused) {
    // The launch's tag is the counter + 1, unless the give-up mark names this
    // dispatch: then this workgroup started after its own launch's selection
    // gave up and published the counter, and it keeps that launch's tag (its
    // entries must not carry the next launch's tag).
    const LaunchMark m = launch_mark();
    bool late = true;
#pragma unroll
    for (int i = 0; i < 4; ++i) late = late && __float_as_uint(rowmax[2 + i]) == m.w[i];
    tag = (uint32_t)wave_uniform((int)(__float_as_uint(rowmax[0]) + (late ? 0u : 1u)));
  }
  // Sign documents (A bytes 0 / 2 from the sign bits): the first MFMA of
  // query tile j starts at 2^23 - sum(q8) in column c, so the accumulator
  // holds 2^23 + (2 (q8 . bits) - sum(q8)) = 2^23 + q8 . signs.
  v4i csign[kSign ? NT : 1];
  if (kSign) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int cj = kMagic - __float_as_int(rowmax[16 * j + c]);
      csign[j] = (v4i){cj, cj, cj, cj};
    }
  }
  // Query tiles: lane (g, c) holds row 16j + c, dims of lane group g; half j
  // of tile h is the linear 1 KiB run 2j + h (no bank conflicts).
  v4i blo[NT], bhi[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    blo[j] = reinterpret_cast<const v4i*>(s_query)[(2 * j) * kWave + lane];
    bhi[j] = reinterpret_cast<const v4i*>(s_query)[(2 * j + 1) * kWave + lane];
  }

  // Running maxima per query tile: float for the scaled forms, the integer
  // 16 * dot for tensor-scale corpora.
  float m[NT];
  int mi[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    m[j] = kNegInf;
    mi[j] = INT32_MIN;
  }
  constexpr float kInf = __builtin_huge_valf();

  // Epilogue constants and C operand of a tile from its table entry (rows in
  // bits 32..36 as rows - 1) and its four token scales.  Rows past a short
  // document are masked: -inf for the scaled forms (c = -inf, or a = +inf on
  // an accumulator starting at -2^30), a -2^30 start for the integer form.
  // The kScanEpiFma C operand, kept in registers for the whole loop (an
  // opaque copy: rebuilding it from a constant would take two moves per tile).
  v4i cmagic = (v4i){kMagic, kMagic, kMagic, kMagic};
  if (EPI == kScanEpiFma) asm volatile("" : "+v"(cmagic));
  auto prep = [&](uint32_t mhi, const v4u& sv, TileEpi& e) -> v4i {
    const uint32_t rows = (mhi & 31u) + 1u;
    v4i cinit = EPI == kScanEpiFma ? cmagic : (v4i){0, 0, 0, 0};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      e.a[r] = kTS ? __uint_as_float(sv[r]) : 1.0f;
      e.c[r] = e.a[r] * -8388608.0f;  // -2^23 a, exact
    }
    if (rows < 16u) {
      const uint32_t r0 = 4u * (uint32_t)g;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool masked = r0 + (uint32_t)r >= rows;
        if (EPI == kScanEpiFma) {
          e.c[r] = masked ? kNegInf : e.c[r];
        } else {
          cinit[r] = masked ? kMaskedAcc : 0;
          if (EPI == kScanEpiCvt) e.a[r] = masked ? kInf : e.a[r];
        }
      }
    }
    return cinit;
  };
  // Half h of the running max over a finished tile's accumulators for query
  // tile j (accumulator rows 2h, 2h + 1).
  //  * kScanEpiFma: acc holds the bits of 2^23 + n (n = 16 dot >= 0) or of
  //    2^23 + n / 2 (n < 0: the binade below 2^23 has half the spacing), so
  //    fma(F, s/16, -2^23 s/16) is one rounding of dot * s, or of dot * s / 2
  //    for negative dots; x -> (x >= 0 ? x : x / 2) is increasing, so the
  //    maximum maps back by min(M, 2M) at the document end.
  //  * kScanEpiCvt: float(acc >> 4) * s (acc = 16 dot exactly; the token
  //    scales themselves, so one rounding of dot * s for any positive s).
  //  * kScanEpiIntMax: the integer maximum of 16 dot.
  auto epilogue_half = [&](const v4i& acc, const TileEpi& e, int j, int h) {
    const int r0 = 2 * h, r1 = 2 * h + 1;
    if constexpr (EPI == kScanEpiIntMax) {
      mi[j] = max(max(mi[j], acc[r0]), acc[r1]);
    } else if constexpr (EPI == kScanEpiFma) {
      const float x0 = __builtin_fmaf(__int_as_float(acc[r0]), e.a[r0], e.c[r0]);
      const float x1 = __builtin_fmaf(__int_as_float(acc[r1]), e.a[r1], e.c[r1]);
      m[j] = max3_op(m[j], x0, x1);
    } else {
      const float x0 = (float)(acc[r0] >> 4) * e.a[r0];
      const float x1 = (float)(acc[r1] >> 4) * e.a[r1];
      m[j] = max3_op(m[j], x0, x1);
    }
  };
  // The MFMAs of the next tile (all first halves, then all second halves, so
  // consecutive MFMAs are independent) interleaved with the epilogue of the
  // previous one, in a fixed order: each MFMA (16 cycles in the matrix core)
  // is followed by the VALU instructions of one epilogue half, which read
  // results of the other accumulator set (no MFMA-to-VALU wait).  The second
  // halves' operand is unpacked beside the first four groups.
  auto issue_and_finish = [&](v4i (&acc_q)[NT], const v4u& w_q, const v4i& cinit, const v4i (&acc_p)[NT],
                              const TileEpi& e_p, bool with_epilogue) {
    // int4: sixteen times the even / odd dims' values.  Sign documents (32
    // bits, bit 8y + i = dim 32g + 8y + i): byte y of operand dword i is 2 x
    // bit 8y + i (lo, i < 4) or bit 8y + i + 4 (hi).
    auto unpack_lo = [&](int x) -> int {
      if (kSign) return (int)((x == 0 ? (w_q[0] << 1) : (w_q[0] >> (x - 1))) & 0x02020202u);
      return (int)((w_q[x] << 4) & 0xF0F0F0F0u);
    };
    auto unpack_hi = [&](int x) -> int {
      if (kSign) return (int)((w_q[0] >> (x + 3)) & 0x02020202u);
      return (int)(w_q[x] & 0xF0F0F0F0u);
    };
    v4i lo, hi;
#pragma unroll
    for (int x = 0; x < 4; ++x) lo[x] = unpack_lo(x);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      acc_q[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(lo, blo[j], kSign ? csign[kSign ? j : 0] : cinit, 0, 0, 0);
      if (with_epilogue) epilogue_half(acc_p[j], e_p, j, 0);
      if (j < 4) hi[j] = unpack_hi(j);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int x = NT; x < 4; ++x) hi[x] = unpack_hi(x);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      acc_q[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(hi, bhi[j], acc_q[j], 0, 0, 0);
      if (with_epilogue) epilogue_half(acc_p[j], e_p, j, 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto epilogue = [&](const v4i (&acc)[NT], const TileEpi& e) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      epilogue_half(acc[j], e, j, 0);
      epilogue_half(acc[j], e, j, 1);
    }
  };

  // 32-token queries: batch row g is summed by lane group g in registers
  // (tokens c and 16 + c in lane c); its query scales are read once here.
  const bool q32 = NT % 2 == 0 && p.query_tokens == 32;
  float sig0 = 0.0f, sig1 = 0.0f;
  if (q32) {
    sig0 = qs[32 * g + c];
    sig1 = qs[32 * g + 16 + c];
  }

  // Document end: per-row maxima over the four lane groups, then the score of
  // local document `local`.
  auto finish = [&](int local) {
    float mf[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) mf[j] = EPI == kScanEpiIntMax ? (float)mi[j] * 0.0625f : m[j];
    auto unfold = [](float v) { return EPI == kScanEpiFma ? fminf(v, v + v) : v; };
    if (q32) {
      // numpy's pairwise float64 sum of 32 terms: accumulator k < 8 adds
      // tokens k, k + 8, k + 16, k + 24 in that order (lane k; row_ror:8
      // brings lane k + 8's products), then ((r0 + r1) + (r2 + r3)) +
      // ((r4 + r5) + (r6 + r7)) by lane swaps within quads (every lane of
      // quad 0 then holds the first half, every lane of quad 1 the second)
      // and a half-row mirror (lane 0 reads lane 7).
      float t0, t1;
      max_scatter_groups<NT>(mf, t0, t1);
      t0 = unfold(t0);
      t1 = unfold(t1);
      const double p0 = (double)t0 * (double)sig0, p1 = (double)t1 * (double)sig1;
      double r = __dadd_rn(p0, dpp_f64<0x128>(p0));
      r = __dadd_rn(r, p1);
      r = __dadd_rn(r, dpp_f64<0x128>(p1));
      r = __dadd_rn(r, dpp_f64<0xB1>(r));   // quad_perm [1,0,3,2]
      r = __dadd_rn(r, dpp_f64<0x4E>(r));   // quad_perm [2,3,0,1]
      r = __dadd_rn(r, dpp_f64<0x141>(r));  // row_half_mirror
      if (c == 0 && g < p.batch) emit(g, d0 + local, pos0 + nempty + nfin, (float)(r * p.scale));
    } else {
#pragma unroll
      for (int j = 0; j < NT; ++j) mf[j] = unfold(max_over_groups(mf[j]));
      if (g == 0) {
#pragma unroll
        for (int j = 0; j < NT; ++j) rowmax[16 * j + c] = mf[j];
      }
      wave_sync_lds();
      scan_finish_doc(rowmax, qs, p.batch, p.query_tokens, p.scale,
                      [&](int b, float v) { emit(b, d0 + local, pos0 + nempty + nfin, v); });
      wave_sync_lds();
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      m[j] = kNegInf;
      mi[j] = INT32_MIN;
    }
    ++nfin;
  };

  // Software pipeline over the wave's tiles.  Step i: the MFMAs of tile
  // i + 1 (raw codes in `w`, scales in `sv`, entry `meta`) go to one
  // accumulator set while the epilogue of tile i reads the other (its
  // results are complete: no MFMA-to-VALU wait); the ring slot of tile i + 1
  // is refilled (tile i + 1 + kPrefetch, starting at token `iss`) and tile
  // i + 2 is read back from the ring.  Table entries are scalar loads one
  // step ahead.
  if (ntiles > 0) {
    v4i acc_a[NT], acc_b[NT];
    TileEpi epi_p;       // epilogue constants of the tile whose results are pending
    uint32_t mhi_p;      // and its table entry (high half)
    uint64_t meta = tt[0], iss = tt[kPrefetch];
    int slot = 0;
    vm_wait_lds<(kStartTiles - 1) * kOps>();
    auto read_codes = [&](int sl) -> v4u {
      if (kSign) return (v4u){reinterpret_cast<const uint32_t*>(&s_codes[wave][sl][0])[lane], 0u, 0u, 0u};
      return s_codes[wave][sl][lane];
    };
    v4u w = read_codes(0);
    v4u sv = kTS ? *reinterpret_cast<const v4u*>(&s_scales[wave][0][0] + 4 * g) : (v4u){0u, 0u, 0u, 0u};
    // Read-ahead after tile `slot` left the ring for registers.  Stage K
    // (1..kRampStages, the advances to tiles 1..kRampStages) issues tiles
    // 3K - 1 .. 3K + 1 into their slots, none of them holding a tile still
    // to be read, and then 2K + 1 tiles past tile K are in flight; stage 0
    // refills the slot just left with tile i_next - 1 + kPrefetch.
    auto advance = [&](int i_next, auto stage) {
      constexpr int K = decltype(stage)::value;
      lds_read_done(w, sv);
      if constexpr (K == 0) {
        load_tile(slot, (uint32_t)iss);
      } else {
#pragma unroll
        for (int x = 3 * K - 1; x <= 3 * K + 1; ++x) load_tile(x % kPrefetch, ramp_tok[x - kStartTiles]);
      }
      const uint64_t meta_n = tt[i_next], iss_n = tt[i_next + kPrefetch];
      slot = slot + 1 == kPrefetch ? 0 : slot + 1;
      if constexpr (K == 0) vm_wait_lds<kRingWait>();
      else vm_wait_lds<(2 * K + 1) * kOps>();
      w = read_codes(slot);
      if (kTS) sv = *reinterpret_cast<const v4u*>(&s_scales[wave][slot][0] + 4 * g);
      meta = meta_n;
      iss = iss_n;
    };
    // Prologue: tile 0's MFMAs.
    {
      mhi_p = (uint32_t)(meta >> 32);
      const v4i cinit = prep(mhi_p, sv, epi_p);
      const v4u w_q = w;
      advance(1, std::integral_constant<int, 1>{});
      issue_and_finish(acc_a, w_q, cinit, acc_b, epi_p, false);
    }
    auto step = [&](int i, v4i (&acc_p)[NT], v4i (&acc_q)[NT], auto stage) {
      const uint32_t mhi_q = (uint32_t)(meta >> 32);
      TileEpi epi_q;
      const v4i cinit = prep(mhi_q, sv, epi_q);
      const v4u w_q = w;
      advance(i + 2, stage);
      issue_and_finish(acc_q, w_q, cinit, acc_p, epi_p, true);
      if ((mhi_p >> 5) & 1u) finish((int)(mhi_p >> 8));
      mhi_p = mhi_q;
      epi_p = epi_q;
    };
    auto last = [&](const v4i (&acc_p)[NT]) {
      mfma_results_fence();  // the last tile's MFMAs were issued just before
      epilogue(acc_p, epi_p);
      finish((int)(mhi_p >> 8));  // the last tile always ends a document
    };
    using Ramp2 = std::integral_constant<int, 2>;
    using Ramp3 = std::integral_constant<int, 3>;
    using Steady = std::integral_constant<int, 0>;
    static_assert(kRampStages == 3, "two ramp stages after the prologue's");
    int i = 0;
    if (ntiles > 2) {
      step(0, acc_a, acc_b, Ramp2{});
      step(1, acc_b, acc_a, Ramp3{});
      i = 2;
    }
    for (; i + 2 < ntiles; i += 2) {
      step(i, acc_a, acc_b, Steady{});
      step(i + 1, acc_b, acc_a, Steady{});
    }
    if (i + 1 < ntiles) {
      if (i == 0) step(0, acc_a, acc_b, Ramp2{});  // two tiles: the ramp's second stage reads tile 2
      else step(i, acc_a, acc_b, Steady{});
      last(acc_b);
    } else {
      last(acc_a);
    }
  }
  // No LDS-destination load may still be in flight when the wave ends (a
  // fused launch waits later: that wait also covers its key stores).
  if (!fused) vm_wait_lds<0>();

  // Empty documents score 0 (the wave's entries of the empty-document list).
  // Fused: they all score 0, so the wave's three lowest ids (its first
  // entries) are the only ones that can enter its top three.
  for (int e = lane; e < nempty; e += kWave) {
    const int64_t doc = wave_info_ptr[p.num_waves * kWaveInfoWords + e0 + e];
    for (int b = 0; b < p.batch; ++b) emit(b, doc, pos0 + e, 0.0f, false);
  }
  if (fused && lane == 0) {
    for (int e = 0; e < min(nempty, 3); ++e) {
      const int64_t doc = wave_info_ptr[p.num_waves * kWaveInfoWords + e0 + e];
      for (int b = 0; b < p.batch; ++b) emit(b, doc, pos0 + e, 0.0f);
    }
  }
  if constexpr (!fused) return;

  // Fused selection.  The workgroup's record per batch row (one thread per
  // row, after an LDS-only barrier: the key stores stay in flight): its two
  // largest full keys and the third one's score key, each word tagged.
  // Every workgroup but 0 is then done; workgroup 0 selects (each of its
  // waves once its own tile ring has drained).
  int bs[kTailBlocksPerLane], blen[kTailBlocksPerLane];
  if (blockIdx.x == 0) tail_block_ranges(p.block_pos, (int)gridDim.x, bs, blen);
  group_sync_lds();
  if ((int)threadIdx.x < p.batch) {
    // The waves' sorted top threes merged as a tree: the i-th largest of two
    // sorted lists x, y is the maximum over j of min(x[j - 1], y[i - j - 1])
    // (x[-1] = y[-1] = +inf), so the top three of x and y are
    // max(x0, y0), max(x1, y1, min(x0, y0)), max(x2, y2, min(x1, y0), min(x0, y1)).
    struct Top3 {
      uint64_t k0, k1, k2;
    };
    auto merge3 = [](const Top3& x, const Top3& y) {
      Top3 z;
      z.k0 = max(x.k0, y.k0);
      z.k1 = max(max(x.k1, y.k1), min(x.k0, y.k0));
      z.k2 = max(max(x.k2, y.k2), max(min(x.k1, y.k0), min(x.k0, y.k1)));
      return z;
    };
    static_assert(kScanWaves == 4, "two merge levels");
    Top3 t[kScanWaves];
#pragma unroll
    for (int w = 0; w < kScanWaves; ++w)
      t[w] = {s_top[w][threadIdx.x][0], s_top[w][threadIdx.x][1], s_top[w][threadIdx.x][2]};
    const Top3 all = merge3(merge3(t[0], t[1]), merge3(t[2], t[3]));
    const uint64_t a0 = all.k0, a1 = all.k1, a2 = all.k2;
    const uint64_t ktag = tail_key_tag(tag);
    uint64_t* rec = p.tail_rec + (int64_t)threadIdx.x * 3 * kScanTailBlocks + blockIdx.x;
    __hip_atomic_store(rec, a0 != 0 ? a0 : ktag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(rec + kScanTailBlocks, a1 != 0 ? a1 : ktag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(rec + 2 * kScanTailBlocks, ((a2 >> 32) << 32) | tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  vm_wait_lds<0>();
  if (blockIdx.x != 0) return;
  // Wave w selects batch rows w, w + 4, ... in its tile ring's LDS.
  uint64_t* lds = reinterpret_cast<uint64_t*>(&s_codes[wave][0][0]);
  bool row0_selected = true;
  for (int b = wave; b < p.batch; b += kScanWaves) {
    const bool selected =
        tail_topk(p.tail_keys + (int64_t)b * kScanTailRow, p.tail_rec + (int64_t)b * 3 * kScanTailBlocks,
                  (int)gridDim.x, (int)p.num_docs, p.topk_k, p.tail_cap, tag, lds, bs, blen,
                  p.top_scores + (int64_t)b * p.topk_k, p.top_ids + (int64_t)b * p.topk_k, p.tail_wait_ticks,
                  p.epoch + 1);
    if (b == 0) row0_selected = selected;
  }
  if (threadIdx.x == 0) {
    if (row0_selected) {
      // Every workgroup wrote its row-0 record, so every one read the
      // counter at its start: the next launch's tag can be published.
      __hip_atomic_store(p.epoch, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      // Workgroups of this launch may not have started yet: the mark names
      // this dispatch, then (release) the counter.  A workgroup that reads
      // both keeps this launch's tag.
      const LaunchMark m = launch_mark();
#pragma unroll
      for (int i = 0; i < 4; ++i) __hip_atomic_store(p.epoch + 2 + i, m.w[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.epoch, tag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // Key tags repeat every kTailTagMask launches, so launches whose key tags
  // collide are a multiple of it apart, and a launch whose tag is
  // kTailTagMask - 1 modulo it lies between them: that launch zeroes every
  // key row once the selection's waves are done with them.
  if (tag % kTailTagMask == kTailTagMask - 1u) {
    __syncthreads();
    for (int64_t w = threadIdx.x; w < p.tail_key_words; w += kScanThreads)
      __hip_atomic_store(p.tail_keys + w, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int EPI, bool kTail, bool kSign>
static void launch_scan_nt(const ScanArgs& a, int nt, int64_t blocks, hipStream_t stream) {
  const dim3 grid((unsigned)blocks), block(kScanThreads);
  switch (nt) {
#define MSIM_SCAN_CASE(N)                                                                                   \
  int8q_scan_kernel<N, EPI, kTail, kSign><<<grid, block, 0, stream>>>(a, a.codes, a.token_scale16, a.offsets, \
                                                                      a.wave_info, a.tile_table, a.qpack,     \
                                                                      a.qscale, a.scores)
    case 1: MSIM_SCAN_CASE(1); break;
    case 2: MSIM_SCAN_CASE(2); break;
    case 3: MSIM_SCAN_CASE(3); break;
    case 4: MSIM_SCAN_CASE(4); break;
    case 5: MSIM_SCAN_CASE(5); break;
    case 6: MSIM_SCAN_CASE(6); break;
    case 7: MSIM_SCAN_CASE(7); break;
    default: MSIM_SCAN_CASE(8); break;
#undef MSIM_SCAN_CASE
  }
}

template <int EPI>
static void launch_scan_epi(const ScanArgs& a, int nt, int64_t blocks, bool tail, hipStream_t stream) {
  if (tail) launch_scan_nt<EPI, true, false>(a, nt, blocks, stream);
  else launch_scan_nt<EPI, false, false>(a, nt, blocks, stream);
}

hipError_t launch_int8q_scan(const ScanArgs& args, int epilogue, hipStream_t stream) {
  const int rows = args.batch * args.query_tokens;
  if (rows <= 0 || rows > 128 || args.num_waves <= 0 || args.num_waves % kScanWaves != 0)
    return hipErrorInvalidValue;
  if (epilogue != kScanEpiIntMax && epilogue != kScanEpiFma && epilogue != kScanEpiCvt) return hipErrorInvalidValue;
  if ((epilogue == kScanEpiIntMax) != (args.token_scale16 == nullptr)) return hipErrorInvalidValue;
  // Sign documents: the one-fma epilogue over the per-token scales, no fused
  // selection, the query code sums given.
  if (args.doc_sign && (epilogue != kScanEpiFma || args.topk_k > 0 || args.qsum == nullptr)) return hipErrorInvalidValue;
  if (args.topk_k > 0 &&
      (args.topk_k > kScanTailMaxK || args.topk_k > args.num_docs || args.num_docs > kScanTailMaxDocs ||
       args.num_docs < kScanTailMinDocs || args.batch > kScanTailMaxRows ||
       args.num_waves > (int64_t)kScanWaves * kScanTailBlocks || args.epoch == nullptr ||
       args.top_scores == nullptr || args.top_ids == nullptr || args.tail_keys == nullptr ||
       args.tail_rec == nullptr || args.block_pos == nullptr ||
       args.tail_key_words < (int64_t)args.batch * kScanTailRow))
    return hipErrorInvalidValue;
  const int nt = (rows + 15) / 16;
  const int64_t blocks = args.num_waves / kScanWaves;
  const bool tail = args.topk_k > 0;
  if (args.doc_sign) {
    launch_scan_nt<kScanEpiFma, false, true>(args, nt, blocks, stream);
    return hipGetLastError();
  }
  switch (epilogue) {
    case kScanEpiIntMax: launch_scan_epi<kScanEpiIntMax>(args, nt, blocks, tail, stream); break;
    case kScanEpiFma: launch_scan_epi<kScanEpiFma>(args, nt, blocks, tail, stream); break;
    default: launch_scan_epi<kScanEpiCvt>(args, nt, blocks, tail, stream); break;
  }
  return hipGetLastError();
}

}  // namespace msim
