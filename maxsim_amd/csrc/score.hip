// score.hip -- generalized MaxSim scoring on gfx950 MFMA: int4 or sign-bit
// documents (optionally with an int4 residual stream), fp32 or int8 queries,
// the reference's five reducers, full-corpus or candidate targets.
//
// Semantics restated from the reference:
//  * reducers: MaxSim / weighted MaxSim / TopK2 / TopK4 / SmoothSim policies
//    cu:477-653, CPU closed form _api.py:558-585; an empty document scores 0;
//    the document scale is applied after the reduction except for SmoothSim,
//    whose similarities are scaled first (cu:602-605);
//  * int4 similarity s_t * scale * (q . v_t) (cu:1268-1323, K6 with the int4
//    loader); residual fused similarity p s^p_t (q . v^p_t) + r s^r_t
//    (q . v^r_t) reduced once (cu:967-1266, cascade.py:272-291);
//  * sign documents: q . sign(d_t) times the token scale (cu:297-352), the
//    int8-query form 2 (q8 . bits) - sum(q8) (cu:1368-1447).
//
// Design (MI355X): the dot products run on v_mfma_i32_16x16x64_i8.  An fp32
// query row q is split into three int8 limbs on a common grid,
//   q ~= sigma (a + b / 254 + c / 254^2),  sigma = max|q| / 127,
// |a|, |b|, |c| <= 127, so q . v = sigma (A + B / 254 + C / 254^2) with exact
// int32 limb dots A, B, C; the limb grid resolves q to 2^-24 of max|q|, as
// fine as fp32 itself.  Three int8 MFMA passes cost less than one fp32 VALU
// pass (int8 MFMA 5 POPS vs 157 TFLOP/s fp32).  An int8 query uses one limb.
//
// Work split: a wave owns a range of targets (documents, or candidate
// positions) and walks their 16-token tiles from a table (or, in direct
// mode, one candidate per wave, the tiles of its document's token range); a
// tile is the MFMA A operand (16 tokens x 128 dims), the query rows of the pass
// are B operands held in registers.  Each lane keeps the reducer state of
// its query column over its four token rows; at a target's last tile the
// four lane groups are merged and the per-row pooled values are written to
// pooled[target][row]; pool_sum_kernel then sums over each batch row's query
// tokens.
#include "common.hpp"
#include "internal.hpp"

namespace msim {

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerGroup = kThreads / kWave;
constexpr float kLimbStep = 1.0f / 254.0f;
constexpr float kLimbStep2 = 1.0f / 64516.0f;  // 254^-2
// Limb accumulator starts of the biased three-limb form (score_kernel):
// limb 1 starts at -kLimb1Bias, limb 2 at the bits of kLimb1Bias * 254 =
// 12583160 = 2^23 + 4194552 (the float's bits 0x4B000000 + 4194552).
constexpr int kLimb1Bias = 49540;
constexpr int kLimb2Bias = 0x4B000000 + 4194552;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLowest = -3.402823466e+38f;

template <int RED>
struct ReducerState;

// kRedMax: running maximum.
template <>
struct ReducerState<kRedMax> {
  float m;
  __device__ void init() { m = kNegInf; }
  // Two three-way maxima (v_max3_f32) for four values: exact, any order.
  __device__ void add4(const float (&z)[4], float) { m = max3_op(max3_op(m, z[0], z[1]), z[2], z[3]); }
  __device__ void merge_xor(int mask, float) { m = fmaxf(m, __shfl_xor(m, mask)); }
  __device__ float finish(int len, float colmul, float, float weight, float doc_scale) const {
    return len == 0 ? 0.0f : m * colmul * weight * doc_scale;
  }
};

// kRedTop2 / kRedTop4: the K largest values, sorted descending.
template <int K>
struct TopState {
  float t[K];
  __device__ void init() {
#pragma unroll
    for (int i = 0; i < K; ++i) t[i] = kNegInf;
  }
  // With t sorted descending, the new i-th largest of t and v is the median
  // of t[i - 1], t[i] and v (the maximum for i = 0): one v_med3_f32 each,
  // all from the old values.  Only selections, so the result is exact.
  __device__ void insert(float v) {
    float n[K];
    n[0] = fmaxf(t[0], v);
#pragma unroll
    for (int i = 1; i < K; ++i) n[i] = __builtin_amdgcn_fmed3f(t[i - 1], t[i], v);
#pragma unroll
    for (int i = 0; i < K; ++i) t[i] = n[i];
  }
  __device__ void add4(const float (&z)[4], float) {
#pragma unroll
    for (int r = 0; r < 4; ++r) insert(z[r]);
  }
  __device__ void merge_xor(int mask, float) {
    float o[K];
#pragma unroll
    for (int i = 0; i < K; ++i) o[i] = __shfl_xor(t[i], mask);
#pragma unroll
    for (int i = 0; i < K; ++i) insert(o[i]);
  }
  __device__ float finish(int len, float colmul, float, float, float doc_scale) const {
    const int kept = len < K ? len : K;
    if (kept == 0) return 0.0f;
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < K; ++i)
      if (i < kept) total += t[i];
    return total / (float)kept * colmul * doc_scale;
  }
};
template <>
struct ReducerState<kRedTop2> : TopState<2> {};
template <>
struct ReducerState<kRedTop4> : TopState<4> {};

// kRedLse: online log-sum-exp in base 2 over u = z * k with k = colmul *
// doc_scale * log2(e) / tau, i.e. u = x log2(e) / tau for the scaled
// similarity x = z * colmul * doc_scale: m = running maximum of u (starts at
// the lowest finite float so that masked -inf values never form inf - inf),
// s = sum 2^(u - m).  Every exponent is <= 0 and the maximum's term is 1, so
// v_exp_f32 itself serves (exp2f adds a rescaling path for results below
// 2^-126, which are negligible next to that 1).  The score, max x + tau ln
// sum e^((x - max x) / tau), is then (m + log2 s) * tau * ln 2.  (Folding
// log2(e) / tau into k saves a multiply per similarity.)
__device__ __forceinline__ float exp2_nonpos(float x) { return __builtin_amdgcn_exp2f(x); }
template <>
struct ReducerState<kRedLse> {
  float m, s, k;  // k = colmul * doc_scale * log2(e) / tau for the current target
  __device__ void init() {
    m = kLowest;
    s = 0.0f;
  }
  __device__ void add4(const float (&z)[4], float) {
    float u[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) u[r] = z[r] * k;
    const float mn = max3_op(max3_op(m, u[0], u[1]), u[2], u[3]);
    float acc = s * exp2_nonpos(m - mn);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc += exp2_nonpos(u[r] - mn);
    s = acc;
    m = mn;
  }
  __device__ void merge_xor(int mask, float) {
    const float mo = __shfl_xor(m, mask), so = __shfl_xor(s, mask);
    const float mn = fmaxf(m, mo);
    s = s * exp2_nonpos(m - mn) + so * exp2_nonpos(mo - mn);
    m = mn;
  }
  __device__ float finish(int len, float, float temperature, float, float) const {
    return len == 0 ? 0.0f : (m + log2f(s)) * (temperature * kLn2);
  }
};

// One tile of a stream, as loaded: lane (g, c) holds token c's bytes of lane
// group g in each 128-dim chunk and the scales of token rows 4g .. 4g + 3.
template <int DOC, int KC>
struct TileCodes;
template <int KC>
struct TileCodes<kDocInt4, KC> {
  v4u w[KC];  // 16 bytes per chunk: dims 128 kc + 32g .. + 31 as nibbles
};
template <int KC>
struct TileCodes<kDocSign, KC> {
  unsigned w[KC];  // 32 sign bits per chunk: dims 128 kc + 32g .. + 31
};

// A operands (two MFMAs of 64 dims) from the tile bytes of one chunk.
__device__ __forceinline__ void unpack_a(const v4u& w, v4i& a0, v4i& a1) {
  // Nibbles moved to the high half of each byte: the int8 value is 16 v.
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    a0[x] = (int)((w[x] << 4) & 0xF0F0F0F0u);  // even dims
    a1[x] = (int)(w[x] & 0xF0F0F0F0u);         // odd dims
  }
}
__device__ __forceinline__ void unpack_a(unsigned w, v4i& a0, v4i& a1) {
  // Dword i holds bits i, i + 8, i + 16, i + 24 as bytes 0/1 (dims 32g + 8j + i).
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a0[i] = (int)((w >> i) & 0x01010101u);
    a1[i] = (int)((w >> (i + 4)) & 0x01010101u);
  }
}
// Sign bits in the int4 lane order (a0: even dims, a1: odd dims), for a sign
// stream that shares its query operands with an int4 stream.  Bits 0, 2, 4, 6
// of a byte move to bits 0, 8, 16, 24 by one multiply with 0x41041 (shifts
// 0, 6, 12, 18): the partial products overlap only at bits 6, 12 and 18,
// whose carries stop at bits 7, 13 and 19, away from the kept bits.
__device__ __forceinline__ void unpack_a_int4_order(unsigned w, v4i& a0, v4i& a1) {
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const unsigned b = w >> (8 * x);
    a0[x] = (int)(((b & 0x55u) * 0x41041u) & 0x01010101u);
    a1[x] = (int)((((b >> 1) & 0x55u) * 0x41041u) & 0x01010101u);
  }
}

// Three limbs, four row blocks, one stream: the row-block pipeline in table
// mode (direct mode keeps the tile ring), in workgroups of eight waves, two
// per SIMD, that share a list of work units.
constexpr bool score_block_pipe(int nt, int limbs, bool res, int kc) { return nt > 2 && limbs == 3 && !res && kc == 1; }
constexpr int score_group_waves(int nt, int limbs, bool res, int kc) {
  return score_block_pipe(nt, limbs, res, kc) ? 8 : kWavesPerGroup;
}

// INTMAX (sign documents, one int8 limb, no token scale, MaxSim): the
// +-1 dot 2 (q8 . bits) - sum(q8) is increasing in the MFMA result, so the
// running maximum is kept on the int32 accumulators and converted once per
// document.  KC: 128-dim chunks per token (dims above 128), each two more
// MFMAs into the same accumulators.
template <int DOC, bool RES, int L, int NT, int RED, bool INTMAX, int KC = 1>
__global__ __launch_bounds__(kWave * score_group_waves(NT, L, RES, KC), NT == 8 ? 2 : 1) void score_kernel(
    ScoreArgs p) {
  static_assert(!INTMAX || (DOC == kDocSign && !RES && L == 1 && RED == kRedMax), "integer maximum form");
  static_assert(KC == 1 || (L == 3 && !(DOC == kDocSign && RES)), "chunked dims: fp32 queries, one document format");
  constexpr int kCodeBytes = (DOC == kDocInt4 ? 64 : 16) * KC;  // bytes per token of `codes`
  constexpr int kResBytes = 64 * KC;                            // and of `rcodes`
  constexpr int kQueryBytes = 128 * KC;                          // bytes per query row of a limb
  constexpr bool kBlockPipe = score_block_pipe(NT, L, RES, KC);
  constexpr int kGroupWaves = score_group_waves(NT, L, RES, KC);
  __shared__ float s_pool[kGroupWaves][16 * NT];
  const int lane = lane_id();
  const int wave = wave_uniform(threadIdx.x / kWave);
  const int g = lane >> 4, c = lane & 15;
  const int grp = (int)blockIdx.y / p.subs, sub = (int)blockIdx.y % p.subs;
  const int64_t gw = (int64_t)blockIdx.x * kGroupWaves + wave;
  const auto targets = p.targets ? as_constant(p.targets) + grp * p.targets_grp_stride : nullptr;
  const int lr0 = sub * 16 * NT;                           // first local row of the pass
  const int64_t grow0 = (int64_t)grp * p.grp_rows + lr0;  // its global query row

  // Row-block pipeline: the waves of a workgroup share one pass of query
  // rows, so its B operands are read from global memory once per workgroup,
  // as whole 128-byte rows, and each wave takes its registers from LDS
  // (before any wave may leave).  s_next counts the work units taken.
  constexpr int kStageVecs = kBlockPipe ? L * NT * 2 * kWave : 1;
  __shared__ v4i s_bq[kStageVecs];
  __shared__ int s_next;
  if constexpr (kBlockPipe) {
    if (threadIdx.x == 0) s_next = 0;
    // Piece x: 16 bytes at 16 (x % 8) of limb row x / 8 (limb l = row /
    // (16 NT), local row 16 j + c); bytes 32 g + 16 h are lane 16 g + c's
    // operand h of row block j.
    for (int x = (int)threadIdx.x; x < kStageVecs; x += kGroupWaves * kWave) {
      const int piece = x & 7, row = x >> 3;
      const int l = row / (16 * NT), lr = row % (16 * NT);
      const v4i v = *reinterpret_cast<const v4i*>(p.qpack + (l * p.rows_padded + grow0 + lr) * 128 + 16 * piece);
      s_bq[((l * NT + lr / 16) * 2 + (piece & 1)) * kWave + (piece >> 1) * 16 + (lr & 15)] = v;
    }
    __syncthreads();
  }

  // Table mode: the wave's first target, tile count and tiles from the
  // tables.  Direct mode: target gw of the group, its tiles from the token
  // range of its document.
  const bool direct = p.direct_offsets != nullptr;
  int64_t t0, ds = 0, de = 0;
  int ntiles;
  const __attribute__((address_space(4))) uint64_t* tt = nullptr;
  if (direct) {
    if (gw >= p.direct_count) return;  // no barriers below: a wave may leave early
    t0 = gw;
    const int64_t doc = targets[gw];
    ds = as_constant(p.direct_offsets)[doc];
    de = as_constant(p.direct_offsets)[doc + 1];
    ntiles = ds == de ? 1 : (int)((de - ds + 15) / 16);
  } else if (kBlockPipe && p.group_units > 0) {
    t0 = 0;  // work units: taken below; tile entries hold absolute targets
    ntiles = 0;
  } else {
    if (gw >= p.num_waves) return;  // the last workgroup's waves past the table
    const auto info = as_constant(p.wave_info) + grp * p.info_grp_stride + gw * kScoreInfoWords;
    t0 = info[0];
    ntiles = (int)info[2];
    if (ntiles == 0) return;
    tt = as_constant(p.tiles) + info[3];
  }
  // Tile i of the wave (i >= ntiles: a padding entry at token 0).
  auto entry = [&](int i) -> uint64_t {
    if (i >= ntiles) return score_tile_entry(0, 1, false, false, 0);
    if (!direct) return tt[i];
    if (ds == de) return score_tile_entry(0, 1, true, true, 0);
    const int64_t x = ds + 16 * (int64_t)i;
    return score_tile_entry(x, min<int64_t>(16, de - x), x + 16 >= de, false, 0);
  };
  const auto doc_scale = p.doc_scale ? as_constant(p.doc_scale) : nullptr;

  // Query B operands and per-column constants.
  v4i bq[L][NT][KC][2];
  float colmul[NT], weight[NT];
  int qsum[L][NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int64_t r = grow0 + 16 * j + c;
#pragma unroll
    for (int l = 0; l < L; ++l) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        if constexpr (kBlockPipe) {
          bq[l][j][kc][0] = s_bq[((l * NT + j) * 2 + 0) * kWave + lane];
          bq[l][j][kc][1] = s_bq[((l * NT + j) * 2 + 1) * kWave + lane];
        } else {
          const v4i* src =
              reinterpret_cast<const v4i*>(p.qpack + (l * p.rows_padded + r) * kQueryBytes + 128 * kc + 32 * g);
          bq[l][j][kc][0] = src[0];
          bq[l][j][kc][1] = src[1];
        }
      }
      qsum[l][j] = DOC == kDocSign ? p.qsum[l * p.rows_padded + r] : 0;
    }
    colmul[j] = p.colmul[r];
    weight[j] = p.weights ? p.weights[r] : 1.0f;
  }
  const float k2 = kLog2e / p.temperature;

  ReducerState<RED> st[NT];
  int imax[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    st[j].init();
    imax[j] = INT32_MIN;
  }

  struct Tile {
    uint64_t e;  // its table entry (table mode)
    TileCodes<DOC, KC> a;
    TileCodes<kDocInt4, KC> r;
    float s[4], sr[4];
  };
  // Every load is unconditional: rows past a short document read its last
  // token again (masked below); table padding entries point at token 0.
  auto load = [&](uint64_t e, Tile& t) {
    t.e = e;
    const int64_t start = (int64_t)(e & kTileStartMask);
    const int rows1 = (int)((e >> kTileRowsShift) & 15);
    const int64_t tok = start + min(c, rows1);
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      if constexpr (DOC == kDocInt4)
        t.a.w[kc] = *reinterpret_cast<const v4u*>(p.codes + tok * kCodeBytes + 64 * kc + 16 * g);
      else
        t.a.w[kc] = *reinterpret_cast<const unsigned*>(p.codes + tok * kCodeBytes + 16 * kc + 4 * g);
      if constexpr (RES) t.r.w[kc] = *reinterpret_cast<const v4u*>(p.rcodes + tok * kResBytes + 64 * kc + 16 * g);
    }
    if constexpr (!INTMAX) {
      // Token rows 4g .. 4g + 3 in one load; rows past the tile read 0
      // (buffer bounds at the tile's last row; they are masked below).
      const uint32_t nbytes = (uint32_t)(rows1 + 1) * 4u;
      const v4u sv = load_b128(make_rsrc(p.tscale + start, nbytes), 16 * g);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) t.s[rr] = __uint_as_float(sv[rr]);
      if constexpr (RES) {
        const v4u rv = load_b128(make_rsrc(p.rtscale + start, nbytes), 16 * g);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) t.sr[rr] = __uint_as_float(rv[rr]);
      }
    }
  };

  int len = 0;  // tokens of the current target seen so far (wave-uniform)
  float dscale = 1.0f;
  bool fresh = true;

  // Accumulators of one tile, and what its epilogue needs once its ring slot
  // is reused.
  struct Acc {
    v4i s[L][NT];
    v4i r[RES ? L : 1][RES ? NT : 1];
  };
  // int4 documents with three limbs and one or two 128-dim chunks: limb 1's
  // accumulator starts at -kLimb1Bias and limb 2's at the bits of
  // K = 254 kLimb1Bias = 12583160, in [2^23, 2^24) with room for
  // |a2| <= 128 * 127 * 128 * KC < 2^22 on either side, so it holds the
  // float K + a2 exactly.  The similarity s (a0 + a1 / 254 + a2 / 254^2)
  // (s: token scale times tmul) is then
  //   fma(W, s / 254, fma(F2, s / 254^2, add)),  W = 254 a0 + a1 - kLimb1Bias
  // (one v_mad_i32_i24; |a0| < 2^23, |W| < 2^31), F2 the accumulator read as
  // a float: four VALU instructions instead of five (no conversion of a2),
  // the biases cancelling as -kLimb1Bias s / 254 + K s / 254^2 = 0.  With
  // q1 = s / 254 and q2 = s / 254^2 rounded separately the cancellation
  // leaves at most about 2^-23 K q2 < 2 s / 254^2 < 3.1e-5 s, and the
  // rounding of fma(F2, q2, add) near K q2 adds 0.5 ulp of it, about 0.75 s
  // / 254^2: against terms of s a0, |a0| in the thousands for any sizeable
  // similarity.  `add` (-0 or a mask's -inf) joins the inner fma.
  // (Not with the residual stream at two chunks: its registers would drop
  // the kernel to one wave per SIMD.)
  constexpr bool kBias2 = L == 3 && DOC == kDocInt4 && (KC == 1 || (KC == 2 && !RES));
  struct Pend {
    uint64_t e;
    float s[4], sr[4];
    float q1[kBias2 ? 4 : 1], q2[kBias2 ? 4 : 1];
    float r1[kBias2 && RES ? 4 : 1], r2[kBias2 && RES ? 4 : 1];
  };
  auto pend_of = [&](const Tile& t) {
    Pend q;
    q.e = t.e;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      q.s[rr] = t.s[rr];
      q.sr[rr] = RES ? t.sr[rr] : 0.0f;
      if constexpr (kBias2) {
        q.q1[rr] = t.s[rr] * (p.tmul * kLimbStep);
        q.q2[rr] = t.s[rr] * (p.tmul * kLimbStep2);
        if constexpr (RES) {
          q.r1[rr] = t.sr[rr] * (p.rmul * kLimbStep);
          q.r2[rr] = t.sr[rr] * (p.rmul * kLimbStep2);
        }
      }
    }
    return q;
  };
  // C operand of a limb's first MFMA of a tile.
  v4i cbias1 = {-kLimb1Bias, -kLimb1Bias, -kLimb1Bias, -kLimb1Bias};
  v4i cbias2 = {kLimb2Bias, kLimb2Bias, kLimb2Bias, kLimb2Bias};
  if constexpr (kBias2) asm volatile("" : "+v"(cbias1), "+v"(cbias2));  // kept in VGPRs
  auto cstart = [&](int l) -> v4i {
    const v4i zero = {0, 0, 0, 0};
    return !kBias2 || l == 0 ? zero : l == 1 ? cbias1 : cbias2;
  };
  struct Ops {
    v4i a0, a1, r0, r1;
  };
  // (The pipelined form, one limb, always has one chunk.)
  auto unpack = [&](const Tile& t) {
    Ops o;
    if constexpr (DOC == kDocSign && RES)
      unpack_a_int4_order(t.a.w[0], o.a0, o.a1);
    else
      unpack_a(t.a.w[0], o.a0, o.a1);
    if constexpr (RES) unpack_a(t.r.w[0], o.r0, o.r1);
    return o;
  };
  // MFMAs of K half h of row block j (h = 0 starts from zero).
  auto mfma_half = [&](Acc& A, const Ops& o, int h, int j) __attribute__((always_inline)) {
    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int l = 0; l < L; ++l)
      A.s[l][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(h ? o.a1 : o.a0, bq[l][j][0][h], h ? A.s[l][j] : zero, 0, 0, 0);
    if constexpr (RES) {
#pragma unroll
      for (int l = 0; l < L; ++l)
        A.r[l][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(h ? o.r1 : o.r0, bq[l][j][0][h], h ? A.r[l][j] : zero, 0, 0, 0);
    }
  };
  // Start of a tile's epilogue: its row count, and the document constants
  // when it is its target's first tile.
  auto begin_tile = [&](const Pend& P) __attribute__((always_inline)) {
    const uint64_t e = P.e;
    const int local = (int)(e >> kTileLocalShift);
    if (fresh) {
      const int64_t tg = t0 + local;
      const int64_t doc = targets ? targets[tg] : tg;
      dscale = doc_scale ? doc_scale[doc] : p.scale;
      if constexpr (RED == kRedLse) {
#pragma unroll
        for (int j = 0; j < NT; ++j) st[j].k = colmul[j] * dscale * k2;
      }
    }
    return ((e >> kTileEmptyShift) & 1) ? 0 : (int)((e >> kTileRowsShift) & 15) + 1;
  };
  // Similarity of token row 4g + rr (accumulator row rr) and column c of row
  // block j.  `add` joins the first product in its rounding: -0 leaves it
  // unchanged (x + -0 = x for every x, signed zeros included), -inf masks
  // the row.
  auto zval = [&](const Acc& A, const Pend& P, int j, int rr, float add) __attribute__((always_inline)) {
    // Limb dots combined smallest first; sign documents recover the +-1 dot
    // as 2 (q . bits) - sum(q).
    // int4 documents with three limbs, where the biased form does not apply
    // (four chunks, or the residual stream at two): the two small limbs
    // first as one exact integer, 254 a1 + a2 (|a| <= 128 * 127 * 128 KC <
    // 2^23 for KC <= 4, so the 24-bit multiply and the int32 sum are exact).
    auto limbs3 = [&](const v4i (&a)[L][NT]) {
      const int z12 = __mul24(a[1 % L][j][rr], 254) + a[2 % L][j][rr];  // v_mad_i32_i24
      return fmaf((float)z12, kLimbStep2, (float)a[0][j][rr]);
    };
    if constexpr (kBias2) {
      // The biased form (see Pend).
      auto biased = [&](const v4i (&a)[L][NT], float q1, float q2, float add_) {
        const int w = __mul24(a[0][j][rr], 254) + a[1 % L][j][rr];  // v_mad_i32_i24
        return fmaf((float)w, q1, fmaf(__int_as_float(a[2 % L][j][rr]), q2, add_));
      };
      float z = biased(A.s, P.q1[rr], P.q2[rr], add);
      if constexpr (RES) z = z + biased(A.r, P.r1[rr], P.r2[rr], -0.0f);
      return z;
    }
    float Y;
    if constexpr (L == 3 && DOC == kDocInt4) {
      Y = limbs3(A.s);
    } else {
      float y[L];
#pragma unroll
      for (int l = 0; l < L; ++l)
        // Sign documents: 2 (q . bits) - sum(q) as one fma on the
        // converted dot (every term an integer below 2^24: exact).
        y[l] = DOC == kDocSign ? fmaf((float)A.s[l][j][rr], 2.0f, (float)-qsum[l][j]) : (float)A.s[l][j][rr];
      Y = y[0];
      if constexpr (L == 3) Y = fmaf(fmaf(y[2], kLimbStep, y[1]), kLimbStep, y[0]);
    }
    float z = fmaf(Y, P.s[rr] * p.tmul, add);
    if constexpr (RES) {
      float YR;
      if constexpr (L == 3) {
        YR = limbs3(A.r);
      } else {
        YR = (float)A.r[0][j][rr];
      }
      z = z + YR * (P.sr[rr] * p.rmul);
    }
    return z;
  };
  // Epilogue of row block j of a tile.
  auto epi_j = [&](const Acc& A, const Pend& P, int rows, int j) __attribute__((always_inline)) {
    if constexpr (INTMAX) {
      v4i a = A.s[0][j];
      if (rows < 16) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          if (4 * g + rr >= rows) a[rr] = INT32_MIN;
      }
      imax[j] = max(max(imax[j], max(a[0], a[1])), max(a[2], a[3]));
    } else {
      float z[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) z[rr] = zval(A, P, j, rr, -0.0f);
      if (rows < 16) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          if (4 * g + rr >= rows) z[rr] = kNegInf;
      }
      st[j].add4(z, k2);
    }
  };
  // Score of target tg from the reducer state over its `len` tokens.
  auto finish_target = [&](int64_t tg) __attribute__((always_inline)) {
    float v[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      if constexpr (INTMAX) {
        int m = max(imax[j], __shfl_xor(imax[j], 16));
        m = max(m, __shfl_xor(m, 32));
        v[j] = len == 0 ? 0.0f : (float)(2 * m - qsum[0][j]) * colmul[j] * weight[j] * dscale;
        imax[j] = INT32_MIN;
      } else {
        st[j].merge_xor(16, k2);
        st[j].merge_xor(32, k2);
        v[j] = st[j].finish(len, colmul[j], p.temperature, weight[j], dscale);
        st[j].init();
      }
    }
    if (p.out || p.iout) {
      // Whole batch rows in this pass: sum each row's query tokens here
      // (sequentially from its first token) and write the score.
      if (g == 0) {
#pragma unroll
        for (int j = 0; j < NT; ++j) s_pool[wave][16 * j + c] = v[j];
      }
      wave_sync_lds();
      const int nb = min(16 * NT, p.grp_rows - lr0) / p.query_tokens;
      if (lane < nb) {
        float sum = 0.0f;
        for (int q = 0; q < p.query_tokens; ++q) sum += s_pool[wave][lane * p.query_tokens + q];
        const int64_t b = (grow0 / p.query_tokens) + lane;
        if (p.out) p.out[b * p.out_stride + tg] = sum;
        if (p.iout) p.iout[b * p.iout_stride + tg] = (int32_t)sum;
      }
      wave_sync_lds();
    } else {
      float* out = p.pooled + grp * p.pooled_grp_stride + tg * p.grp_rows;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int lr = lr0 + 16 * j + c;
        if (g == 0 && lr < p.grp_rows) out[lr] = v[j];
      }
    }
    len = 0;
  };
  // End of a tile's epilogue: at its target's last tile, the target's score.
  auto end_tile = [&](const Pend& P, int rows) __attribute__((always_inline)) {
    const uint64_t e = P.e;
    const bool last = ((e >> kTileLastShift) & 1) != 0;
    len += rows;
    if (last) finish_target(t0 + (int)(e >> kTileLocalShift));
    fresh = last;
  };
  // The epilogue of a tile whose MFMAs were issued just before.
  auto consume_now = [&](const Acc& A, const Pend& P, int rows) __attribute__((always_inline)) {
    mfma_results_fence();
#pragma unroll
    for (int j = 0; j < NT; ++j) epi_j(A, P, rows, j);
  };
  // Pipelined form: the MFMAs of tile q, the epilogue of the previous tile p
  // (its accumulators a whole tile old) interleaved with q's second halves.
  auto issue_consume = [&](Acc& Q, const Tile& tq, const Acc& A, const Pend& P, int rows)
                           __attribute__((always_inline)) {
    const Ops o = unpack(tq);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NT; ++j) mfma_half(Q, o, 0, j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      mfma_half(Q, o, 1, j);
      epi_j(A, P, rows, j);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // All MFMAs of a tile: the first stream's halves, chunk by chunk, then the
  // residual's (its operands unpacked only then, so fewer registers are
  // live).  Chunk 0's first half starts from the limb's start value
  // (cstart); every later MFMA adds to the same accumulators.
  auto issue = [&](Acc& Q, const Tile& tq) __attribute__((always_inline)) {
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      v4i a0, a1;
      if constexpr (DOC == kDocSign && RES)
        unpack_a_int4_order(tq.a.w[kc], a0, a1);
      else
        unpack_a(tq.a.w[kc], a0, a1);
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int l = 0; l < L; ++l)
          Q.s[l][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bq[l][j][kc][0], kc == 0 ? cstart(l) : Q.s[l][j], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int l = 0; l < L; ++l)
          Q.s[l][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bq[l][j][kc][1], Q.s[l][j], 0, 0, 0);
    }
    if constexpr (RES) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        v4i r0, r1;
        unpack_a(tq.r.w[kc], r0, r1);
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int l = 0; l < L; ++l)
            Q.r[l][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(r0, bq[l][j][kc][0], kc == 0 ? cstart(l) : Q.r[l][j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int l = 0; l < L; ++l)
            Q.r[l][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(r1, bq[l][j][kc][1], Q.r[l][j], 0, 0, 0);
      }
    }
  };

  // Tiles in flight (a ring of kAhead + 1, tile i in slot i % (kAhead + 1),
  // the loads of tile i + kAhead issued before tile i is computed): three for
  // the two-tile passes (candidate rescoring: few waves per SIMD, short
  // documents), one for eight row blocks (registers).  One-limb two-tile
  // passes interleave each tile's epilogue with the next tile's MFMAs (two
  // accumulator sets); the others fence each tile.  Chunked dims hold more
  // bytes per tile: one in flight.
  constexpr int kAhead = NT <= 2 && KC == 1 ? 3 : 1;
  constexpr bool kPipe = NT <= 2 && L == 1;
  static_assert(!kPipe || (kAhead + 1) % 2 == 0, "tiles alternate between two accumulator sets");

  // The ring loop over tiles 0 .. n - 1: fetch(i, Tile&) issues tile i's
  // loads (i >= n allowed), meta(i, Pend&) returns its row count after
  // starting its epilogue, done(Pend&, rows) ends it.
  auto run_ring = [&](int n, auto fetch, auto meta, auto done) __attribute__((always_inline)) {
    Tile ring[kAhead + 1];
#pragma unroll
    for (int u = 0; u < kAhead; ++u) fetch(u, ring[u]);
    if constexpr (kPipe) {
      Acc acc[2];
      Pend pend[2];
      fetch(kAhead, ring[kAhead]);
      issue(acc[0], ring[0]);
      pend[0] = pend_of(ring[0]);
      int rows_p = meta(0, pend[0]);
      // Tile i (i >= 1) is in slot (u + 1) % (kAhead + 1) and set (u + 1) % 2;
      // its loads reuse the slot of tile i - 1, whose epilogue data is in pend.
      for (int i0 = 1; i0 < n; i0 += kAhead + 1) {
#pragma unroll
        for (int u = 0; u <= kAhead; ++u) {
          if (i0 + u >= n) break;
          const int sl = (u + 1) % (kAhead + 1), so = u % (kAhead + 1);
          const int sq = (u + 1) % 2, sp = u % 2;
          fetch(i0 + u + kAhead, ring[so]);
          pend[sq] = pend_of(ring[sl]);
          issue_consume(acc[sq], ring[sl], acc[sp], pend[sp], rows_p);
          done(pend[sp], rows_p);
          rows_p = meta(i0 + u, pend[sq]);
        }
      }
      if ((n - 1) % 2 == 0) {
        consume_now(acc[0], pend[0], rows_p);
        done(pend[0], rows_p);
      } else {
        consume_now(acc[1], pend[1], rows_p);
        done(pend[1], rows_p);
      }
    } else {
      for (int i0 = 0; i0 < n; i0 += kAhead + 1) {
#pragma unroll
        for (int u = 0; u <= kAhead; ++u) {
          if (i0 + u >= n) break;
          fetch(i0 + u + kAhead, ring[(u + kAhead) % (kAhead + 1)]);
          Acc a;
          issue(a, ring[u]);
          Pend P = pend_of(ring[u]);
          const int rows = meta(i0 + u, P);
          consume_now(a, P, rows);
          done(P, rows);
        }
      }
    }
  };

  if (direct) {
    // One document per wave (tokens [ds, de)): one buffer per stream over
    // the document, a tile's loads at offsets from it (rows past the end
    // read 0 and are masked), the document's constants once before its
    // tiles and its score once after them.
    const int ntok = (int)(de - ds);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.codes + ds * kCodeBytes, (uint32_t)ntok * kCodeBytes);
    const __amdgpu_buffer_rsrc_t rr =
        make_rsrc(RES ? p.rcodes + ds * kResBytes : p.codes, RES ? (uint32_t)ntok * (uint32_t)kResBytes : 0u);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.tscale + ds, (uint32_t)ntok * 4u);
    const __amdgpu_buffer_rsrc_t rsr = make_rsrc(RES ? p.rtscale + ds : p.tscale, RES ? (uint32_t)ntok * 4u : 0u);
    {
      const int64_t doc = targets[gw];
      dscale = doc_scale ? doc_scale[doc] : p.scale;
      if constexpr (RED == kRedLse) {
#pragma unroll
        for (int j = 0; j < NT; ++j) st[j].k = colmul[j] * dscale * k2;
      }
    }
    auto fetch = [&](int i, Tile& t) __attribute__((always_inline)) {
      t.e = 0;
      const int row = 16 * i + c;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        if constexpr (DOC == kDocInt4)
          t.a.w[kc] = load_b128(ra, row * kCodeBytes + 64 * kc + 16 * g);
        else
          t.a.w[kc] = load_b32(ra, row * kCodeBytes + 16 * kc + 4 * g);
        if constexpr (RES) t.r.w[kc] = load_b128(rr, row * kResBytes + 64 * kc + 16 * g);
      }
      if constexpr (!INTMAX) {
        const v4u sv = load_b128(rs, (16 * i + 4 * g) * 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) t.s[q] = __uint_as_float(sv[q]);
        if constexpr (RES) {
          const v4u rv = load_b128(rsr, (16 * i + 4 * g) * 4);
#pragma unroll
          for (int q = 0; q < 4; ++q) t.sr[q] = __uint_as_float(rv[q]);
        }
      }
    };
    auto meta = [&](int i, Pend&) { return max(0, min(16, ntok - 16 * i)); };
    auto done = [&](Pend&, int) {};
    run_ring(ntiles, fetch, meta, done);
    len = ntok;
    finish_target(t0);
  } else if constexpr (kBlockPipe) {
    // Row-block pipeline over a stream of tiles.  Step (i, j) issues the 2L
    // MFMAs of row block j of tile i, each followed by a quarter of the
    // epilogue of the row block two steps back: block j - 2 of tile i, or
    // block NT - 2 + j of tile i - 1.  Its accumulators are then at least 2L
    // MFMAs old (no fence needed), and the matrix core and the VALU work at
    // once within the wave.  Row block j keeps accumulator set j: block
    // j - 2's epilogue reads set j - 2 while set j is written, and set j is
    // rewritten (tile i + 1) only after block j's epilogue (step j + 2, or
    // step j + 2 - NT of tile i + 1).  A tile's masked rows (past a short
    // document) get -inf in the same rounding as their product (the fma
    // addend of zval).  Tiles in flight: a ring of kRing, the loads of tile
    // i + kRing - 1 issued before tile i is computed.
    //
    // The stream: the wave's table (static tables), or the work units it
    // takes from its workgroup's list (group_units > 0): unit A holds the
    // current tile, unit B the next one, taken as A starts.  Every unit but
    // a workgroup's last has at least kRing - 1 tiles, so the tiles loaded
    // ahead lie in A or B.  The two waves of a SIMD do not share it evenly
    // (the older wave issues first); taking units as they go, both finish
    // with the workgroup's list.
    constexpr int kRing = 4;
    static_assert(kScoreUnitMinTiles >= kRing - 1, "units cover the tiles loaded ahead");
    const bool units = p.group_units > 0;
    const auto unit_info = as_constant(p.wave_info) + grp * p.info_grp_stride +
                           (int64_t)blockIdx.x * p.group_units * kScoreInfoWords;
    using TilePtr = const __attribute__((address_space(4))) uint64_t*;
    auto take = [&](TilePtr& tp, int& n) __attribute__((always_inline)) {
      int k = 0;
      if (lane == 0) k = atomicAdd(&s_next, 1);
      k = __builtin_amdgcn_readfirstlane(k);
      n = 0;
      if (k < p.group_units) {
        const auto rec = unit_info + (int64_t)k * kScoreInfoWords;
        n = (int)rec[2];
        tp = as_constant(p.tiles) + rec[3];
      }
    };
    TilePtr ta = tt, tb = nullptr;
    int na = ntiles, nb = 0, base = 0;
    if (units) {
      take(ta, na);
      if (na == 0) return;  // no barriers below
      take(tb, nb);
    }
    auto entry_s = [&](int pos) -> uint64_t {
      int q = pos - base;
      if (q < na) return ta[q];
      q -= na;
      if (q < nb) return tb[q];
      return score_tile_entry(0, 1, false, false, 0);
    };
    Tile ring[kRing];
#pragma unroll
    for (int u = 0; u < kRing - 1; ++u) load(entry_s(u), ring[u]);
    Acc A;
    Pend Pc, Pp;
    float mc[4], mp[4];
    int rows_c = 0, rows_p = 0;
    auto mask_of = [&](int rows, float (&m)[4]) __attribute__((always_inline)) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) m[rr] = 4 * g + rr >= rows ? kNegInf : -0.0f;
    };
    auto step = [&](const Ops& o, int jq, bool epi, const Pend& P, const float (&m)[4], int jp)
                    __attribute__((always_inline)) {
      float z[4];
#pragma unroll
      for (int k = 0; k < 2 * L; ++k) {
        const int l = k % L, h = k / L;
        A.s[l][jq] = __builtin_amdgcn_mfma_i32_16x16x64_i8(h ? o.a1 : o.a0, bq[l][jq][0][h],
                                                          h ? A.s[l][jq] : cstart(l), 0, 0, 0);
        if (epi && k < 4) z[k] = zval(A, P, jp, k, m[k]);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (epi) st[jp].add4(z, k2);
    };
    // Steps 0 .. NT - 1 of a tile (FIRST: tile 0, no previous tile).
    auto tile_steps = [&](auto first_c, const Tile& t) __attribute__((always_inline)) {
      constexpr bool kFirst = decltype(first_c)::value;
      const Ops o = unpack(t);
      Pc = pend_of(t);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (j < 2) {
          step(o, j, !kFirst, Pp, mp, NT - 2 + j);
          if (!kFirst && j == 1) end_tile(Pp, rows_p);
        } else {
          if (j == 2) {
            rows_c = begin_tile(Pc);
            mask_of(rows_c, mc);
          }
          step(o, j, true, Pc, mc, j - 2);
        }
      }
      Pp = Pc;
      rows_p = rows_c;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) mp[rr] = mc[rr];
    };
    // Tile i is in slot i % kRing; tile i + kRing - 1 goes to the slot of
    // tile i - 1, whose steps are done.
    load(entry_s(kRing - 1), ring[kRing - 1]);
    tile_steps(std::integral_constant<bool, true>(), ring[0]);
    for (int i0 = 1;; i0 += kRing) {
      bool done = false;
#pragma unroll
      for (int u = 0; u < kRing; ++u) {
        const int i = i0 + u;
        if (i - base >= na) {  // unit A done: B follows
          if (nb == 0) {
            done = true;
            break;
          }
          base += na;
          ta = tb;
          na = nb;
          nb = 0;
          if (units) take(tb, nb);
        }
        load(entry_s(i + kRing - 1), ring[u]);
        tile_steps(std::integral_constant<bool, false>(), ring[(u + 1) % kRing]);
      }
      if (done) break;
    }
    // The last tile's blocks NT - 2 and NT - 1, right after their MFMAs.
    mfma_results_fence();
#pragma unroll
    for (int j = NT - 2; j < NT; ++j) {
      float z[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) z[rr] = zval(A, Pp, j, rr, mp[rr]);
      st[j].add4(z, k2);
    }
    end_tile(Pp, rows_p);
  } else if constexpr (NT > 2) {
    // Eight row blocks (one limb): a tight loop over the table's tiles, one
    // in flight.
    Tile cur, nxt;
    uint64_t e = tt[0];
    load(e, cur);
    for (int i = 0; i < ntiles; ++i) {
      const uint64_t en = tt[i + 1];  // i + 1 <= ntiles: the table's padding entry last
      load(en, nxt);
      Acc a;
      issue(a, cur);
      Pend P = pend_of(cur);
      const int rows = begin_tile(P);
      consume_now(a, P, rows);
      end_tile(P, rows);
      cur = nxt;
      e = en;
    }
  } else {
    auto fetch = [&](int i, Tile& t) __attribute__((always_inline)) { load(entry(i), t); };
    auto meta = [&](int, Pend& P) { return begin_tile(P); };
    run_ring(ntiles, fetch, meta, end_tile);
  }
}

// ------------------------------------------------------------ quantisation

// Byte position of dim d in a 128-byte query row for the MFMA B operands.
// int4 documents: lane group g = d / 32 holds the even dims of its 32 in
// bytes [32g, 32g + 16) and the odd dims in [32g + 16, 32g + 32) (the order
// of the low / high nibbles).  Sign documents: byte 32g + 16 (i / 4) +
// 4 (i % 4) + j holds dim 32g + 8j + i (the order of the unpacked bits).
__device__ __forceinline__ int query_byte(int d, int layout) {
  const int g = d >> 5, e = d & 31;
  if (layout == kDocInt4) return 32 * g + (e & 1) * 16 + (e >> 1);
  const int j = e >> 3, i = e & 7;
  return 32 * g + 16 * (i >> 2) + 4 * (i & 3) + j;
}

// One wave per query row of 128 * chunks dims (lane l holds dims 128 kc +
// 2l, 128 kc + 2l + 1 of each chunk kc; each chunk's bytes in the B-operand
// order of a 128-dim row).  sigma = f32(max|q| / 127) over the whole row
// (0 -> 1); limb l: a_l = clip(rint(r_l / s_l), -127, 127), r_{l+1} = r_l -
// a_l s_l (one rounding), s_{l+1} = s_l / 254.  With `recip` (one limb) the
// quotient is q * (1 / sigma), the binary int8 query rounding of
// cu:1328-1366.  colmul = sigma; qsum[l] = sum of limb l.  With qpack2
// (one chunk), the same codes also in layout2 (a cascade's two passes).
__global__ __launch_bounds__(256) void quantize_limbs_kernel(const float* __restrict__ query, int64_t rows,
                                                             int64_t rows_padded, int limbs, int layout,
                                                             int recip, int8_t* __restrict__ qpack,
                                                             float* __restrict__ colmul,
                                                             int32_t* __restrict__ qsum, int layout2,
                                                             int8_t* __restrict__ qpack2, int chunks) {
  constexpr int kMaxChunks = 4;
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= rows_padded) return;
  const int64_t width = 128 * (int64_t)chunks;
  const int d0 = 2 * lane, d1 = 2 * lane + 1;
  const int p0 = query_byte(d0, layout), p1 = query_byte(d1, layout);
  const int p20 = query_byte(d0, layout2), p21 = query_byte(d1, layout2);
  if (row >= rows) {
    for (int l = 0; l < limbs; ++l) {
      int8_t* dst = qpack + (l * rows_padded + row) * width;
      for (int kc = 0; kc < chunks; ++kc) {
        dst[128 * kc + p0] = 0;
        dst[128 * kc + p1] = 0;
      }
      if (qpack2) {
        int8_t* dst2 = qpack2 + (l * rows_padded + row) * 128;
        dst2[p20] = 0;
        dst2[p21] = 0;
      }
      if (lane == 0) qsum[l * rows_padded + row] = 0;
    }
    if (lane == 0) colmul[row] = 0.0f;
    return;
  }
  float rx[kMaxChunks], ry[kMaxChunks];
  float mabs = 0.0f;
#pragma unroll
  for (int kc = 0; kc < kMaxChunks; ++kc) {
    rx[kc] = ry[kc] = 0.0f;
    if (kc < chunks) {
      const float2 v = reinterpret_cast<const float2*>(query + row * width + 128 * kc)[lane];
      rx[kc] = v.x;
      ry[kc] = v.y;
      mabs = fmaxf(mabs, fmaxf(fabsf(v.x), fabsf(v.y)));
    }
  }
  const float m = wave_reduce(mabs, [](float x, float y) { return fmaxf(x, y); });
  const float sigma = m == 0.0f ? 1.0f : __fdiv_rn(m, 127.0f);
  float s = sigma;
  for (int l = 0; l < limbs; ++l) {
    const float inv = recip ? __fdiv_rn(1.0f, s) : 0.0f;
    int8_t* dst = qpack + (l * rows_padded + row) * width;
    int lane_sum = 0;
#pragma unroll
    for (int kc = 0; kc < kMaxChunks; ++kc) {
      if (kc >= chunks) break;
      const float qx = recip ? rx[kc] * inv : __fdiv_rn(rx[kc], s);
      const float qy = recip ? ry[kc] * inv : __fdiv_rn(ry[kc], s);
      const int a = max(-127, min(127, (int)rintf(qx)));
      const int b = max(-127, min(127, (int)rintf(qy)));
      dst[128 * kc + p0] = (int8_t)a;
      dst[128 * kc + p1] = (int8_t)b;
      if (qpack2) {
        int8_t* dst2 = qpack2 + (l * rows_padded + row) * 128;
        dst2[p20] = (int8_t)a;
        dst2[p21] = (int8_t)b;
      }
      lane_sum += a + b;
      rx[kc] = fmaf(-(float)a, s, rx[kc]);
      ry[kc] = fmaf(-(float)b, s, ry[kc]);
    }
    const int sum = wave_reduce(lane_sum, [](int x, int y) { return x + y; });
    if (lane == 0) qsum[l * rows_padded + row] = sum;
    s = s * kLimbStep;
  }
  if (lane == 0) colmul[row] = sigma;
}

// Sign-binarised query rows (pack_signs bit order, 16 bytes per row) as
// +-1 int8 codes in the sign-document layout; colmul = 1.
__global__ __launch_bounds__(256) void quantize_bits_kernel(const uint8_t* __restrict__ qbits, int64_t rows,
                                                            int64_t rows_padded, int8_t* __restrict__ qpack,
                                                            float* __restrict__ colmul,
                                                            int32_t* __restrict__ qsum) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= rows_padded) return;
  const int d0 = 2 * lane, d1 = 2 * lane + 1;
  int8_t* dst = qpack + row * 128;
  int a = 0, b = 0;
  if (row < rows) {
    const unsigned byte = qbits[row * 16 + (d0 >> 3)];
    a = ((byte >> (d0 & 7)) & 1) ? 1 : -1;
    b = ((byte >> (d1 & 7)) & 1) ? 1 : -1;
  }
  dst[query_byte(d0, kDocSign)] = (int8_t)a;
  dst[query_byte(d1, kDocSign)] = (int8_t)b;
  const int sum = wave_reduce(a + b, [](int x, int y) { return x + y; });
  if (lane == 0) {
    qsum[row] = sum;
    colmul[row] = row < rows ? 1.0f : 0.0f;
  }
}

// out[b, t] = sum over q < Q of pooled[b * bs + t * ts + q] (sequential, f32).
__global__ __launch_bounds__(256) void pool_sum_kernel(const float* __restrict__ pooled, int64_t batch,
                                                       int64_t query_tokens, int64_t targets, int64_t bs,
                                                       int64_t ts, float* __restrict__ out, int64_t out_stride,
                                                       int32_t* __restrict__ iout) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= batch * targets) return;
  const int64_t b = idx / targets, t = idx % targets;
  const float* src = pooled + b * bs + t * ts;
  float sum = 0.0f;
  for (int64_t q = 0; q < query_tokens; ++q) sum += src[q];
  if (out) out[b * out_stride + t] = sum;
  if (iout) iout[b * targets + t] = (int32_t)sum;
}

template <int DOC, bool RES, int L, int NT, int KC = 1>
hipError_t launch_red(const ScoreArgs& a, int reducer, dim3 grid, hipStream_t s) {
  // Workgroups of kGroupWaves waves (the last one's waves past num_waves leave).
  constexpr int kGroupWaves = score_group_waves(NT, L, RES, KC);
  constexpr int kThr = kGroupWaves * kWave;
  grid.x = (unsigned)(a.group_units > 0 ? a.num_waves / a.group_units : (a.num_waves + kGroupWaves - 1) / kGroupWaves);
  if (a.group_units > 0 && !score_block_pipe(NT, L, RES, KC)) return hipErrorInvalidValue;
  if constexpr (DOC == kDocSign && !RES && L == 1) {
    if (reducer == kRedMax && a.unit_tscale) {
      score_kernel<DOC, RES, L, NT, kRedMax, true><<<grid, kThr, 0, s>>>(a);
      return hipGetLastError();
    }
  }
  switch (reducer) {
    case kRedMax: score_kernel<DOC, RES, L, NT, kRedMax, false, KC><<<grid, kThr, 0, s>>>(a); break;
    case kRedTop2: score_kernel<DOC, RES, L, NT, kRedTop2, false, KC><<<grid, kThr, 0, s>>>(a); break;
    case kRedTop4: score_kernel<DOC, RES, L, NT, kRedTop4, false, KC><<<grid, kThr, 0, s>>>(a); break;
    case kRedLse: score_kernel<DOC, RES, L, NT, kRedLse, false, KC><<<grid, kThr, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

int score_rows_per_pass(int limbs, int64_t rows, int chunks) {
  // Three limbs keep at most four 16-row tiles of B operands in registers
  // per 128-dim chunk budget (two tiles at two chunks, one at four), one limb
  // eight; small queries use two tiles.
  if (chunks == 2) return 32;
  if (chunks >= 4) return 16;
  const int max_nt = limbs == 3 ? 4 : 8;
  return 16 * (rows <= 32 ? 2 : max_nt);
}

hipError_t launch_score(const ScoreArgs& a, int doc, bool residual, int limbs, int reducer, int64_t groups,
                        hipStream_t stream) {
  if (a.num_waves <= 0 || a.subs <= 0 || groups <= 0) return hipErrorInvalidValue;
  if (a.group_units > 0 ? a.num_waves % a.group_units != 0 : a.num_waves % kWavesPerGroup != 0)
    return hipErrorInvalidValue;
  if (a.tscale == nullptr || (residual && (a.rcodes == nullptr || a.rtscale == nullptr)))
    return hipErrorInvalidValue;
  const int chunks = a.chunks <= 0 ? 1 : a.chunks;
  const int rpp = score_rows_per_pass(limbs, a.grp_rows, chunks);
  const int nt = rpp / 16;
  const dim3 grid((unsigned)(a.num_waves / kWavesPerGroup), (unsigned)(groups * a.subs));
  if (chunks != 1) {
    // Dims above 128: fp32 queries (three limbs) against int4 documents (with
    // or without the int4 residual) or sign documents.
    if (limbs != 3 || (doc == kDocSign && residual)) return hipErrorInvalidValue;
    if (chunks == 2) {
      if (doc == kDocInt4 && !residual) return launch_red<kDocInt4, false, 3, 2, 2>(a, reducer, grid, stream);
      if (doc == kDocInt4) return launch_red<kDocInt4, true, 3, 2, 2>(a, reducer, grid, stream);
      return launch_red<kDocSign, false, 3, 2, 2>(a, reducer, grid, stream);
    }
    if (chunks == 4) {
      if (doc == kDocInt4 && !residual) return launch_red<kDocInt4, false, 3, 1, 4>(a, reducer, grid, stream);
      if (doc == kDocInt4) return launch_red<kDocInt4, true, 3, 1, 4>(a, reducer, grid, stream);
      return launch_red<kDocSign, false, 3, 1, 4>(a, reducer, grid, stream);
    }
    return hipErrorInvalidValue;
  }
#define MSIM_SCORE_NT(DOC, RES, L)                                              \
  return nt == 2 ? launch_red<DOC, RES, L, 2>(a, reducer, grid, stream)         \
                 : launch_red<DOC, RES, L, (L == 3 ? 4 : 8)>(a, reducer, grid, stream)
  if (doc == kDocInt4 && !residual && limbs == 3) { MSIM_SCORE_NT(kDocInt4, false, 3); }
  if (doc == kDocInt4 && residual && limbs == 3) { MSIM_SCORE_NT(kDocInt4, true, 3); }
  if (doc == kDocSign && !residual && limbs == 3) { MSIM_SCORE_NT(kDocSign, false, 3); }
  if (doc == kDocSign && !residual && limbs == 1) { MSIM_SCORE_NT(kDocSign, false, 1); }
  if (doc == kDocSign && residual && limbs == 1) { MSIM_SCORE_NT(kDocSign, true, 1); }
  if (doc == kDocSign && residual && limbs == 3) { MSIM_SCORE_NT(kDocSign, true, 3); }
#undef MSIM_SCORE_NT
  return hipErrorInvalidValue;
}

hipError_t launch_quantize_limbs(const float* d_query, int64_t rows, int64_t rows_padded, int limbs, int layout,
                                 bool recip, int8_t* qpack, float* colmul, int32_t* qsum, hipStream_t stream,
                                 int layout2, int8_t* qpack2, int chunks) {
  if (rows_padded <= 0) return hipSuccess;
  if (chunks != 1 && chunks != 2 && chunks != 4) return hipErrorInvalidValue;
  if (qpack2 && chunks != 1) return hipErrorInvalidValue;
  const int64_t blocks = (rows_padded + 3) / 4;
  quantize_limbs_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(d_query, rows, rows_padded, limbs, layout,
                                                                        recip ? 1 : 0, qpack, colmul, qsum,
                                                                        qpack2 ? layout2 : layout, qpack2, chunks);
  return hipGetLastError();
}

hipError_t launch_quantize_bits(const uint8_t* d_qbits, int64_t rows, int64_t rows_padded, int8_t* qpack,
                                float* colmul, int32_t* qsum, hipStream_t stream) {
  if (rows_padded <= 0) return hipSuccess;
  const int64_t blocks = (rows_padded + 3) / 4;
  quantize_bits_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(d_qbits, rows, rows_padded, qpack, colmul,
                                                                       qsum);
  return hipGetLastError();
}

hipError_t launch_pool_sum(const float* pooled, int64_t batch, int64_t query_tokens, int64_t targets, int64_t bs,
                           int64_t ts, float* out, int64_t out_stride, int32_t* iout, hipStream_t stream) {
  const int64_t n = batch * targets;
  if (n <= 0) return hipSuccess;
  pool_sum_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream>>>(pooled, batch, query_tokens, targets,
                                                                             bs, ts, out, out_stride, iout);
  return hipGetLastError();
}

}  // namespace msim

// ------------------------------------------------------------ fp4 Hamming

namespace msim {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

// 32 sign bits of one lane (dims 32g .. 32g + 31, bit b = dim 32g + b; set =
// +1) as the fp4 (e2m1) operand of v_mfma_scale_f32_16x16x128_f8f6f4: dword
// q holds dims 32g + 4i + q in nibble i, +1 as 0x2 and -1 as 0xA.  Queries and
// documents use the same dim order, so the MFMA's K order is irrelevant.
__device__ __forceinline__ v4i fp4_signs(unsigned w) {
  const unsigned n = ~w;
  v4i a;
  a[0] = (int)(0x22222222u | ((n << 3) & 0x88888888u));
  a[1] = (int)(0x22222222u | ((n << 2) & 0x88888888u));
  a[2] = (int)(0x22222222u | ((n << 1) & 0x88888888u));
  a[3] = (int)(0x22222222u | (n & 0x88888888u));
  return a;
}

__device__ __forceinline__ v4f mfma_fp4(const v4i& a, const v4i& b) {
  typedef int v8i __attribute__((ext_vector_type(8)));
  const v8i a8 = {a[0], a[1], a[2], a[3], 0, 0, 0, 0}, b8 = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
  const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // Formats 4 / 4: fp4 A and B; E8M0 scales 127 = 2^0.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b8, zero, 4, 4, 0, 127, 0, 127);
}

// MaxSim of sign-bit queries against sign documents, Hamming form: the +-1
// dot q . d = 128 - 2 popcount(q ^ d) of each (query row, token), its maximum
// over a document's tokens, summed over the query tokens of a batch row (the
// sum cpu_extension.cpp:82-126 computes for +-1 queries; every value an
// integer below 2^24, so float sums and maxima are exact).  One v_mfma_scale_f32_16x16x128_f8f6f4 on fp4 +-1
// operands covers 16 tokens x 16 query rows x 128 dims (twice the K of the
// int8 MFMA at the same issue rate), so a pass holds 256 query rows (NT = 16
// blocks).  Table mode over every document (build_score_tables), tiles in a
// ring of eight words per lane; rows past a short document read its last
// token again, which leaves every maximum unchanged.
template <int NT>
__global__ __launch_bounds__(kThreads, 2) void hamming_kernel(ScoreArgs p) {
  constexpr int kRing = 8;
  __shared__ float s_pool[kWavesPerGroup][16 * NT];
  const int lane = lane_id();
  const int wave = wave_uniform(threadIdx.x / kWave);
  const int g = lane >> 4, c = lane & 15;
  const int sub = (int)blockIdx.y;
  const int64_t gw = (int64_t)blockIdx.x * kWavesPerGroup + wave;
  const auto info = as_constant(p.wave_info) + gw * kScoreInfoWords;
  const int64_t t0 = info[0];
  const int ntiles = (int)info[2];
  if (ntiles == 0) return;
  const auto tt = as_constant(p.tiles) + info[3];
  const int lr0 = sub * 16 * NT;  // first query row of the pass

  // Query operands: rows lr0 + 16 j + c (rows past the query read 0 bits).
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.qbits, (uint32_t)p.grp_rows * 16u);
  v4i bq[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) bq[j] = fp4_signs(load_b32(rq, (lr0 + 16 * j + c) * 16 + 4 * g));

  float m[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) m[j] = -1.0e30f;
  int len = 0;

  auto entry = [&](int i) -> uint64_t { return i < ntiles ? tt[i] : score_tile_entry(0, 1, false, false, 0); };
  auto word = [&](uint64_t e) -> unsigned {
    const int64_t start = (int64_t)(e & kTileStartMask);
    const int rows1 = (int)((e >> kTileRowsShift) & 15);
    return *reinterpret_cast<const unsigned*>(p.codes + (start + min(c, rows1)) * 16 + 4 * g);
  };
  auto finish = [&](int64_t tg) {
    float v[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      float x = fmaxf(m[j], __shfl_xor(m[j], 16));
      x = fmaxf(x, __shfl_xor(x, 32));
      v[j] = len == 0 ? 0.0f : x * p.scale;
      m[j] = -1.0e30f;
    }
    if (p.out || p.iout) {
      if (g == 0) {
#pragma unroll
        for (int j = 0; j < NT; ++j) s_pool[wave][16 * j + c] = v[j];
      }
      wave_sync_lds();
      const int nb = min(16 * NT, p.grp_rows - lr0) / p.query_tokens;
      if (lane < nb) {
        float sum = 0.0f;
        for (int q = 0; q < p.query_tokens; ++q) sum += s_pool[wave][lane * p.query_tokens + q];
        const int64_t b = lr0 / p.query_tokens + lane;
        if (p.out) p.out[b * p.out_stride + tg] = sum;
        if (p.iout) p.iout[b * p.iout_stride + tg] = (int32_t)sum;
      }
      wave_sync_lds();
    } else {
      float* out = p.pooled + tg * p.grp_rows;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int lr = lr0 + 16 * j + c;
        if (g == 0 && lr < p.grp_rows) out[lr] = v[j];
      }
    }
    len = 0;
  };

  // Ring: tile i's word in slot i % kRing, loaded kRing tiles ahead.  A
  // tile's maxima wait behind the MFMA-result fence (two accumulator sets,
  // one tile old, would spill at 256 query rows per pass).
  uint64_t es[kRing];
  unsigned ws[kRing];
#pragma unroll
  for (int u = 0; u < kRing; ++u) {
    es[u] = entry(u);
    ws[u] = word(es[u]);
  }
  for (int i0 = 0; i0 < ntiles; i0 += kRing) {
#pragma unroll
    for (int u = 0; u < kRing; ++u) {
      if (i0 + u >= ntiles) break;
      const uint64_t e = es[u];
      const unsigned w = ws[u];
      es[u] = entry(i0 + u + kRing);
      ws[u] = word(es[u]);
      if (((e >> kTileEmptyShift) & 1) == 0) {
        const v4i a = fp4_signs(w);
        v4f acc[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j] = mfma_fp4(a, bq[j]);
        mfma_results_fence();
#pragma unroll
        for (int j = 0; j < NT; ++j) m[j] = fmaxf(fmaxf(m[j], fmaxf(acc[j][0], acc[j][1])), fmaxf(acc[j][2], acc[j][3]));
        len += (int)((e >> kTileRowsShift) & 15) + 1;
      }
      if ((e >> kTileLastShift) & 1) finish(t0 + (int64_t)(e >> kTileLocalShift));
    }
  }
}

}  // namespace

hipError_t launch_hamming(const ScoreArgs& a, hipStream_t stream) {
  if (a.num_waves <= 0 || a.num_waves % kWavesPerGroup != 0 || a.subs <= 0 || a.qbits == nullptr ||
      a.wave_info == nullptr || a.tiles == nullptr)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)(a.num_waves / kWavesPerGroup), (unsigned)a.subs);
  hamming_kernel<kHammingRowsPerPass / 16><<<grid, kThreads, 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace msim
