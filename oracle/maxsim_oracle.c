/*
 * maxsim_oracle.c -- CPU restatement of the reference MaxSim semantics.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py.  The product never links this file.
 *
 * Build: make -C oracle   (plain gcc, -ffp-contract=off so every float
 * operation below is the single rounding it reads as).
 *
 * Every function is pinned by tests/test_oracle.py against the reference's
 * known answers, closed forms or brute force (none is "parity unpinned");
 * the binary LUT score also against the reference's own cpu_extension.cpp,
 * compiled into oracle/_ref by oracle/Makefile.
 */
#include "maxsim_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ sums */

/* numpy's pairwise summation (numpy/_core/src/umath/loops_utils.h.src,
 * PW_BLOCKSIZE 128), which np.add.reduce uses for contiguous float vectors;
 * the reference's float64 `(best * q_scales).sum()` (tests/test_int4_int8q.py:25)
 * and float32 `.sum(dtype=np.float32)` (_api.py:568-584) both reduce this way. */
double orc_pairwise_sum_f64(const double* a, int64_t n) {
  if (n < 8) {
    double res = 0.0;
    for (int64_t i = 0; i < n; ++i) res += a[i];
    return res;
  }
  if (n <= 128) {
    double r[8];
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    int64_t i = 8;
    for (; i < n - (n % 8); i += 8)
      for (int j = 0; j < 8; ++j) r[j] += a[i + j];
    double res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += a[i];
    return res;
  }
  int64_t n2 = n / 2;
  n2 -= n2 % 8;
  return orc_pairwise_sum_f64(a, n2) + orc_pairwise_sum_f64(a + n2, n - n2);
}

float orc_pairwise_sum_f32(const float* a, int64_t n) {
  if (n < 8) {
    float res = 0.0f;
    for (int64_t i = 0; i < n; ++i) res += a[i];
    return res;
  }
  if (n <= 128) {
    float r[8];
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    int64_t i = 8;
    for (; i < n - (n % 8); i += 8)
      for (int j = 0; j < 8; ++j) r[j] += a[i + j];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += a[i];
    return res;
  }
  int64_t n2 = n / 2;
  n2 -= n2 % 8;
  return orc_pairwise_sum_f32(a, n2) + orc_pairwise_sum_f32(a + n2, n - n2);
}

/* --------------------------------------------------------------- packing */

static uint8_t nibble(int v) { return (uint8_t)(v & 0x0F); }

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* experimental.py:237-242: s_t = f32(max|x_t|) / f32(7) (0 -> 1);
 * v = clip(rint(x / s_t), -7, 7); bytes = lo | hi << 4 (experimental.py:604-609). */
void orc_pack_int4_token(const float* x, int64_t num_tokens, int dim,
                         uint8_t* codes, int8_t* values, float* token_scale) {
  for (int64_t t = 0; t < num_tokens; ++t) {
    const float* row = x + t * dim;
    float m = 0.0f;
    for (int d = 0; d < dim; ++d) {
      float a = fabsf(row[d]);
      m = a > m ? a : m;
    }
    float s = m / 7.0f;
    if (s == 0.0f) s = 1.0f;
    token_scale[t] = s;
    for (int d = 0; d < dim; ++d) {
      int v = clampi((int)rintf(row[d] / s), -7, 7);
      if (values) values[t * dim + d] = (int8_t)v;
      if (d % 2 == 0)
        codes[t * (dim / 2) + d / 2] = nibble(v);
      else
        codes[t * (dim / 2) + d / 2] |= (uint8_t)(nibble(v) << 4);
    }
  }
}

/* experimental.py:246-258: scale = float(max|x|) / 7.0 in double (1.0 when
 * zero); numpy then divides the float32 array by that Python float, which
 * under NEP 50 is the float32 value of the scale. */
double orc_pack_int4_tensor(const float* x, int64_t num_tokens, int dim,
                            uint8_t* codes, int8_t* values) {
  float m = 0.0f;
  for (int64_t i = 0; i < num_tokens * dim; ++i) {
    float a = fabsf(x[i]);
    m = a > m ? a : m;
  }
  double scale = m == 0.0f ? 1.0 : (double)m / 7.0;
  float fs = (float)scale;
  for (int64_t t = 0; t < num_tokens; ++t) {
    for (int d = 0; d < dim; ++d) {
      int v = clampi((int)rintf(x[t * dim + d] / fs), -7, 7);
      if (values) values[t * dim + d] = (int8_t)v;
      if (d % 2 == 0)
        codes[t * (dim / 2) + d / 2] = nibble(v);
      else
        codes[t * (dim / 2) + d / 2] |= (uint8_t)(nibble(v) << 4);
    }
  }
  return scale;
}

/* sdk.py:1085-1093. */
void orc_unpack_int4(const uint8_t* codes, int64_t num_tokens, int dim, int8_t* values) {
  for (int64_t t = 0; t < num_tokens; ++t) {
    for (int b = 0; b < dim / 2; ++b) {
      int lo = codes[t * (dim / 2) + b] & 0x0F;
      int hi = (codes[t * (dim / 2) + b] >> 4) & 0x0F;
      values[t * dim + 2 * b] = (int8_t)(lo >= 8 ? lo - 16 : lo);
      values[t * dim + 2 * b + 1] = (int8_t)(hi >= 8 ? hi - 16 : hi);
    }
  }
}

/* _api.py:47-52: bit (j % 8) of byte j / 8 is set when x_j >= 0. */
void orc_pack_signs(const float* x, int64_t num_tokens, int dim, uint8_t* out) {
  memset(out, 0, (size_t)(num_tokens * (dim / 8)));
  for (int64_t t = 0; t < num_tokens; ++t)
    for (int d = 0; d < dim; ++d)
      if (x[t * dim + d] >= 0.0f) out[t * (dim / 8) + d / 8] |= (uint8_t)(1u << (d % 8));
}

/* ------------------------------------------------------- int8 query path */

/* tests/test_int4_int8q.py:11-14: sigma = f32(max|q| / 127) (0 -> 1),
 * q8 = clip(rint(q / sigma), -127, 127). */
void orc_quantize_int8(const float* q, int64_t rows, int dim, int8_t* q8, float* qscale) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = q + r * dim;
    float m = 0.0f;
    for (int d = 0; d < dim; ++d) {
      float a = fabsf(row[d]);
      m = a > m ? a : m;
    }
    float s = m == 0.0f ? 1.0f : m / 127.0f;
    qscale[r] = s;
    for (int d = 0; d < dim; ++d) q8[r * dim + d] = (int8_t)clampi((int)rintf(row[d] / s), -127, 127);
  }
}

static int32_t idot(const int8_t* a, const int8_t* b, int dim) {
  int32_t acc = 0;
  for (int d = 0; d < dim; ++d) acc += (int32_t)a[d] * (int32_t)b[d];
  return acc;
}

/* Sum over query tokens of best[q] * sigma[q] in float64, numpy order, times scale. */
static float finish_int8q(const float* best, const float* qscale, int64_t query_tokens,
                          double scale, double* scratch) {
  for (int64_t q = 0; q < query_tokens; ++q) scratch[q] = (double)best[q] * (double)qscale[q];
  return (float)(orc_pairwise_sum_f64(scratch, query_tokens) * scale);
}

/* tests/test_int4_int8q.py:7-26. */
void orc_int4_int8q_scores(const int8_t* q8, const float* qscale, int64_t batch,
                           int64_t query_tokens, int dim, const int8_t* values,
                           const float* token_scale, double scale,
                           const int64_t* offsets, int64_t num_docs, float* out) {
  float* best = (float*)malloc(sizeof(float) * (size_t)(query_tokens > 0 ? query_tokens : 1));
  double* scratch = (double*)malloc(sizeof(double) * (size_t)(query_tokens > 0 ? query_tokens : 1));
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t n = 0; n < num_docs; ++n) {
      int64_t start = offsets[n], end = offsets[n + 1];
      if (start == end) {
        out[b * num_docs + n] = 0.0f;
        continue;
      }
      for (int64_t q = 0; q < query_tokens; ++q) {
        const int8_t* qrow = q8 + (b * query_tokens + q) * dim;
        float m = -INFINITY;
        for (int64_t t = start; t < end; ++t) {
          float sim = (float)idot(qrow, values + t * dim, dim);
          if (token_scale) sim = sim * token_scale[t];
          m = sim > m ? sim : m;
        }
        best[q] = m;
      }
      out[b * num_docs + n] =
          finish_int8q(best, qscale + b * query_tokens, query_tokens, scale, scratch);
    }
  }
  free(best);
  free(scratch);
}

void orc_int8_dots(const int8_t* q8, int64_t rows, int dim, const int8_t* values,
                   int64_t num_tokens, int32_t* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t t = 0; t < num_tokens; ++t)
      out[r * num_tokens + t] = idot(q8 + r * dim, values + t * dim, dim);
}

/* -------------------------------------------------------------- reducers */

static int cmp_desc_f32(const void* a, const void* b) {
  float x = *(const float*)a, y = *(const float*)b;
  return (x < y) - (x > y);
}

/* _api.py:558-585 on one [Q, T] similarity block (row-major). */
static float reduce_block(const float* sims, int64_t query_tokens, int64_t tokens, int reducer,
                          const float* weights, float temperature, float* pooled, float* work) {
  if (tokens == 0 || query_tokens == 0) return 0.0f;
  for (int64_t q = 0; q < query_tokens; ++q) {
    const float* row = sims + q * tokens;
    float m = row[0];
    for (int64_t t = 1; t < tokens; ++t) m = row[t] > m ? row[t] : m;
    switch (reducer) {
      case ORC_MAXSIM:
        pooled[q] = m;
        break;
      case ORC_WEIGHTED:
        pooled[q] = m * weights[q];
        break;
      case ORC_TOPK2:
      case ORC_TOPK4: {
        int64_t want = reducer == ORC_TOPK2 ? 2 : 4;
        int64_t count = want < tokens ? want : tokens;
        memcpy(work, row, sizeof(float) * (size_t)tokens);
        qsort(work, (size_t)tokens, sizeof(float), cmp_desc_f32);
        float s = 0.0f;
        for (int64_t i = 0; i < count; ++i) s += work[i];
        pooled[q] = s / (float)count;
        break;
      }
      case ORC_SMOOTHSIM: {
        for (int64_t t = 0; t < tokens; ++t) work[t] = expf((row[t] - m) / temperature);
        float se = orc_pairwise_sum_f32(work, tokens);
        pooled[q] = m + temperature * logf(se);
        break;
      }
      default:
        pooled[q] = 0.0f;
    }
  }
  return orc_pairwise_sum_f32(pooled, query_tokens);
}

void orc_dense_scores(const float* q, int64_t batch, int64_t query_tokens, int dim,
                      const float* docs, const int64_t* offsets, int64_t num_docs,
                      const int64_t* candidates, int64_t num_candidates,
                      int reducer, const float* weights, float temperature, float* out) {
  int64_t targets = candidates ? num_candidates : num_docs;
  int64_t max_len = 1;
  for (int64_t n = 0; n < num_docs; ++n)
    if (offsets[n + 1] - offsets[n] > max_len) max_len = offsets[n + 1] - offsets[n];
  int64_t qt = query_tokens > 0 ? query_tokens : 1;
  float* sims = (float*)malloc(sizeof(float) * (size_t)(qt * max_len));
  float* pooled = (float*)malloc(sizeof(float) * (size_t)qt);
  float* work = (float*)malloc(sizeof(float) * (size_t)max_len);
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t i = 0; i < targets; ++i) {
      int64_t n = candidates ? candidates[i] : i;
      int64_t start = offsets[n], len = offsets[n + 1] - start;
      for (int64_t qi = 0; qi < query_tokens; ++qi) {
        const float* qrow = q + (b * query_tokens + qi) * dim;
        for (int64_t t = 0; t < len; ++t) {
          const float* drow = docs + (start + t) * dim;
          double acc = 0.0;
          for (int d = 0; d < dim; ++d) acc += (double)qrow[d] * (double)drow[d];
          sims[qi * len + t] = (float)acc;
        }
      }
      out[b * targets + i] = reduce_block(sims, query_tokens, len, reducer,
                                          weights ? weights + b * query_tokens : NULL,
                                          temperature, pooled, work);
    }
  }
  free(sims);
  free(pooled);
  free(work);
}

/* experimental.py:403-420: dequantize values * f32(scale) [* token_scale]
 * in float32, then score densely. */
void orc_int4_fp32_scores(const float* q, int64_t batch, int64_t query_tokens, int dim,
                          const int8_t* values, float scale, const float* token_scale,
                          const int64_t* offsets, int64_t num_docs,
                          const int64_t* candidates, int64_t num_candidates,
                          int reducer, const float* weights, float temperature, float* out) {
  int64_t num_tokens = offsets[num_docs];
  float* docs = (float*)malloc(sizeof(float) * (size_t)(num_tokens * dim > 0 ? num_tokens * dim : 1));
  for (int64_t t = 0; t < num_tokens; ++t)
    for (int d = 0; d < dim; ++d) {
      float v = (float)values[t * dim + d] * scale;
      if (token_scale) v = v * token_scale[t];
      docs[t * dim + d] = v;
    }
  orc_dense_scores(q, batch, query_tokens, dim, docs, offsets, num_docs, candidates,
                   num_candidates, reducer, weights, temperature, out);
  free(docs);
}

/* ---------------------------------------------------------------- binary */

/* cpu_extension.cpp:59-80 (LUT build) and 82-126 (scan): per (q, byte) a
 * 256-entry float32 table of sequential +/-q sums, then per token the
 * sequential float32 sum of dim/8 lookups, max over tokens, sequential sum
 * over query tokens (empty docs contribute nothing), times scale. */
void orc_binary_lut_maxsim(const float* q, int64_t query_tokens, int dim,
                           const uint8_t* codes, const int64_t* offsets,
                           int64_t num_docs, float scale, float* out) {
  const int bytes = dim / 8;
  float* luts = (float*)malloc(sizeof(float) * (size_t)(query_tokens * bytes * 256 + 1));
  for (int64_t qi = 0; qi < query_tokens; ++qi)
    for (int bi = 0; bi < bytes; ++bi)
      for (int v = 0; v < 256; ++v) {
        float sum = 0.0f;
        for (int bit = 0; bit < 8; ++bit) {
          float sign = ((v >> bit) & 1) ? 1.0f : -1.0f;
          sum += sign * q[qi * dim + bi * 8 + bit];
        }
        luts[(qi * bytes + bi) * 256 + v] = sum;
      }
  for (int64_t n = 0; n < num_docs; ++n) {
    float doc_score = 0.0f;
    int64_t start = offsets[n], end = offsets[n + 1];
    for (int64_t qi = 0; qi < query_tokens; ++qi) {
      float best = -INFINITY;
      for (int64_t t = start; t < end; ++t) {
        float dot = 0.0f;
        for (int bi = 0; bi < bytes; ++bi) dot += luts[(qi * bytes + bi) * 256 + codes[t * bytes + bi]];
        best = dot > best ? dot : best;
      }
      if (start != end) doc_score += best;
    }
    out[n] = doc_score * scale;
  }
  free(luts);
}

static int popcount8(uint8_t x) { return __builtin_popcount((unsigned)x); }

void orc_binary_hamming_maxsim(const uint8_t* qbits, int64_t batch, int64_t query_tokens,
                               int dim, const uint8_t* codes, const int64_t* offsets,
                               int64_t num_docs, int32_t* out) {
  const int bytes = dim / 8;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t n = 0; n < num_docs; ++n) {
      int64_t start = offsets[n], end = offsets[n + 1];
      int32_t total = 0;
      if (start != end) {
        for (int64_t qi = 0; qi < query_tokens; ++qi) {
          const uint8_t* qrow = qbits + (b * query_tokens + qi) * bytes;
          int32_t best = -dim - 1;
          for (int64_t t = start; t < end; ++t) {
            int h = 0;
            for (int bi = 0; bi < bytes; ++bi) h += popcount8((uint8_t)(qrow[bi] ^ codes[t * bytes + bi]));
            int32_t sim = dim - 2 * h;
            best = sim > best ? sim : best;
          }
          total += best;
        }
      }
      out[b * num_docs + n] = total;
    }
}

/* ----------------------------------------------------------------- top-k */

typedef struct {
  float score;
  int64_t tie;
  int64_t pos;
} topk_entry;

static int cmp_topk(const void* a, const void* b) {
  const topk_entry* x = (const topk_entry*)a;
  const topk_entry* y = (const topk_entry*)b;
  if (x->score > y->score) return -1;
  if (x->score < y->score) return 1;
  if (x->tie < y->tie) return -1;
  if (x->tie > y->tie) return 1;
  return (x->pos > y->pos) - (x->pos < y->pos);
}

/* np.lexsort((ids, -scores))[:k] (_api.py:732-735); with tie_ids it is the
 * cascade's _stable_topk_indices(scores, k, tie_ids=...) (cascade.py:436-453).
 * out_indices are row positions. */
void orc_topk(const float* scores, int64_t batch, int64_t n, int64_t k,
              const int64_t* tie_ids, float* out_scores, int64_t* out_indices) {
  topk_entry* e = (topk_entry*)malloc(sizeof(topk_entry) * (size_t)(n > 0 ? n : 1));
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t i = 0; i < n; ++i) {
      e[i].score = scores[b * n + i];
      e[i].tie = tie_ids ? tie_ids[b * n + i] : i;
      e[i].pos = i;
    }
    qsort(e, (size_t)n, sizeof(topk_entry), cmp_topk);
    for (int64_t i = 0; i < k; ++i) {
      out_scores[b * k + i] = e[i].score;
      out_indices[b * k + i] = e[i].pos;
    }
  }
  free(e);
}

/* --------------------------------------------- binary prefix + int4 residual */

void orc_pack_binary_residual(const float* x, int64_t num_tokens, int dim,
                              uint8_t* sign_codes, float* prefix_scale,
                              uint8_t* residual_codes, int8_t* residual_values,
                              float* residual_scale) {
  double* absrow = (double*)malloc(sizeof(double) * (size_t)dim);
  float* resid = (float*)malloc(sizeof(float) * (size_t)dim);
  orc_pack_signs(x, num_tokens, dim, sign_codes);
  for (int64_t t = 0; t < num_tokens; ++t) {
    const float* row = x + t * dim;
    for (int d = 0; d < dim; ++d) absrow[d] = (double)fabsf(row[d]);
    float a = (float)(orc_pairwise_sum_f64(absrow, dim) / (double)dim);
    prefix_scale[t] = a;
    for (int d = 0; d < dim; ++d) resid[d] = row[d] - (row[d] >= 0.0f ? a : -a);
    orc_pack_int4_token(resid, 1, dim, residual_codes + t * (dim / 2),
                        residual_values ? residual_values + t * dim : NULL, residual_scale + t);
  }
  free(absrow);
  free(resid);
}

static int32_t sign_dot(const int8_t* q8, const uint8_t* bits, int dim) {
  int32_t acc = 0;
  for (int d = 0; d < dim; ++d) acc += ((bits[d / 8] >> (d % 8)) & 1) ? q8[d] : -q8[d];
  return acc;
}

void orc_binres_prefix_scores(const int8_t* q8, const float* qscale, int64_t batch,
                              int64_t query_tokens, int dim, const uint8_t* sign_codes,
                              const float* prefix_scale, const int64_t* offsets,
                              int64_t num_docs, float* out) {
  int64_t qt = query_tokens > 0 ? query_tokens : 1;
  float* best = (float*)malloc(sizeof(float) * (size_t)qt);
  double* scratch = (double*)malloc(sizeof(double) * (size_t)qt);
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t n = 0; n < num_docs; ++n) {
      int64_t start = offsets[n], end = offsets[n + 1];
      if (start == end) {
        out[b * num_docs + n] = 0.0f;
        continue;
      }
      for (int64_t qi = 0; qi < query_tokens; ++qi) {
        const int8_t* qrow = q8 + (b * query_tokens + qi) * dim;
        float m = -INFINITY;
        for (int64_t t = start; t < end; ++t) {
          float sim = prefix_scale[t] * (float)sign_dot(qrow, sign_codes + t * (dim / 8), dim);
          m = sim > m ? sim : m;
        }
        best[qi] = m;
      }
      out[b * num_docs + n] = finish_int8q(best, qscale + b * query_tokens, query_tokens, 1.0, scratch);
    }
  free(best);
  free(scratch);
}

void orc_binres_fused_scores(const int8_t* q8, const float* qscale, int64_t batch,
                             int64_t query_tokens, int dim, const uint8_t* sign_codes,
                             const float* prefix_scale, const int8_t* residual_values,
                             const float* residual_scale, const int64_t* offsets,
                             int64_t num_docs, const int64_t* candidates,
                             int64_t num_candidates, float* out) {
  int64_t qt = query_tokens > 0 ? query_tokens : 1;
  int64_t targets = candidates ? num_candidates : num_docs;
  float* best = (float*)malloc(sizeof(float) * (size_t)qt);
  double* scratch = (double*)malloc(sizeof(double) * (size_t)qt);
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t i = 0; i < targets; ++i) {
      int64_t n = candidates ? candidates[b * num_candidates + i] : i;
      int64_t start = offsets[n], end = offsets[n + 1];
      if (start == end) {
        out[b * targets + i] = 0.0f;
        continue;
      }
      for (int64_t qi = 0; qi < query_tokens; ++qi) {
        const int8_t* qrow = q8 + (b * query_tokens + qi) * dim;
        float m = -INFINITY;
        for (int64_t t = start; t < end; ++t) {
          float ps = prefix_scale[t] * (float)sign_dot(qrow, sign_codes + t * (dim / 8), dim);
          float rs = residual_scale[t] * (float)idot(qrow, residual_values + t * dim, dim);
          float sim = ps + rs;
          m = sim > m ? sim : m;
        }
        best[qi] = m;
      }
      out[b * targets + i] = finish_int8q(best, qscale + b * query_tokens, query_tokens, 1.0, scratch);
    }
  free(best);
  free(scratch);
}
