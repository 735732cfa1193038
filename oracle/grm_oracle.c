/*
 * grm_oracle.c -- CPU restatement of the GRM graft-route laws.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP route
 * library is compared against; it is never linked into, loaded by, or
 * called from the product path (graftrepository_amd/).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
 *
 * Every law below restates the reference's CPU router (file:line citations
 * are into DragonShadows1978/GraftRepository):
 *
 *   tie law          cpp/grm_runtime.cpp:75-82   score_node_better:
 *                    score DESC, node_id ASC; non-finite scores never ranked
 *                    (cpp/grm_runtime.cpp:4332-4335, 4353-4355).
 *   MLA row norm     cpp/grm_runtime.cpp:3232-3241  norm = float(sqrt(sum
 *                    (double)v*(double)v)) accumulated sequentially.
 *   MLA query norm   cpp/grm_runtime.cpp:4310-4314  qnorm = sqrt(sum (double)q^2)
 *   MLA score        cpp/grm_runtime.cpp:3518-3545  exact_mla_entry_score:
 *                    float(dot / (qnorm * (double)norm + 1e-8)), dot in fp64,
 *                    sequential over d.
 *   MLA route        cpp/grm_runtime.cpp:4299-4361  route_mla_arena (no
 *                    lexical keys, no filters): score every entry, drop
 *                    non-finite, order by the tie law, keep topk.
 *   GQA score        cpp/grm_runtime.cpp:2980-3029  gqa_raw_score: mean over
 *                    query heads h of max over (query token, key token) of
 *                    |q.k| / sqrt(head_dim), dot and mean in fp64; any
 *                    non-finite query/key value makes the score NaN; zero
 *                    key tokens give 0.0.
 *   GQA route        cpp/grm_runtime.cpp:4498-4881  route_gqa_raw without
 *                    lexical keys: raw scores ordered by the tie law.
 *   INT8 dequant     core/graft_quant.py:136-144  fp16(float(code) * float(scale))
 *
 * All fp64 sums run in the reference's sequential order so that the
 * float-rounded scores are bit-identical to the reference C++.  Build with
 * -ffp-contract=off (the Makefile does): a fused multiply-add would change
 * the rounding of `qnorm * norm + 1e-8`.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define GRM_ORACLE_EXPORT __attribute__((visibility("default")))

enum {
  GRM_ORACLE_F32 = 0,
  GRM_ORACLE_BF16 = 1,
  GRM_ORACLE_F16 = 2,
  GRM_ORACLE_I8 = 3,
};

/* ------------------------------------------------------------ fp16/bf16 */

/* IEEE binary16 -> binary32 (exact). */
static float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      /* subnormal: value = man * 2^-24 */
      float v = (float)man * 5.9604644775390625e-08f;
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

/* binary32 -> binary16, round to nearest even, with subnormals, overflow to
 * infinity and NaN preserved as a quiet NaN. */
static uint16_t float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {                 /* inf or nan */
    return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  }
  if (ax >= 0x477ff000u) {                 /* rounds to >= 65520: overflow */
    return (uint16_t)(sign | 0x7c00u);
  }
  if (ax < 0x38800000u) {                  /* below 2^-14: subnormal or zero */
    /* value = ax_float; subnormal half step is 2^-24.  Shift the 24-bit
     * significand (with implicit bit) right and round to nearest even. */
    if (ax < 0x33000000u) {                /* < 2^-25: rounds to zero */
      return sign;
    }
    const uint32_t e = ax >> 23;           /* biased f32 exponent, 102..112 */
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;       /* 14..24 */
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) {
      q += 1u;
    }
    return (uint16_t)(sign | q);
  }
  /* normal range: rebias exponent, round the 13 dropped mantissa bits. */
  uint32_t h = ((ax >> 13) - (112u << 10));
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
    h += 1u;                               /* may carry into the exponent */
  }
  return (uint16_t)(sign | h);
}

static float bf16_to_float(uint16_t b) {
  const uint32_t bits = (uint32_t)b << 16;
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

GRM_ORACLE_EXPORT void grm_oracle_f16_from_f32(const float* in, uint64_t n,
                                               uint16_t* out) {
  for (uint64_t i = 0; i < n; ++i) {
    out[i] = float_to_half(in[i]);
  }
}

GRM_ORACLE_EXPORT void grm_oracle_f32_from_f16(const uint16_t* in, uint64_t n,
                                               float* out) {
  for (uint64_t i = 0; i < n; ++i) {
    out[i] = half_to_float(in[i]);
  }
}

/* INT8 dequant law, core/graft_quant.py:136-144:
 * (codes.astype(f32) * scale.astype(f32)).astype(f16), read back as f32. */
static float dequant_i8(int8_t code, float scale) {
  return half_to_float(float_to_half((float)code * scale));
}

/* --------------------------------------------------------------- top-k */

typedef struct {
  float score;
  uint64_t id;
} scored_t;

/* score_node_better, cpp/grm_runtime.cpp:75-82. */
static int better(float s, uint64_t id, float ts, uint64_t tid) {
  if (s != ts) {
    return s > ts;
  }
  return id < tid;
}

/* Insert into a sorted list of `k` entries (best first); `*count` valid. */
static void topk_insert(scored_t* list, uint64_t* count, uint64_t k,
                        float s, uint64_t id) {
  if (k == 0) {
    return;
  }
  if (*count == k && !better(s, id, list[k - 1].score, list[k - 1].id)) {
    return;
  }
  uint64_t pos = (*count < k) ? *count : k - 1;
  while (pos > 0 && better(s, id, list[pos - 1].score, list[pos - 1].id)) {
    list[pos] = list[pos - 1];
    --pos;
  }
  list[pos].score = s;
  list[pos].id = id;
  if (*count < k) {
    *count += 1;
  }
}

/* Select the best `topk` finite scores; unfilled slots get UINT64_MAX / NaN
 * (the reference CUDA sidecar's sentinel, scripts/grm_mla_cuda_probe.py:175-178). */
static void select_topk(const float* scores, const uint64_t* node_ids,
                        const uint8_t* live, uint64_t n, uint64_t topk,
                        uint64_t* out_ids, float* out_scores,
                        uint64_t* out_count) {
  scored_t* list = (scored_t*)malloc(sizeof(scored_t) * (topk ? topk : 1));
  uint64_t count = 0;
  for (uint64_t i = 0; i < n; ++i) {
    if (live && !live[i]) {
      continue;
    }
    const float s = scores[i];
    if (!isfinite(s)) {
      continue;
    }
    topk_insert(list, &count, topk, s, node_ids ? node_ids[i] : i);
  }
  for (uint64_t j = 0; j < topk; ++j) {
    if (j < count) {
      out_ids[j] = list[j].id;
      if (out_scores) out_scores[j] = list[j].score;
    } else {
      out_ids[j] = UINT64_MAX;
      if (out_scores) out_scores[j] = NAN;
    }
  }
  if (out_count) *out_count = count;
  free(list);
}

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) {
    omp_set_num_threads(threads);
  }
#else
  (void)threads;
#endif
}

/* ----------------------------------------------------------------- MLA */

/* cpp/grm_runtime.cpp:3232-3241 (rebuild_mla_arena): norm per row. */
GRM_ORACLE_EXPORT void grm_oracle_mla_row_norms(const float* rows, uint64_t n,
                                                uint64_t dim, float* out,
                                                int threads) {
  set_threads(threads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)n; ++i) {
    const float* r = rows + (uint64_t)i * dim;
    double acc = 0.0;
    for (uint64_t d = 0; d < dim; ++d) {
      acc += (double)r[d] * (double)r[d];
    }
    out[i] = (float)sqrt(acc);
  }
}

/* cpp/grm_runtime.cpp:4310-4314: query norm in fp64. */
GRM_ORACLE_EXPORT double grm_oracle_mla_qnorm(const float* q, uint64_t dim) {
  double acc = 0.0;
  for (uint64_t d = 0; d < dim; ++d) {
    acc += (double)q[d] * (double)q[d];
  }
  return sqrt(acc);
}

/* cpp/grm_runtime.cpp:3531-3537 (exact_mla_entry_score, one row). */
static float mla_row_score(const float* q, double qnorm, const float* row,
                           float norm, uint64_t dim) {
  double dot = 0.0;
  for (uint64_t d = 0; d < dim; ++d) {
    dot += (double)q[d] * (double)row[d];
  }
  return (float)(dot / ((qnorm * (double)norm) + 1.0e-8));
}

/* Score every row for every query (fp64 law); scores [q_count][n]. */
GRM_ORACLE_EXPORT void grm_oracle_mla_scores(const float* rows, uint64_t n,
                                             uint64_t dim, const float* norms,
                                             const float* queries,
                                             uint64_t q_count, float* scores,
                                             int threads) {
  set_threads(threads);
  for (uint64_t qi = 0; qi < q_count; ++qi) {
    const float* q = queries + qi * dim;
    const double qnorm = grm_oracle_mla_qnorm(q, dim);
    float* out = scores + qi * n;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) {
      out[i] = mla_row_score(q, qnorm, rows + (uint64_t)i * dim, norms[i], dim);
    }
  }
}

/* route_mla_arena without lexical/filters, cpp/grm_runtime.cpp:4299-4361.
 * node_ids may be NULL (row index is the id); live may be NULL (all live).
 * out_ids / out_scores are [q_count][topk]; out_counts is [q_count]. */
GRM_ORACLE_EXPORT int grm_oracle_mla_route(const float* rows, uint64_t n,
                                           uint64_t dim,
                                           const uint64_t* node_ids,
                                           const uint8_t* live,
                                           const float* queries,
                                           uint64_t q_count, uint64_t topk,
                                           int threads, uint64_t* out_ids,
                                           float* out_scores,
                                           uint64_t* out_counts) {
  if (!rows || !queries || !out_ids || dim == 0 || topk == 0) {
    return -1;
  }
  float* norms = (float*)malloc(sizeof(float) * (n ? n : 1));
  float* scores = (float*)malloc(sizeof(float) * (n ? n : 1));
  if (!norms || !scores) {
    free(norms);
    free(scores);
    return -2;
  }
  grm_oracle_mla_row_norms(rows, n, dim, norms, threads);
  for (uint64_t qi = 0; qi < q_count; ++qi) {
    grm_oracle_mla_scores(rows, n, dim, norms, queries + qi * dim, 1, scores,
                          threads);
    select_topk(scores, node_ids, live, n, topk, out_ids + qi * topk,
                out_scores ? out_scores + qi * topk : NULL,
                out_counts ? out_counts + qi : NULL);
  }
  free(norms);
  free(scores);
  return 0;
}

/* The per-call part of route_mla_arena (cpp/grm_runtime.cpp:4299-4361):
 * the arena build computes the row norms once (:3232-3241), so a route
 * reads them; `norms` holds grm_oracle_mla_row_norms' output.  Used to time
 * the CPU baseline at the reference's per-call cost. */
GRM_ORACLE_EXPORT int grm_oracle_mla_route_normed(
    const float* rows, uint64_t n, uint64_t dim, const float* norms,
    const float* queries, uint64_t q_count, uint64_t topk, int threads,
    uint64_t* out_ids, float* out_scores, uint64_t* out_counts) {
  if (!rows || !norms || !queries || !out_ids || dim == 0 || topk == 0) {
    return -1;
  }
  float* scores = (float*)malloc(sizeof(float) * (n ? n : 1));
  if (!scores) {
    return -2;
  }
  for (uint64_t qi = 0; qi < q_count; ++qi) {
    grm_oracle_mla_scores(rows, n, dim, norms, queries + qi * dim, 1, scores,
                          threads);
    select_topk(scores, NULL, NULL, n, topk, out_ids + qi * topk,
                out_scores ? out_scores + qi * topk : NULL,
                out_counts ? out_counts + qi : NULL);
  }
  free(scores);
  return 0;
}

/* ----------------------------------------------------------------- GQA */

/* cpp/grm_runtime.cpp:2980-3029 (gqa_raw_score) over f32 values.
 * q: [H][Qt][hd]; key: [KV][L][hd]. */
static float gqa_raw_score(const float* q, uint64_t H, uint64_t Qt,
                           uint64_t hd, const float* key, uint64_t KV,
                           uint64_t L) {
  if (H == 0 || Qt == 0 || hd == 0 || KV == 0 || H % KV != 0) {
    return 0.0f;
  }
  if (L == 0) {
    return 0.0f;
  }
  const uint64_t repeat = H / KV;
  const double denom = sqrt((double)hd);
  double total = 0.0;
  for (uint64_t h = 0; h < H; ++h) {
    const uint64_t kh = h / repeat;
    double best = 0.0;
    for (uint64_t qi = 0; qi < Qt; ++qi) {
      const float* qrow = q + (h * Qt + qi) * hd;
      for (uint64_t ki = 0; ki < L; ++ki) {
        const float* krow = key + (kh * L + ki) * hd;
        double dot = 0.0;
        for (uint64_t d = 0; d < hd; ++d) {
          const float qv = qrow[d];
          const float kv = krow[d];
          if (!isfinite(qv) || !isfinite(kv)) {
            return NAN;
          }
          dot += (double)qv * (double)kv;
        }
        const double v = fabs(dot) / denom;
        if (best < v) {            /* std::max(best, v) */
          best = v;
        }
      }
    }
    total += best;
  }
  return (float)(total / (double)H);
}

/* Decode one node's key block [KV][L][hd] to f32 by the storage law. */
static void gqa_decode_node(const void* keys, int key_dtype,
                            const void* scales, int scale_dtype,
                            uint64_t group_size, uint64_t tok_off, uint64_t L,
                            uint64_t KV, uint64_t hd, float* out) {
  const uint64_t count = KV * L * hd;
  const uint64_t base = tok_off * KV * hd;
  switch (key_dtype) {
    case GRM_ORACLE_F32:
      memcpy(out, (const float*)keys + base, count * sizeof(float));
      break;
    case GRM_ORACLE_BF16: {
      const uint16_t* src = (const uint16_t*)keys + base;
      for (uint64_t i = 0; i < count; ++i) out[i] = bf16_to_float(src[i]);
      break;
    }
    case GRM_ORACLE_F16: {
      const uint16_t* src = (const uint16_t*)keys + base;
      for (uint64_t i = 0; i < count; ++i) out[i] = half_to_float(src[i]);
      break;
    }
    case GRM_ORACLE_I8: {
      const int8_t* src = (const int8_t*)keys + base;
      const uint64_t groups = hd / group_size;
      const uint64_t sbase = tok_off * KV * groups;
      for (uint64_t i = 0; i < count; ++i) {
        const uint64_t row = i / hd;
        const uint64_t g = (i % hd) / group_size;
        const uint64_t si = sbase + row * groups + g;
        const float s = scale_dtype == GRM_ORACLE_F16
                            ? half_to_float(((const uint16_t*)scales)[si])
                            : ((const float*)scales)[si];
        out[i] = dequant_i8(src[i], s);
      }
      break;
    }
    default:
      break;
  }
}

/* Exact GQA scores for every node and query: scores [q_count][n].
 * keys: CSR token-major per node, node i's block [KV][L_i][hd] starts at
 * value offset tok_offsets[i] * KV * hd.  queries: [q_count][H][Qt][hd]. */
GRM_ORACLE_EXPORT int grm_oracle_gqa_scores(
    const void* keys, int key_dtype, const void* scales, int scale_dtype,
    uint64_t group_size, const uint64_t* tok_offsets, uint64_t n, uint64_t KV,
    uint64_t hd, const float* queries, uint64_t q_count, uint64_t H,
    uint64_t Qt, float* scores, int threads) {
  if (!keys || !tok_offsets || !queries || !scores || hd == 0 || KV == 0) {
    return -1;
  }
  if (key_dtype == GRM_ORACLE_I8 &&
      (!scales || group_size == 0 || hd % group_size != 0)) {
    return -1;
  }
  uint64_t max_l = 0;
  for (uint64_t i = 0; i < n; ++i) {
    const uint64_t L = tok_offsets[i + 1] - tok_offsets[i];
    if (L > max_l) max_l = L;
  }
  set_threads(threads);
  int rc = 0;
#pragma omp parallel
  {
    float* buf = (float*)malloc(sizeof(float) * (KV * max_l * hd + 1));
    if (!buf) {
#pragma omp atomic write
      rc = -2;
    } else {
#pragma omp for schedule(dynamic, 4)
      for (int64_t i = 0; i < (int64_t)n; ++i) {
        const uint64_t off = tok_offsets[i];
        const uint64_t L = tok_offsets[i + 1] - off;
        gqa_decode_node(keys, key_dtype, scales, scale_dtype, group_size, off,
                        L, KV, hd, buf);
        for (uint64_t qi = 0; qi < q_count; ++qi) {
          scores[qi * n + (uint64_t)i] = gqa_raw_score(
              queries + qi * H * Qt * hd, H, Qt, hd, buf, KV, L);
        }
      }
      free(buf);
    }
  }
  return rc;
}

/* route_gqa_raw without lexical keys, cpp/grm_runtime.cpp:4498-4881 (the
 * scores follow gqa_raw_score; see the header). */
GRM_ORACLE_EXPORT int grm_oracle_gqa_route(
    const void* keys, int key_dtype, const void* scales, int scale_dtype,
    uint64_t group_size, const uint64_t* tok_offsets, uint64_t n, uint64_t KV,
    uint64_t hd, const uint64_t* node_ids, const uint8_t* live,
    const float* queries, uint64_t q_count, uint64_t H, uint64_t Qt,
    uint64_t topk, int threads, uint64_t* out_ids, float* out_scores,
    uint64_t* out_counts) {
  if (!out_ids || topk == 0) {
    return -1;
  }
  float* scores = (float*)malloc(sizeof(float) * (n * q_count + 1));
  if (!scores) {
    return -2;
  }
  int rc = grm_oracle_gqa_scores(keys, key_dtype, scales, scale_dtype,
                                 group_size, tok_offsets, n, KV, hd, queries,
                                 q_count, H, Qt, scores, threads);
  if (rc == 0) {
    for (uint64_t qi = 0; qi < q_count; ++qi) {
      select_topk(scores + qi * n, node_ids, live, n, topk,
                  out_ids + qi * topk,
                  out_scores ? out_scores + qi * topk : NULL,
                  out_counts ? out_counts + qi : NULL);
    }
  }
  free(scores);
  return rc;
}

/* Top-k selection alone (for tests of the tie law on given score vectors). */
GRM_ORACLE_EXPORT void grm_oracle_select_topk(const float* scores,
                                              const uint64_t* node_ids,
                                              const uint8_t* live, uint64_t n,
                                              uint64_t topk, uint64_t* out_ids,
                                              float* out_scores,
                                              uint64_t* out_count) {
  select_topk(scores, node_ids, live, n, topk, out_ids, out_scores, out_count);
}
