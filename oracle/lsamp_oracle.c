/*
 * lsamp_oracle.c — CPU restatement of the reference's logits-to-token stage.
 *
 * TEST INFRASTRUCTURE ONLY (see lsamp_oracle.h): loaded by tests/, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg
 * as the timed CPU baseline.  The shipped library never links it.
 *
 * The code follows the reference op sequence stage by stage: dense [V]
 * intermediates per row, a full sort per row for the filters, sequential fp32
 * cumulative sums.  Citations are to files under the reference repository.
 *
 * Parity status of each function (what pins it) is listed in the test files;
 * the functions whose exact fp32 rounding depends on MLX internals that are not
 * vendored (softmax / logsumexp reduction order, argPartition tie choice) are
 * pinned only up to the documented boundary tolerance.
 *
 * Build: gcc -O3 -march=native -ffp-contract=off -fno-fast-math -fPIC -shared
 * (contraction must stay off: the reference evaluates x - f*c - p*[c>0] as
 * separately rounded ops, and the fixed-point draw needs every fp32 op rounded
 * exactly as written).
 */
#include "lsamp_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ dtypes */

static inline float bits_f32(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}
static inline uint32_t f32_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

float lso_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* Round-to-nearest-even float -> bfloat16 (NaN stays a quiet NaN). */
uint16_t lso_f32_to_bf16(float f) {
  uint32_t b = f32_bits(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40u);
  uint32_t bias = 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)((b + bias) >> 16);
}

float lso_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);
    /* subnormal half: man * 2^-24 is exact in float */
    float v = (float)man * 5.9604644775390625e-08f;
    return (sign ? -v : v);
  }
  if (exp == 31) return bits_f32(sign | 0x7f800000u | (man << 13));
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* Round-to-nearest-even float -> IEEE half. */
uint16_t lso_f32_to_f16(float f) {
  uint32_t b = f32_bits(f);
  uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
  uint32_t a = b & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  if (a < 0x38800000u) {                                   /* half subnormal */
    float v = bits_f32(a);
    /* v * 2^24 rounded to nearest even integer */
    float s = v * 16777216.0f;
    float r = rintf(s);
    return (uint16_t)(sign | (uint16_t)r);
  }
  uint32_t exp = (a >> 23) - 112u;
  uint32_t man = a & 0x7fffffu;
  uint32_t h = (exp << 10) | (man >> 13);
  uint32_t rest = man & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

/* Array forms of the converters, for the known-answer tests. */
void lso_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = lso_f32_to_bf16(in[i]);
}
void lso_f32_to_f16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = lso_f32_to_f16(in[i]);
}
void lso_f16_to_f32_n(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = lso_f16_to_f32(in[i]);
}

static inline float load_logit(const void* row, int32_t dtype, int64_t i) {
  switch (dtype) {
    case LSAMP_DTYPE_BF16: return lso_bf16_to_f32(((const uint16_t*)row)[i]);
    case LSAMP_DTYPE_F16: return lso_f16_to_f32(((const uint16_t*)row)[i]);
    default: return ((const float*)row)[i];
  }
}

/* The value an MLX array of `dtype` holds after an op computed in float. */
static inline float round_dtype(float v, int32_t dtype) {
  switch (dtype) {
    case LSAMP_DTYPE_BF16: return lso_bf16_to_f32(lso_f32_to_bf16(v));
    case LSAMP_DTYPE_F16: return lso_f16_to_f32(lso_f32_to_f16(v));
    default: return v;
  }
}

/* ----------------------------------------------------- deterministic math */

/* dexp: e^d for d <= 0 in a fixed sequence of IEEE fp32 operations, so host
 * and device agree bit for bit.  Cody & Waite (1980) range reduction
 * d = n ln2 + r with a two-part ln2, then the Taylor polynomial of e^r to
 * degree 7 (|r| <= ln2/2, truncation < 3e-9) in Horner form with fma, then an
 * exact scaling by 2^n.  Inputs at or below -80 (weights < 2^-115) give 0. */
float lso_dexp(float d) {
  if (!(d > -80.0f)) return 0.0f;
  if (d > 0.0f) d = 0.0f;
  float n = rintf(d * 1.44269504088896341f);
  float r = fmaf(-n, 0.693145751953125f, d);
  r = fmaf(-n, 1.428606765330187e-06f, r);
  float p = 1.984126984e-04f; /* 1/7! */
  p = fmaf(p, r, 1.388888889e-03f); /* 1/6! */
  p = fmaf(p, r, 8.333333333e-03f); /* 1/5! */
  p = fmaf(p, r, 4.166666667e-02f); /* 1/4! */
  p = fmaf(p, r, 1.666666667e-01f); /* 1/3! */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int32_t ni = (int32_t)n;
  return p * bits_f32((uint32_t)(ni + 127) << 23);
}

/* Fixed-point draw weight of a kept token: 2^40 * dexp(fl(fl(y - y_max)*scale)). */
uint64_t lso_weight(float y, float y_max, float scale) {
  if (!(y > -INFINITY)) return 0;
  float d;
  if (y == y_max) {
    d = 0.0f;
  } else {
    float diff = y - y_max;
    d = diff * scale;
  }
  float e = lso_dexp(d);
  return (uint64_t)(e * 1099511627776.0f);
}

static inline uint32_t uniform_u32(float u) {
  if (!(u > 0.0f)) return 0u;
  if (u >= 1.0f) return 0xffffffffu;
  return (uint32_t)(u * 4294967296.0f);
}

/* (U * W) >> 32 without 128-bit arithmetic. */
static inline uint64_t scaled_target(uint32_t U, uint64_t W) {
  uint64_t hi = W >> 32, lo = W & 0xffffffffull;
  return (uint64_t)U * hi + (((uint64_t)U * lo) >> 32);
}

/* Inverse-CDF draw over kept tokens in token-id order (the library's draw
 * rule; the reference's own draw is MLX's Gumbel race, Evaluate.swift:456,508
 * and SamplerV2.swift:101-106, whose random stream cannot be reproduced here). */
int32_t lso_draw(int32_t n, const float* y, const uint8_t* keep, float scale, float u,
                 uint64_t* total_out) {
  float y_max = -INFINITY;
  for (int32_t i = 0; i < n; ++i)
    if (keep[i] && y[i] > y_max) y_max = y[i];
  uint64_t W = 0;
  for (int32_t i = 0; i < n; ++i)
    if (keep[i]) W += lso_weight(y[i], y_max, scale);
  if (total_out) *total_out = W;
  if (W == 0) return -1;
  uint64_t target = scaled_target(uniform_u32(u), W);
  uint64_t cum = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (!keep[i]) continue;
    cum += lso_weight(y[i], y_max, scale);
    if (cum > target) return i;
  }
  return -1; /* unreachable: target < W */
}

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11). */
void lso_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
  uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
  uint32_t k0 = key_in[0], k1 = key_in[1];
  for (int round = 0; round < 10; ++round) {
    if (round > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    uint32_t n0 = hi1 ^ c1 ^ k0;
    uint32_t n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

/* SamplerV2.mix (SamplerV2.swift:183-191). */
static inline uint64_t splitmix64(uint64_t v) {
  uint64_t z = v + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
uint64_t lso_rng_key(uint64_t seed, uint64_t id, uint64_t step) {
  return splitmix64(splitmix64(splitmix64(seed) ^ id) ^ step);
}

float lso_rng_uniform(uint64_t key, uint32_t purpose) {
  uint32_t ctr[4] = {purpose, 0u, 0u, 0u};
  uint32_t k[2] = {(uint32_t)key, (uint32_t)(key >> 32)};
  uint32_t out[4];
  lso_philox4x32_10(ctr, k, out);
  return (float)(out[0] >> 8) * 5.9604644775390625e-08f;
}

/* ------------------------------------------------------------ mask apply */

/* xgrammar ApplyMask32Bits / ApplyMask16Bits (grammar_matcher.cc:89-171) and
 * bitmaskToMLXArray (GuidedGenerationLoop.swift:595-610): bit i of word i/32,
 * LSB first; 0 = forbidden.  Past mask_bits the tail policy decides. */
static inline int mask_allows(const uint32_t* mrow, int32_t mask_words, int32_t mask_bits,
                              int32_t tail, int32_t i) {
  if (!mrow) return 1;
  if (i >= mask_bits || (i >> 5) >= mask_words) return tail == LSAMP_MASK_TAIL_KEEP;
  return (int)((mrow[i >> 5] >> (i & 31)) & 1u);
}

/* ------------------------------------------------------------ sort helpers */

typedef struct {
  float v;
  int32_t i;
} vi_t;

/* value descending, id ascending: MLX argSort(-x) on a stable sort
 * (LogitsPipelineV2.swift:426); the reference's tie order is unvendored, the
 * library adopts "equal values: lower id first". */
static int cmp_desc_idasc(const void* a, const void* b) {
  const vi_t* x = (const vi_t*)a;
  const vi_t* y = (const vi_t*)b;
  if (x->v > y->v) return -1;
  if (x->v < y->v) return 1;
  return (x->i > y->i) - (x->i < y->i);
}

/* value ascending, id ascending: a stable ascending argSort
 * (Evaluate.swift:463). */
static int cmp_asc_idasc(const void* a, const void* b) {
  const vi_t* x = (const vi_t*)a;
  const vi_t* y = (const vi_t*)b;
  if (x->v < y->v) return -1;
  if (x->v > y->v) return 1;
  return (x->i > y->i) - (x->i < y->i);
}

/* ------------------------------------------------------------ row scratch */

typedef struct {
  int32_t V;
  float* x;       /* processed logits                           */
  float* y;       /* filter-space / sampling logits             */
  float* dense_a; /* dense count tensor                         */
  float* dense_b; /* dense bias / presence tensor               */
  uint8_t* keep;
  vi_t* order;
  float* cum;
} scratch_t;

static int scratch_init(scratch_t* s, int32_t V) {
  s->V = V;
  s->x = (float*)malloc(sizeof(float) * (size_t)V);
  s->y = (float*)malloc(sizeof(float) * (size_t)V);
  s->dense_a = (float*)malloc(sizeof(float) * (size_t)V);
  s->dense_b = (float*)malloc(sizeof(float) * (size_t)V);
  s->keep = (uint8_t*)malloc((size_t)V);
  s->order = (vi_t*)malloc(sizeof(vi_t) * (size_t)V);
  s->cum = (float*)malloc(sizeof(float) * (size_t)V);
  return s->x && s->y && s->dense_a && s->dense_b && s->keep && s->order && s->cum;
}
static void scratch_free(scratch_t* s) {
  free(s->x);
  free(s->y);
  free(s->dense_a);
  free(s->dense_b);
  free(s->keep);
  free(s->order);
  free(s->cum);
}

/* SuppressTokensProcessor.process (SuppressTokens.swift:67-81): putAlong of
 * -inf at the suppressed ids, ids at or past the vocabulary dropped (the
 * reference's slow path), negative ids dropped at init (:55-56). */
static void suppress_apply(const lso_sample_args* a, float* x) {
  for (int32_t j = 0; j < a->n_suppress; ++j) {
    const int32_t id = a->suppress_ids[j];
    if (id >= 0 && id < a->vocab) x[id] = -INFINITY;
  }
}

/* ------------------------------------------------------- CBv2 transforms */

/* LogitsPipelineV2.process stages (0)-(3) plus the hard mask
 * (LogitsPipelineV2.swift:303-344), on dense per-row tensors built the way
 * setRows builds them (:240-261): `dense_a` = output counts, `dense_b` =
 * window presence / bias. */
static void cbv2_transform(const lso_sample_args* a, int32_t r, scratch_t* s) {
  const int32_t V = a->vocab;
  const lsamp_row_params* p = &a->params[r];
  const void* raw = (const char*)a->logits +
                    (size_t)r * (size_t)a->row_stride * (a->dtype == LSAMP_DTYPE_F32 ? 4 : 2);
  float* x = s->x;
  /* (0) cast to float32 (:303) */
  for (int32_t i = 0; i < V; ++i) x[i] = load_logit(raw, a->dtype, i);

  int32_t e0 = 0, e1 = 0;
  if (a->penalty_row_ptr && a->penalty_entries) {
    e0 = a->penalty_row_ptr[r];
    e1 = a->penalty_row_ptr[r + 1];
  }
  const lsamp_penalty_entry* ent = a->penalty_entries;

  /* (1) logit bias (:317-319): dense bias matrix row */
  int any_bias = 0;
  for (int32_t e = e0; e < e1; ++e)
    if (ent[e].bias != 0.0f) any_bias = 1;
  if (any_bias) {
    memset(s->dense_b, 0, sizeof(float) * (size_t)V);
    for (int32_t e = e0; e < e1; ++e) s->dense_b[ent[e].token] = ent[e].bias;
    for (int32_t i = 0; i < V; ++i) x[i] = x[i] + s->dense_b[i];
  }
  /* (2a) repetition over the window counts (:322-326) */
  if (p->repetition_penalty != 1.0f) {
    memset(s->dense_b, 0, sizeof(float) * (size_t)V);
    int any = 0;
    for (int32_t e = e0; e < e1; ++e)
      if (ent[e].flags & LSAMP_PEN_REPETITION) {
        s->dense_b[ent[e].token] = 1.0f;
        any = 1;
      }
    if (any) {
      const float rp = p->repetition_penalty;
      for (int32_t i = 0; i < V; ++i) {
        if (s->dense_b[i] > 0.0f) {
          float v = x[i];
          x[i] = v > 0.0f ? v / rp : v * rp;
        }
      }
    }
  }
  /* (2b) frequency then presence over output counts (:327-330) */
  if (p->frequency_penalty != 0.0f || p->presence_penalty != 0.0f) {
    memset(s->dense_a, 0, sizeof(float) * (size_t)V);
    for (int32_t e = e0; e < e1; ++e) s->dense_a[ent[e].token] = (float)ent[e].count;
    const float f = p->frequency_penalty, pr = p->presence_penalty;
    for (int32_t i = 0; i < V; ++i) {
      float fc = f * s->dense_a[i];
      x[i] = x[i] - fc;
      float pm = pr * (s->dense_a[i] > 0.0f ? 1.0f : 0.0f);
      x[i] = x[i] - pm;
    }
  }
  /* (3) temperature (:333-335); greedy rows are pinned to 1.0 (:171,193) */
  if (p->kind != LSAMP_KIND_ARGMAX && p->temperature != 1.0f) {
    const float t = p->temperature;
    for (int32_t i = 0; i < V; ++i) x[i] = x[i] / t;
  }
  /* hard mask after the arithmetic transforms (:337-344,
   * TokenConstraintSamplerV2.swift:177-179) */
  if (a->bitmask) {
    const uint32_t* mrow = a->bitmask + (size_t)r * (size_t)a->mask_words;
    for (int32_t i = 0; i < V; ++i)
      if (!mask_allows(mrow, a->mask_words, a->mask_bits, a->mask_tail, i)) x[i] = -INFINITY;
  }
  suppress_apply(a, x);
}

/* ------------------------------------------------------ mlx-lm transforms */

/* PenaltyProcessor.process (Evaluate.swift:687-693) followed by the custom
 * (grammar) and suppress processors (GenerationComponents.swift:112-141,
 * SuppressTokens.swift:67-81), which both reduce to -inf at masked ids.
 * RepetitionContext / PresencePenaltyContext compute in the logits dtype with
 * the Float penalty converted to that dtype; FrequencyPenaltyContext's float32
 * histogram promotes the row to float32. */
static void mlxlm_transform(const lso_sample_args* a, int32_t r, scratch_t* s) {
  const int32_t V = a->vocab;
  const lsamp_row_params* p = &a->params[r];
  const int32_t dt = a->dtype;
  const void* raw = (const char*)a->logits +
                    (size_t)r * (size_t)a->row_stride * (dt == LSAMP_DTYPE_F32 ? 4 : 2);
  float* x = s->x;
  for (int32_t i = 0; i < V; ++i) x[i] = load_logit(raw, dt, i);

  int32_t e0 = 0, e1 = 0;
  if (a->penalty_row_ptr && a->penalty_entries) {
    e0 = a->penalty_row_ptr[r];
    e1 = a->penalty_row_ptr[r + 1];
  }
  const lsamp_penalty_entry* ent = a->penalty_entries;

  /* RepetitionContext.process (:586-596): takeAlong, where(x<0, x*p, x/p),
   * putAlong; duplicate ring ids write the same value, so once per id. */
  if (p->repetition_penalty != 1.0f) {
    const float rp = round_dtype(p->repetition_penalty, dt);
    for (int32_t e = e0; e < e1; ++e) {
      if (!(ent[e].flags & LSAMP_PEN_REPETITION)) continue;
      float v = x[ent[e].token];
      x[ent[e].token] = round_dtype(v < 0.0f ? v * rp : v / rp, dt);
    }
  }
  /* PresencePenaltyContext.process (:620-625) */
  if (p->presence_penalty != 0.0f) {
    const float pp = round_dtype(p->presence_penalty, dt);
    for (int32_t e = e0; e < e1; ++e) {
      if (!(ent[e].flags & LSAMP_PEN_PRESENCE)) continue;
      x[ent[e].token] = round_dtype(x[ent[e].token] - pp, dt);
    }
  }
  /* FrequencyPenaltyContext.process (:649-658): dense float32 histogram */
  if (p->frequency_penalty != 0.0f) {
    memset(s->dense_a, 0, sizeof(float) * (size_t)V);
    for (int32_t e = e0; e < e1; ++e) s->dense_a[ent[e].token] = (float)ent[e].count;
    const float f = p->frequency_penalty;
    for (int32_t i = 0; i < V; ++i) {
      float h = s->dense_a[i] * f;
      x[i] = x[i] - h;
    }
  }
  if (a->bitmask) {
    const uint32_t* mrow = a->bitmask + (size_t)r * (size_t)a->mask_words;
    for (int32_t i = 0; i < V; ++i)
      if (!mask_allows(mrow, a->mask_words, a->mask_bits, a->mask_tail, i)) x[i] = -INFINITY;
  }
  suppress_apply(a, x);
}

/* ----------------------------------------------------------------- filters */

/* LogitsPipelineV2.applyTopKTopPMinP (LogitsPipelineV2.swift:421-453):
 * one descending sort, softmax, cumsum; keep iff rank < k, (cum - p) <= topP
 * and p >= minP * p_0.  Disabled filters carry k = V, topP = 2, minP = 0. */
static void cbv2_filter(const lsamp_row_params* p, int32_t V, const float* x, scratch_t* s,
                        float* tp_margin, float* mp_margin, double* tp_exact) {
  vi_t* o = s->order;
  for (int32_t i = 0; i < V; ++i) {
    o[i].v = x[i];
    o[i].i = i;
  }
  qsort(o, (size_t)V, sizeof(vi_t), cmp_desc_idasc);
  const float m = o[0].v;
  /* softmax normalizer: MLX's reduction order is not vendored; it is
   * accumulated here in double and rounded once, so that it carries no
   * order-dependent error of its own. */
  double zd = 0.0, zx = 0.0;
  for (int32_t r = 0; r < V; ++r) {
    s->cum[r] = expf(o[r].v - m); /* reuse cum[] for e_r */
    zd += (double)s->cum[r];
    zx += exp((double)o[r].v - (double)m);
  }
  const float z = (float)zd;
  const int32_t k = (p->top_k > 0 && p->top_k < V) ? p->top_k : V;
  const float tp = (p->top_p >= 1.0f) ? 2.0f : (p->top_p <= 0.0f ? 0.0f : p->top_p);
  const float mp = p->min_p > 0.0f ? (p->min_p > 1.0f ? 1.0f : p->min_p) : 0.0f;
  const float p0 = s->cum[0] / z;
  const float mp_thr = mp * p0;
  /* The top-p test uses the exclusive mass in double precision: MLX's fp32
   * cumsum order is not vendored, and a sequential fp32 sum over thousands
   * of terms drifts by more than the 1e-6 of cumulative mass the parity rule
   * allows.  The fp32 sequential margin is still reported (tp_margin). */
  float cum = 0.0f;
  double cum_x = 0.0; /* exclusive mass, double precision */
  for (int32_t r = 0; r < V; ++r) {
    const float pr = s->cum[r] / z;
    cum += pr;
    const float excl = cum - pr;
    const double excl_x = cum_x;
    if (tp_exact) tp_exact[o[r].i] = (double)tp - excl_x;
    cum_x += exp((double)o[r].v - (double)m) / zx;
    const int keep = (r < k) && (excl_x <= (double)tp) && (pr >= mp_thr);
    const int32_t i = o[r].i;
    s->keep[i] = (uint8_t)(keep && x[i] > -INFINITY);
    if (tp_margin) tp_margin[i] = tp - excl;
    if (mp_margin) mp_margin[i] = pr - mp_thr;
  }
}

/* TopPSampler.sample filters (Evaluate.swift:432-491) on log-probabilities:
 * top-p (ascending sort, cumsum(exp), keep cum > 1 - topP), then min-p
 * (lp >= max lp + log minP), then top-k (argPartition; equal values at the
 * k boundary: lower id kept, the library's rule). */
static void mlxlm_filter(const lsamp_row_params* p, int32_t V, const float* x, scratch_t* s,
                         float* tp_margin, float* mp_margin, double* tp_exact) {
  float* lp = s->y;
  /* logSoftmax (:438) */
  float m = -INFINITY;
  for (int32_t i = 0; i < V; ++i)
    if (x[i] > m) m = x[i];
  /* logsumexp: accumulated in double and rounded once (MLX's reduction order
   * is not vendored) */
  double zd = 0.0;
  for (int32_t i = 0; i < V; ++i) zd += (double)expf(x[i] - m);
  const float lse = m + logf((float)zd);
  double zx = 0.0;
  for (int32_t i = 0; i < V; ++i) zx += exp((double)x[i] - (double)m);
  const double lse_x = (double)m + log(zx);
  for (int32_t i = 0; i < V; ++i) lp[i] = x[i] - lse;
  for (int32_t i = 0; i < V; ++i) s->keep[i] = 1;

  vi_t* o = s->order;
  /* applyTopP (:462-471) */
  if (p->top_p > 0.0f && p->top_p < 1.0f) {
    for (int32_t i = 0; i < V; ++i) {
      o[i].v = lp[i];
      o[i].i = i;
    }
    qsort(o, (size_t)V, sizeof(vi_t), cmp_asc_idasc);
    /* keep where the inclusive ascending mass exceeds 1 - topP; the mass is
     * summed in double (see cbv2_filter), the threshold is the reference's
     * fp32 constant */
    const float thr = 1.0f - p->top_p;
    float cum = 0.0f;
    double cum_x = 0.0;
    for (int32_t r = 0; r < V; ++r) {
      cum += expf(o[r].v);
      const int32_t i = o[r].i;
      cum_x += exp((double)x[i] - lse_x);
      if (!(cum_x > (double)thr)) s->keep[i] = 0;
      if (tp_margin) tp_margin[i] = cum - thr;
      if (tp_exact) tp_exact[i] = cum_x - (double)thr;
    }
    for (int32_t i = 0; i < V; ++i)
      if (!s->keep[i]) lp[i] = -INFINITY;
  }
  /* applyMinP (:475-480) */
  if (p->min_p > 0.0f) {
    float mx = -INFINITY;
    for (int32_t i = 0; i < V; ++i)
      if (lp[i] > mx) mx = lp[i];
    const float thr = mx + logf(p->min_p);
    for (int32_t i = 0; i < V; ++i) {
      if (mp_margin) mp_margin[i] = lp[i] - thr;
      if (!(lp[i] >= thr)) {
        lp[i] = -INFINITY;
        s->keep[i] = 0;
      }
    }
  }
  /* applyTopK (:484-491) */
  if (p->top_k > 0 && p->top_k < V) {
    for (int32_t i = 0; i < V; ++i) {
      o[i].v = lp[i];
      o[i].i = i;
    }
    qsort(o, (size_t)V, sizeof(vi_t), cmp_desc_idasc);
    for (int32_t r = p->top_k; r < V; ++r) {
      lp[o[r].i] = -INFINITY;
      s->keep[o[r].i] = 0;
    }
  }
  for (int32_t i = 0; i < V; ++i)
    if (!(x[i] > -INFINITY)) s->keep[i] = 0;
}

/* Index of the largest value, lowest id on ties (MLX argMax). */
static int32_t argmax_lowest(int32_t V, const float* x) {
  int32_t best = -1;
  float bv = -INFINITY;
  for (int32_t i = 0; i < V; ++i)
    if (x[i] > bv) {
      bv = x[i];
      best = i;
    }
  return best;
}

/* ------------------------------------------------------------- one row */

static void fill_stats(lsamp_row_stats* st, int32_t V, const float* y, const uint8_t* keep,
                       float scale, int32_t token, uint64_t W, int32_t probe) {
  float y_max = -INFINITY;
  for (int32_t i = 0; i < V; ++i)
    if (y[i] > y_max) y_max = y[i];
  double zn = 0.0;
  for (int32_t i = 0; i < V; ++i)
    if (y[i] > -INFINITY) zn += exp((double)y[i] - (double)y_max);
  float kmax = -INFINITY, kmin = INFINITY;
  int32_t kept = 0;
  for (int32_t i = 0; i < V; ++i)
    if (keep[i]) {
      ++kept;
      if (y[i] > kmax) kmax = y[i];
      if (y[i] < kmin) kmin = y[i];
    }
  double km = 0.0, ke = 0.0;
  for (int32_t i = 0; i < V; ++i)
    if (keep[i]) {
      double d = ((double)y[i] - (double)kmax) * (double)scale;
      double e = exp(d);
      km += e;
      ke += e * d;
    }
  st->max_value = y_max;
  st->log_normalizer = (float)log(zn);
  st->kept = kept;
  st->token = token;
  st->kept_weight = W;
  st->probe_weight = 0;
  st->probe_prob = 0.0f;
  if (probe >= 0 && probe < V && keep[probe]) {
    st->probe_weight = lso_weight(y[probe], kmax, scale);
    st->probe_prob = W ? (float)((double)st->probe_weight / (double)W) : 0.0f;
  }
  st->cut_value = kept ? kmin : -INFINITY;
  st->kept_mass = (float)km;
  st->kept_entropy = km > 0.0 ? (float)(log(km) - ke / km) : 0.0f;
}

static void sample_row(const lso_sample_args* a, int32_t r, scratch_t* s) {
  const int32_t V = a->vocab;
  const lsamp_row_params* p = &a->params[r];
  uint32_t flags = 0;
  /* non-finite flag on the raw row (CBv2NonFiniteLogits.swift:30-34) */
  {
    const void* raw = (const char*)a->logits +
                      (size_t)r * (size_t)a->row_stride * (a->dtype == LSAMP_DTYPE_F32 ? 4 : 2);
    for (int32_t i = 0; i < V; ++i) {
      float v = load_logit(raw, a->dtype, i);
      if (!isfinite(v)) {
        flags |= LSAMP_ROW_NONFINITE;
        break;
      }
    }
  }
  if (a->semantics == LSAMP_SEM_CBV2)
    cbv2_transform(a, r, s);
  else
    mlxlm_transform(a, r, s);
  float* x = s->x;
  /* NaN defines no token: it is treated as masked (the row is flagged). */
  for (int32_t i = 0; i < V; ++i)
    if (x[i] != x[i]) x[i] = -INFINITY;
  if (a->processed) memcpy(a->processed + (size_t)r * (size_t)V, x, sizeof(float) * (size_t)V);

  float* tpm = a->top_p_margin ? a->top_p_margin + (size_t)r * (size_t)V : NULL;
  float* mpm = a->min_p_margin ? a->min_p_margin + (size_t)r * (size_t)V : NULL;
  double* tpx = a->top_p_margin_exact ? a->top_p_margin_exact + (size_t)r * (size_t)V : NULL;
  if (tpx)
    for (int32_t i = 0; i < V; ++i) tpx[i] = INFINITY;
  if (tpm)
    for (int32_t i = 0; i < V; ++i) tpm[i] = INFINITY;
  if (mpm)
    for (int32_t i = 0; i < V; ++i) mpm[i] = INFINITY;

  float x_max = -INFINITY;
  for (int32_t i = 0; i < V; ++i)
    if (x[i] > x_max) x_max = x[i];

  float scale = 1.0f;
  const float* y = x;
  if (x_max == -INFINITY) {
    memset(s->keep, 0, (size_t)V);
  } else if (p->kind == LSAMP_KIND_ARGMAX || !(p->temperature > 0.0f && p->temperature < INFINITY)) {
    /* ArgMaxSampler (Evaluate.swift:394-396); CBv2 greedy rows
     * (SamplerV2.swift:92); the first maximum, +inf included.  A sampled row
     * whose temperature defines no distribution is drawn the same way. */
    memset(s->keep, 0, (size_t)V);
    s->keep[argmax_lowest(V, x)] = 1;
  } else if (x_max == INFINITY) {
    /* +inf logits in a sampled row: the limit of the softmax is uniform over
     * the +inf ids. */
    for (int32_t i = 0; i < V; ++i) s->keep[i] = (uint8_t)(x[i] == INFINITY);
  } else if (a->semantics == LSAMP_SEM_CBV2) {
    cbv2_filter(p, V, x, s, tpm, mpm, tpx);
  } else if (p->kind == LSAMP_KIND_CATEGORICAL) {
    /* CategoricalSampler (Evaluate.swift:506-510): categorical(x * (1/T)) */
    for (int32_t i = 0; i < V; ++i) s->keep[i] = (uint8_t)(x[i] > -INFINITY);
    scale = 1.0f / p->temperature;
  } else {
    mlxlm_filter(p, V, x, s, tpm, mpm, tpx);
    scale = 1.0f / p->temperature;
  }
  if (a->keep) memcpy(a->keep + (size_t)r * (size_t)V, s->keep, (size_t)V);

  float u = a->uniforms ? a->uniforms[r] : lso_rng_uniform(a->philox_keys[r], 0u);
  uint64_t W = 0;
  int32_t token = lso_draw(V, y, s->keep, scale, u, &W);
  if (token < 0) flags |= LSAMP_ROW_EMPTY;
  if (a->tokens) a->tokens[r] = token;
  if (a->row_flags) a->row_flags[r] = flags;
  if (a->stats)
    fill_stats(&a->stats[r], V, y, s->keep, scale, token, W,
               a->probe_tokens ? a->probe_tokens[r] : -1);
}

/* ------------------------------------------------------------- threading */

typedef struct {
  const lso_sample_args* a;
  int32_t tid, nthreads;
  int32_t status;
} worker_t;

static void* sample_worker(void* arg) {
  worker_t* w = (worker_t*)arg;
  scratch_t s;
  if (!scratch_init(&s, w->a->vocab)) {
    w->status = LSAMP_ERR_CAPACITY;
    scratch_free(&s);
    return NULL;
  }
  for (int32_t r = w->tid; r < w->a->rows; r += w->nthreads) sample_row(w->a, r, &s);
  scratch_free(&s);
  w->status = 0;
  return NULL;
}

static int32_t validate(const lso_sample_args* a) {
  if (!a || !a->logits || !a->params) return LSAMP_ERR_INVALID_ARGUMENT;
  if (a->rows <= 0 || a->vocab <= 0 || a->row_stride < a->vocab) return LSAMP_ERR_SHAPE;
  if (a->dtype < 0 || a->dtype > 2) return LSAMP_ERR_DTYPE;
  if (!a->uniforms && !a->philox_keys) return LSAMP_ERR_INVALID_ARGUMENT;
  if (a->bitmask && (a->mask_words <= 0 || a->mask_bits < 0)) return LSAMP_ERR_SHAPE;
  return 0;
}

int32_t lso_sample(const lso_sample_args* a) {
  int32_t st = validate(a);
  if (st) return st;
  int32_t nt = a->threads > 1 ? a->threads : 1;
  if (nt > a->rows) nt = a->rows;
  if (nt == 1) {
    worker_t w = {a, 0, 1, 0};
    sample_worker(&w);
    return w.status;
  }
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nt);
  worker_t* ws = (worker_t*)malloc(sizeof(worker_t) * (size_t)nt);
  for (int32_t t = 0; t < nt; ++t) {
    ws[t].a = a;
    ws[t].tid = t;
    ws[t].nthreads = nt;
    ws[t].status = 0;
    pthread_create(&th[t], NULL, sample_worker, &ws[t]);
  }
  int32_t status = 0;
  for (int32_t t = 0; t < nt; ++t) {
    pthread_join(th[t], NULL);
    if (ws[t].status) status = ws[t].status;
  }
  free(th);
  free(ws);
  return status;
}

/* ------------------------------------------------------------- MTP verify */

/* One verify row: CBv2 transform (no penalties, no mask) and filter with the
 * sequence's params, then fixed-point weights (scale 1). */
static void verify_row(const void* logits, int32_t dtype, int32_t V, const lsamp_row_params* p,
                       scratch_t* s, uint64_t* w, uint64_t* W_out, float* y_out,
                       const int32_t* pen_rp, const lsamp_penalty_entry* pen_ent) {
  lso_sample_args a;
  memset(&a, 0, sizeof a);
  a.semantics = LSAMP_SEM_CBV2;
  a.rows = 1;
  a.vocab = V;
  a.dtype = dtype;
  a.row_stride = V;
  a.logits = logits;
  a.params = p;
  a.penalty_row_ptr = pen_rp;
  a.penalty_entries = pen_ent;
  cbv2_transform(&a, 0, s);
  float* x = s->x;
  for (int32_t i = 0; i < V; ++i)
    if (x[i] != x[i]) x[i] = -INFINITY;
  float x_max = -INFINITY;
  for (int32_t i = 0; i < V; ++i)
    if (x[i] > x_max) x_max = x[i];
  if (x_max == -INFINITY) {
    memset(s->keep, 0, (size_t)V);
  } else if (p->kind == LSAMP_KIND_ARGMAX) {
    memset(s->keep, 0, (size_t)V);
    s->keep[argmax_lowest(V, x)] = 1;
  } else {
    cbv2_filter(p, V, x, s, NULL, NULL, NULL);
  }
  float kmax = -INFINITY;
  for (int32_t i = 0; i < V; ++i)
    if (s->keep[i] && x[i] > kmax) kmax = x[i];
  uint64_t W = 0;
  for (int32_t i = 0; i < V; ++i) {
    w[i] = s->keep[i] ? lso_weight(x[i], kmax, 1.0f) : 0;
    W += w[i];
  }
  *W_out = W;
  if (y_out) memcpy(y_out, x, sizeof(float) * (size_t)V);
}

static int32_t draw_from_weights(int32_t V, const uint64_t* w, uint64_t W, float u) {
  if (W == 0) return -1;
  uint64_t target = scaled_target(uniform_u32(u), W);
  uint64_t cum = 0;
  for (int32_t i = 0; i < V; ++i) {
    cum += w[i];
    if (w[i] && cum > target) return i;
  }
  return -1;
}

typedef struct {
  const lso_verify_args* a;
  int32_t tid, nthreads, status;
} vworker_t;

static void* verify_worker(void* arg) {
  vworker_t* vw = (vworker_t*)arg;
  const lso_verify_args* a = vw->a;
  const int32_t V = a->vocab, W = a->window, D = W - 1;
  const size_t esz = a->dtype == LSAMP_DTYPE_F32 ? 4 : 2;
  scratch_t s;
  uint64_t* wt = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
  uint64_t* wd = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
  uint64_t* res = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
  float* yt = (float*)malloc(sizeof(float) * (size_t)V);
  float* cnt = (float*)malloc(sizeof(float) * (size_t)V);
  lsamp_penalty_entry* ent = (lsamp_penalty_entry*)malloc(sizeof(lsamp_penalty_entry) * (size_t)V);
  if (!scratch_init(&s, V) || !wt || !wd || !res || !yt || !cnt || !ent) {
    vw->status = LSAMP_ERR_CAPACITY;
    goto done;
  }
  for (int32_t sq = vw->tid; sq < a->sequences; sq += vw->nthreads) {
    const lsamp_row_params* p = &a->params[sq];
    const float* u = a->uniforms + (size_t)sq * (size_t)W;
    int32_t* tok = a->tokens + (size_t)sq * (size_t)W;
    uint8_t* am = a->accept_mask ? a->accept_mask + (size_t)sq * (size_t)D : NULL;
    const int32_t* drafts = a->draft_tokens + (size_t)sq * (size_t)D;
    for (int32_t j = 0; j < W; ++j) tok[j] = -1;
    if (am) memset(am, 0, (size_t)D);
    if (a->mode == LSAMP_VERIFY_RESIDUAL) {
      int32_t j = 0;
      int32_t emitted = -1;
      for (; j < D; ++j) {
        uint64_t Wt, Wd;
        const void* trow = (const char*)a->target_logits + ((size_t)sq * W + j) * (size_t)V * esz;
        const void* drow = (const char*)a->draft_logits + ((size_t)sq * D + j) * (size_t)V * esz;
        verify_row(trow, a->dtype, V, p, &s, wt, &Wt, NULL, NULL, NULL);
        verify_row(drow, a->dtype, V, p, &s, wd, &Wd, NULL, NULL, NULL);
        const int32_t x = drafts[j];
        const double pt = (x >= 0 && x < V && Wt) ? (double)wt[x] / (double)Wt : 0.0;
        const double pd = (x >= 0 && x < V && Wd) ? (double)wd[x] / (double)Wd : 0.0;
        int accept = pd > 0.0 ? ((double)u[j] < pt / pd) : (pt > 0.0);
        if (accept) {
          tok[j] = x;
          if (am) am[j] = 1;
          continue;
        }
        /* residual max(0, p_t - p_d), quantized to 2^-52 */
        uint64_t R = 0;
        for (int32_t i = 0; i < V; ++i) {
          uint64_t qt = Wt ? (uint64_t)(((double)wt[i] / (double)Wt) * 4503599627370496.0) : 0;
          uint64_t qd = Wd ? (uint64_t)(((double)wd[i] / (double)Wd) * 4503599627370496.0) : 0;
          res[i] = qt > qd ? qt - qd : 0;
          R += res[i];
        }
        emitted = R ? draw_from_weights(V, res, R, u[D]) : draw_from_weights(V, wt, Wt, u[D]);
        tok[j] = emitted;
        break;
      }
      if (j == D) {
        uint64_t Wt;
        const void* trow = (const char*)a->target_logits + ((size_t)sq * W + D) * (size_t)V * esz;
        verify_row(trow, a->dtype, V, p, &s, wt, &Wt, NULL, NULL, NULL);
        tok[D] = draw_from_weights(V, wt, Wt, u[D]);
      }
      a->accepted[sq] = j;
    } else {
      int32_t prefix = 0, still = 1;
      /* applyWindowPenalties (DefaultSamplerV2.swift:503-580) for rows with a
       * frequency or presence penalty: counts = the confirmed output counts
       * plus the one-hot of the drafts before the position, applied as
       * x - f*c - p*(c > 0) (stage 2 of LogitsPipelineV2.process) */
      const int pen = a->out_ptr && (p->frequency_penalty != 0.0f || p->presence_penalty != 0.0f);
      if (pen) {
        memset(cnt, 0, sizeof(float) * (size_t)V);
        for (int32_t i = a->out_ptr[sq]; i < a->out_ptr[sq + 1]; ++i)
          if (a->out_tokens[i] >= 0 && a->out_tokens[i] < V) cnt[a->out_tokens[i]] += 1.0f;
      }
      const int32_t* chain = a->pen_drafts ? a->pen_drafts + (size_t)sq * (size_t)a->pen_stride
                                           : drafts;
      const int32_t off = a->pen_drafts ? a->pen_offset : 0;
      if (pen)
        for (int32_t i = 0; i < off; ++i)
          if (chain[i] >= 0 && chain[i] < V) cnt[chain[i]] += 1.0f;
      for (int32_t j = 0; j < W; ++j) {
        uint64_t Wt;
        const void* trow = (const char*)a->target_logits + ((size_t)sq * W + j) * (size_t)V * esz;
        int32_t rp[2] = {0, 0};
        if (pen) {
          if (j > 0 && chain[off + j - 1] >= 0 && chain[off + j - 1] < V) cnt[chain[off + j - 1]] += 1.0f;
          for (int32_t i = 0; i < V; ++i)
            if (cnt[i] > 0.0f) {
              ent[rp[1]].token = i;
              ent[rp[1]].count = (int32_t)cnt[i];
              ent[rp[1]].flags = 0u;
              ent[rp[1]].bias = 0.0f;
              ++rp[1];
            }
        }
        verify_row(trow, a->dtype, V, p, &s, wt, &Wt, yt, pen ? rp : NULL, pen ? ent : NULL);
        tok[j] = draw_from_weights(V, wt, Wt, u[j]);
        if (j >= D) continue;
        int accept;
        /* greedy rows, and penalty rows when penalties are applied, accept
         * exactly (DefaultSamplerV2.swift:496-502) */
        if (a->mode == LSAMP_VERIFY_EXACT || p->kind == LSAMP_KIND_ARGMAX || pen) {
          accept = tok[j] == drafts[j];
        } else {
          /* CBv2MTPTypicalAcceptanceTests.swift:16-33 restated in double on
           * the filtered, tempered row (DefaultSamplerV2.swift:485-502) */
          double mx = -INFINITY;
          for (int32_t i = 0; i < V; ++i)
            if (s.keep[i] && yt[i] > mx) mx = yt[i];
          double z = 0.0;
          for (int32_t i = 0; i < V; ++i)
            if (s.keep[i]) z += exp((double)yt[i] - mx);
          double h = 0.0;
          for (int32_t i = 0; i < V; ++i)
            if (s.keep[i]) {
              double pi = exp((double)yt[i] - mx) / z;
              if (pi > 0.0) h -= pi * log(pi);
            }
          const int32_t x = drafts[j];
          double pdraft = (x >= 0 && x < V && s.keep[x]) ? exp((double)yt[x] - mx) / z : 0.0;
          double floor_ = fmin(1.0, (double)a->typical_delta * exp(-h));
          accept = pdraft > floor_;
          if (a->typical_margin) a->typical_margin[(size_t)sq * D + j] = pdraft - floor_;
        }
        if (am) am[j] = (uint8_t)accept;
        if (still && accept)
          ++prefix;
        else
          still = 0;
      }
      a->accepted[sq] = prefix;
    }
  }
  vw->status = 0;
done:
  scratch_free(&s);
  free(wt);
  free(wd);
  free(res);
  free(yt);
  free(cnt);
  free(ent);
  return NULL;
}

int32_t lso_verify(const lso_verify_args* a) {
  if (!a || !a->target_logits || !a->draft_tokens || !a->params || !a->uniforms || !a->tokens ||
      !a->accepted)
    return LSAMP_ERR_INVALID_ARGUMENT;
  if (a->sequences <= 0 || a->window < 2 || a->vocab <= 0) return LSAMP_ERR_SHAPE;
  if (a->mode == LSAMP_VERIFY_RESIDUAL && !a->draft_logits) return LSAMP_ERR_INVALID_ARGUMENT;
  if (a->mode == LSAMP_VERIFY_TYPICAL && !(a->typical_delta > 0.0f))
    return LSAMP_ERR_INVALID_ARGUMENT;
  int32_t nt = a->threads > 1 ? a->threads : 1;
  if (nt > a->sequences) nt = a->sequences;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nt);
  vworker_t* ws = (vworker_t*)malloc(sizeof(vworker_t) * (size_t)nt);
  for (int32_t t = 0; t < nt; ++t) {
    ws[t].a = a;
    ws[t].tid = t;
    ws[t].nthreads = nt;
    ws[t].status = 0;
    pthread_create(&th[t], NULL, verify_worker, &ws[t]);
  }
  int32_t status = 0;
  for (int32_t t = 0; t < nt; ++t) {
    pthread_join(th[t], NULL);
    if (ws[t].status) status = ws[t].status;
  }
  free(th);
  free(ws);
  return status;
}

/* ------------------------------------------------------ ranking of raw logits */

/* darkbloom_qwen35_mtp_top2_better, CBv2TopTwo.swift:29-47: a NaN never beats
 * a number; otherwise the larger value wins and an exact tie (+0 == -0) goes
 * to the lower id. */
static int rank_better(float a, int32_t ia, float b, int32_t ib) {
  const int an = isnan(a), bn = isnan(b);
  if (an != bn) return !an;
  if (a > b) return 1;
  if (a < b) return 0;
  return ia < ib;
}

/* log(sum(exp(x))) of one row in double, with MLX's conventions for
 * non-finite rows (logsumexp: the row maximum is returned where it is
 * infinite): NaN if any logit is NaN, +inf if one is +inf, -inf if all are
 * -inf.  The reference evaluates raw - logSumExp(raw) in float32
 * (LogitsPipelineV2.swift:311; Evaluate.swift:805 logSoftmax). */
static double row_lse(const void* row, int32_t dtype, int32_t V, int64_t cs, uint32_t* nonfinite) {
  int nan = 0, pinf = 0;
  double m = -INFINITY;
  for (int32_t i = 0; i < V; ++i) {
    const float x = load_logit(row, dtype, (int64_t)i * cs);
    if (isnan(x)) {
      nan = 1;
    } else {
      if (x == INFINITY) pinf = 1;
      if (x > m) m = x;
    }
    if (!isfinite(x)) *nonfinite = 1;
  }
  if (nan) return NAN;
  if (pinf) return INFINITY;
  if (m == -INFINITY) return -INFINITY;
  double z = 0.0;
  for (int32_t i = 0; i < V; ++i) z += exp((double)load_logit(row, dtype, (int64_t)i * cs) - m);
  return m + log(z);
}

int32_t lso_rank(const lso_rank_args* a) {
  if (!a || !a->logits || a->rows <= 0 || a->vocab <= 0 || a->k < 0 || a->k > a->vocab ||
      a->col_stride < 1 || a->row_stride < 0)
    return LSAMP_ERR_INVALID_ARGUMENT;
  const size_t es = a->dtype == LSAMP_DTYPE_F32 ? 4 : 2;
  const int32_t V = a->vocab, k = a->k;
  float* tv = (float*)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1));
  int32_t* ti = (int32_t*)malloc(sizeof(int32_t) * (size_t)(k > 0 ? k : 1));
  if (!tv || !ti) {
    free(tv);
    free(ti);
    return LSAMP_ERR_CAPACITY;
  }
  for (int32_t r = 0; r < a->rows; ++r) {
    const char* row = (const char*)a->logits + (size_t)r * (size_t)a->row_stride * es;
    /* the k best by insertion into a sorted list (CBv2TopTwo.swift:49-79
     * keeps the best two the same way) */
    int32_t n = 0;
    for (int32_t i = 0; i < V; ++i) {
      const float x = load_logit(row, a->dtype, (int64_t)i * a->col_stride);
      if (n == k && (k == 0 || !rank_better(x, i, tv[k - 1], ti[k - 1]))) continue;
      int32_t p = n < k ? n : k - 1;
      while (p > 0 && rank_better(x, i, tv[p - 1], ti[p - 1])) {
        tv[p] = tv[p - 1];
        ti[p] = ti[p - 1];
        --p;
      }
      tv[p] = x;
      ti[p] = i;
      if (n < k) ++n;
    }
    uint32_t nonfinite = 0;
    const double lse = row_lse(row, a->dtype, V, a->col_stride, &nonfinite);
    uint32_t flags = nonfinite ? LSAMP_ROW_NONFINITE : 0u;
    /* A row whose log-sum-exp is not finite (a NaN or +inf logit, or every
     * logit -inf) defines no log-probabilities.  The reference fails such a
     * row closed: CBv2NonFiniteLogits.flags (CBv2NonFiniteLogits.swift:30-34)
     * marks it and the request finishes with an error, committing nothing
     * from it (:8-14).  Here it carries LSAMP_ROW_NONFINITE, ids -1 and NaN
     * values.  The exact top-2 (raw values) still ranks such rows. */
    const int closed = !a->raw_values && !isfinite(lse);
    for (int32_t j = 0; j < k; ++j) {
      if (a->ids) a->ids[(size_t)r * k + j] = closed ? -1 : ti[j];
      if (a->values)
        a->values[(size_t)r * k + j] =
            a->raw_values ? tv[j] : closed ? NAN : (float)((double)tv[j] - lse);
    }
    if (a->tokens) {
      const int32_t t = a->tokens[r];
      float c = NAN;
      if (t < 0 || t >= V)
        flags |= LSAMP_ROW_TOKEN_RANGE;
      else if (!closed)
        c = (float)((double)load_logit(row, a->dtype, (int64_t)t * a->col_stride) - lse);
      if (a->chosen) a->chosen[r] = c;
    }
    if (a->row_flags) a->row_flags[r] = flags;
    if (a->lse) a->lse[r] = lse;
  }
  free(tv);
  free(ti);
  return 0;
}

/* ------------------------------------------------- incremental penalty state */

/* buildCounts (LogitsPipelineV2.swift:478-487): ids outside [0, vocab) are
 * skipped.  buildRepetitionWindow (:494-510): the most recent
 * min(W, |history|) ids of prompt + output at slots 0.., -1 elsewhere; the
 * write position is 0 when the window is full, else the first empty slot. */
void lso_penalty_state_init(int32_t V, const int32_t* prompt, int32_t np, const int32_t* output,
                            int32_t no, int32_t W, float* counts, float* wcounts,
                            int32_t* window, int32_t* ring_pos) {
  memset(counts, 0, sizeof(float) * (size_t)V);
  memset(wcounts, 0, sizeof(float) * (size_t)V);
  for (int32_t i = 0; i < no; ++i)
    if (output[i] >= 0 && output[i] < V) counts[output[i]] += 1.0f;
  const int32_t n = np + no;
  const int32_t take = n < W ? n : W;
  for (int32_t j = 0; j < W; ++j) window[j] = -1;
  for (int32_t j = 0; j < take; ++j) {
    const int32_t h = n - take + j;
    const int32_t t = h < np ? prompt[h] : output[h - np];
    window[j] = t >= 0 ? t : -1;
    if (t >= 0 && t < V) wcounts[t] += 1.0f;
  }
  *ring_pos = take == W ? 0 : take;
}

/* commit(sampledTokens:) (LogitsPipelineV2.swift:357-384) for one row:
 *   outputCounts[t] += 1;
 *   evicted = window[pos]; repWindowCounts[max(evicted, 0)] -= (evicted >= 0);
 *   repWindowCounts[t] += 1; window[pos] = t; pos = (pos + 1) % W. */
void lso_penalty_commit(int32_t V, uint32_t mode, int32_t W, float* counts, float* wcounts,
                        int32_t* window, int32_t* ring_pos, int32_t t) {
  if (t < 0 || t >= V) return;
  if (mode & LSAMP_STATE_COUNTS) counts[t] += 1.0f;
  if (mode & LSAMP_STATE_REPETITION) {
    const int32_t pos = *ring_pos;
    const int32_t ev = window[pos];
    if (ev >= 0 && ev < V) wcounts[ev] -= 1.0f;
    wcounts[t] += 1.0f;
    window[pos] = t;
    *ring_pos = (pos + 1) % W;
  }
}
