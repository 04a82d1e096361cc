/*
 * lsamp_oracle.h — CPU restatement of the reference's logits-to-token stage.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline), never as the thing measured or shipped.  The
 * product path (liblsamp.so) does not link it.
 *
 * It follows the reference op sequence literally: full per-row sorts for
 * top-p / top-k / min-p, dense per-row penalty tensors, one materialized
 * intermediate per stage.  Each function names the reference lines it restates.
 * Host pointers throughout.
 */
#ifndef LSAMP_ORACLE_H
#define LSAMP_ORACLE_H

#include <stdint.h>

#include "../include/lsamp.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lso_sample_args {
  int32_t semantics;
  int32_t rows;
  int32_t vocab;
  int32_t dtype;
  int64_t row_stride;
  const void* logits;
  const lsamp_row_params* params;
  const int32_t* penalty_row_ptr;
  const lsamp_penalty_entry* penalty_entries;
  const uint32_t* bitmask;
  int32_t mask_words;
  int32_t mask_bits;
  int32_t mask_tail;
  const float* uniforms;       /* or NULL -> lso_rng_uniform(philox_keys[r], 0) */
  const uint64_t* philox_keys;
  const int32_t* probe_tokens; /* or NULL */
  int32_t threads;             /* worker threads over rows (<= 1: serial) */
  /* outputs (NULL = not wanted) */
  int32_t* tokens;       /* [rows] */
  uint32_t* row_flags;   /* [rows] */
  float* processed;      /* [rows, vocab] filter-space logits before the filters */
  uint8_t* keep;         /* [rows, vocab] 1 = token survives the filters */
  float* top_p_margin;   /* [rows, vocab] signed distance of the top-p test
                            in the reference's fp32 sequential cumsum
                            (diagnostic; the decision uses the exact mass) */
  float* min_p_margin;   /* [rows, vocab] signed distance of the min-p test */
  double* top_p_margin_exact; /* [rows, vocab] the top-p distance in exact
                                 (double) arithmetic from the same logits: the
                                 quantity the top-p test decides on */
  lsamp_row_stats* stats;/* [rows] */
  /* SuppressTokensProcessor (SuppressTokens.swift:67-81): ids masked to -inf
   * after the penalties and the bitmask; negatives and ids >= vocab ignored */
  const int32_t* suppress_ids;
  int32_t n_suppress;
} lso_sample_args;

/* Full sampling step (both semantics).  Returns 0 or a negative status. */
int32_t lso_sample(const lso_sample_args* a);

typedef struct lso_verify_args {
  int32_t mode;
  int32_t sequences;
  int32_t window;
  int32_t vocab;
  int32_t dtype;
  const void* target_logits;
  const void* draft_logits;
  const int32_t* draft_tokens;
  const lsamp_row_params* params;
  const float* uniforms;
  float typical_delta;
  int32_t threads;
  int32_t* accepted;
  int32_t* tokens;
  uint8_t* accept_mask;
  double* typical_margin; /* [S, W-1] or NULL: p(draft) - floor (TYPICAL) */
  /* penalty-aware windows (EXACT / TYPICAL), or NULL: each sequence's
   * confirmed output tokens out_tokens[out_ptr[s] .. out_ptr[s+1]), and the
   * round's draft chain pen_drafts [S, pen_stride] (NULL: draft_tokens) of
   * which position j counts chain positions [0, pen_offset + j) */
  const int32_t* out_ptr;
  const int32_t* out_tokens;
  const int32_t* pen_drafts;
  int32_t pen_stride;
  int32_t pen_offset;
} lso_verify_args;

/* MTP verification (RESIDUAL / EXACT / TYPICAL).  Returns 0 or < 0. */
int32_t lso_verify(const lso_verify_args* a);

typedef struct lso_rank_args {
  int32_t rows;
  int32_t vocab;
  int32_t dtype;
  int64_t row_stride;  /* elements */
  int64_t col_stride;  /* elements */
  const void* logits;
  int32_t k;           /* best tokens reported per row */
  int32_t raw_values;  /* 1: values = raw logits (top-2); 0: log-probabilities */
  const int32_t* tokens; /* [rows] or NULL */
  /* outputs (NULL = not wanted) */
  float* chosen;       /* [rows] log-probability of tokens[r] (NaN if out of range) */
  float* values;       /* [rows, k] */
  int32_t* ids;        /* [rows, k] */
  uint32_t* row_flags; /* [rows] LSAMP_ROW_NONFINITE | LSAMP_ROW_TOKEN_RANGE */
  double* lse;         /* [rows] the log-sum-exp */
} lso_rank_args;

/* Exact top-k of raw logits and their log-probabilities (top-2:
 * CBv2TopTwo.swift; log-probabilities: LogitsPipelineV2.swift:307-314,
 * 534-549).  Returns 0 or < 0. */
int32_t lso_rank(const lso_rank_args* a);

/* The CBv2 incremental penalty state of one row, dense over the vocabulary
 * (LogitsPipelineV2.setRows :238-256, buildCounts :478-487,
 * buildRepetitionWindow :494-510): output counts, window counts, the [W]
 * ring (-1 = empty) and its write position. */
void lso_penalty_state_init(int32_t vocab, const int32_t* prompt, int32_t n_prompt,
                            const int32_t* output, int32_t n_output, int32_t window_size,
                            float* counts, float* window_counts, int32_t* window,
                            int32_t* ring_pos);
/* LogitsPipelineV2.commit (:357-384) of one row, dense.  mode: LSAMP_STATE_*
 * bits; a token outside [0, vocab) commits nothing. */
void lso_penalty_commit(int32_t vocab, uint32_t mode, int32_t window_size, float* counts,
                        float* window_counts, int32_t* window, int32_t* ring_pos, int32_t token);

/* Building blocks exposed for known-answer tests. */
float lso_dexp(float d);
uint64_t lso_weight(float y, float y_max, float scale);
int32_t lso_draw(int32_t n, const float* y, const uint8_t* keep, float scale, float u,
                 uint64_t* total_out);
void lso_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
uint64_t lso_rng_key(uint64_t seed, uint64_t id, uint64_t step);
float lso_rng_uniform(uint64_t key, uint32_t purpose);
float lso_bf16_to_f32(uint16_t h);
uint16_t lso_f32_to_bf16(float f);
float lso_f16_to_f32(uint16_t h);
uint16_t lso_f32_to_f16(float f);
void lso_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n);
void lso_f32_to_f16_n(const float* in, uint16_t* out, int64_t n);
void lso_f16_to_f32_n(const uint16_t* in, float* out, int64_t n);

#ifdef __cplusplus
}
#endif

#endif
