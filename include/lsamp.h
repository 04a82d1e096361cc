/*
 * lsamp.h — C ABI of the MI355X (gfx950) logits-to-token stage.
 *
 * One call turns a batch of [rows, vocab] logits that already sit in HBM into
 * one token id per row: penalties, grammar bitmask, temperature,
 * top-k / top-p / min-p and the draw run as hand-written HIP kernels that read
 * every logit once.  The ABI replaces the MLX graph that the reference builds
 * for this stage:
 *
 *   - mlx-lm order (single stream):  PenaltyProcessor.process
 *       (Libraries/MLXLMCommon/Evaluate.swift:687-693) followed by
 *       ArgMaxSampler / TopPSampler / CategoricalSampler .sample
 *       (Evaluate.swift:394-396, 432-491, 506-510);
 *   - CBv2 order (batched):  LogitsPipelineV2.process
 *       (Libraries/MLXLMCommon/ContinuousBatchingV2/LogitsPipelineV2.swift:292-352,
 *       applyTopKTopPMinP :421-453) followed by SamplerV2.sample
 *       (ContinuousBatchingV2/SamplerV2.swift:85-107);
 *   - the grammar mask apply of xgrammar's ApplyTokenBitmaskInplaceCPU
 *       (Libraries/MLXCXGrammar/xgrammar/cpp/grammar_matcher.cc:89-235) and of
 *       GuidedGenerationLoop.bitmaskToMLXArray
 *       (Libraries/MLXGuidedGeneration/GuidedGenerationLoop.swift:595-610);
 *   - MTP verification: CBv2DefaultSampler.verifyWindow
 *       (ContinuousBatchingV2/DefaultSamplerV2.swift:382-503) and textbook
 *       speculative sampling (accept min(1, p_t/p_d), residual max(0, p_t-p_d)).
 *
 * Conventions follow the reference's own C ABI (Libraries/MLXCXGrammar/include/
 * xgrammar_c.h:28-69): opaque handles, caller-owned buffers, int32 status
 * codes (0 = OK, negative = error) and a thread-local last-error string.
 * Every pointer in an args struct is a DEVICE pointer unless stated
 * otherwise; the call enqueues work on `stream` (a hipStream_t, NULL = the
 * default stream) and never synchronizes or allocates.
 *
 * Draw rule.  The reference draws with MLX's Gumbel / exponential race
 * (Evaluate.swift:456,508; SamplerV2.swift:101-106), which consumes V random
 * numbers per row.  This library draws by inverse CDF from ONE uniform per row,
 * in token-id order, with integer (fixed-point) weights so that the CPU
 * restatement reproduces the chosen token bit for bit:
 *     d_i = fl(fl(y_i - y_max) * scale)   (scale = 1 in CBv2, fl(1/T) in mlx-lm)
 *     w_i = (uint64) (dexp(d_i) * 2^40)   for kept tokens, 0 otherwise
 *     W = sum w_i;  U = (uint32)(u * 2^32);  target = (U * W) >> 32
 *     token = smallest id i with  w_0 + ... + w_i > target.
 * dexp is a fixed fp32 Cody-Waite + Taylor-7 exponential evaluated with fma,
 * identical on host and device.
 */
#ifndef LSAMP_H
#define LSAMP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LSAMP_ABI_VERSION 1

/* ---- status codes (xgrammar_c.h:55-61 style) ---------------------------- */
typedef int32_t lsamp_status;
#define LSAMP_OK 0
#define LSAMP_ERR_INVALID_ARGUMENT (-1) /* null pointer, bad enum, bad size   */
#define LSAMP_ERR_SHAPE (-2)            /* rows/vocab/strides out of range     */
#define LSAMP_ERR_DTYPE (-3)            /* unsupported logits dtype            */
#define LSAMP_ERR_CAPACITY (-4)         /* larger than the context was made for */
#define LSAMP_ERR_DEVICE (-5)           /* a HIP runtime call failed           */

/* ---- enums ---------------------------------------------------------------- */
typedef enum lsamp_dtype {
  LSAMP_DTYPE_F32 = 0,
  LSAMP_DTYPE_BF16 = 1,
  LSAMP_DTYPE_F16 = 2
} lsamp_dtype;

/* Which of the reference's two pipelines a call reproduces. */
typedef enum lsamp_semantics {
  /* Evaluate.swift:328-746: penalties in the logits dtype, filters top-p ->
   * min-p -> top-k on un-tempered log-probs, draw from logprobs * (1/T). */
  LSAMP_SEM_MLXLM = 0,
  /* LogitsPipelineV2.swift:292-453: fp32 cast, bias, repetition,
   * frequency/presence, x / T, grammar mask, one joint top-k/top-p/min-p. */
  LSAMP_SEM_CBV2 = 1
} lsamp_semantics;

/* Per-row sampler after parameter resolution. */
typedef enum lsamp_kind {
  LSAMP_KIND_ARGMAX = 0,      /* ArgMaxSampler; CBv2 greedy row (T < 1e-5)  */
  LSAMP_KIND_FILTERED = 1,    /* TopPSampler; CBv2 sampled row              */
  LSAMP_KIND_CATEGORICAL = 2  /* CategoricalSampler (mlx-lm, no filters)    */
} lsamp_kind;

/* Bitmask words past `mask_bits`:
 * KEEP   = ApplyTokenBitmaskInplaceCPU leaves ids >= vocab_size untouched
 *          (grammar_matcher.cc:108-121);
 * FORBID = bitmaskToMLXArray sets ids >= maskBitCount to -inf
 *          (GuidedGenerationLoop.swift:600-601). */
typedef enum lsamp_mask_tail {
  LSAMP_MASK_TAIL_KEEP = 0,
  LSAMP_MASK_TAIL_FORBID = 1
} lsamp_mask_tail;

/* Penalty entry flags. */
#define LSAMP_PEN_REPETITION 1u /* token is in the repetition window        */
#define LSAMP_PEN_PRESENCE 2u   /* mlx-lm only: token is in the presence window */

/* Row flags written to `row_flags`. */
#define LSAMP_ROW_NONFINITE 1u /* a raw logit is NaN or +-inf (CBv2NonFiniteLogits.swift:30-34) */
#define LSAMP_ROW_EMPTY 2u     /* no token survived masking; token = -1       */
#define LSAMP_ROW_OVERFLOW 4u  /* the cut bucket held more candidates than the
                                  context's candidate capacity; token = -1   */
#define LSAMP_ROW_TOKEN_RANGE 8u /* lsamp_logprobs: the row's token lies outside
                                    [0, vocab); its log-probability is NaN  */
#define LSAMP_ROW_TIMEOUT 16u    /* a one-pass top-k step's finalizer gave up
                                    waiting for a slice that had started
                                    (another workload held the CUs); token = -1
                                    (fail closed).  The sampling kernels' other
                                    arrangements never wait for a slice that
                                    has not started, and hand the work of a
                                    slice that gives up to the row's last
                                    arriver: their rows are never timed out */

/* ---- per-row inputs ------------------------------------------------------- */

/* Resolved sampling parameters of one row (32 bytes).  Build them with
 * lsamp_resolve_generate_parameters (mlx-lm) or lsamp_resolve_cbv2_params
 * (CBv2); both reproduce the reference's own resolution rules. */
typedef struct lsamp_row_params {
  int32_t kind;             /* lsamp_kind                                        */
  float temperature;        /* > 0 for FILTERED / CATEGORICAL rows               */
  int32_t top_k;            /* <= 0 or >= vocab: off                             */
  float top_p;              /* >= 1: off; CBv2 keeps the top token at 0          */
  float min_p;              /* <= 0: off                                         */
  float repetition_penalty; /* applied to entries flagged REPETITION; 1 = off   */
  float presence_penalty;   /* 0 = off                                           */
  float frequency_penalty;  /* 0 = off                                           */
} lsamp_row_params;

/* One sparse penalty / bias entry (16 bytes).  A row's entries are the
 * distinct token ids of its history (CSR rows `row_ptr[r] .. row_ptr[r+1]`);
 * a token id appears at most once per row and lies in [0, vocab).  This
 * replaces the dense [B, vocab] float32 count tensors that the reference keeps
 * (LogitsPipelineV2.swift:127-129) and the per-step scatter-add histogram of
 * FrequencyPenaltyContext (Evaluate.swift:649-658). */
typedef struct lsamp_penalty_entry {
  int32_t token;  /* vocabulary id                                            */
  int32_t count;  /* CBv2: occurrences in the output tokens (frequency and
                     presence, LogitsPipelineV2.swift:327-330); mlx-lm:
                     occurrences in the frequency window                      */
  uint32_t flags; /* LSAMP_PEN_*                                              */
  float bias;     /* CBv2 additive logit bias (LogitsPipelineV2.swift:317-319)  */
} lsamp_penalty_entry;

/* Optional per-row statistics (parity / logprobs / MTP).  48 bytes. */
typedef struct lsamp_row_stats {
  float max_value;       /* y_max: largest filter-space logit                    */
  float log_normalizer;  /* log sum exp(y - y_max) over unmasked tokens          */
  int32_t kept;          /* number of tokens that survive the filters            */
  int32_t token;         /* the drawn token (same as tokens[r])                  */
  uint64_t kept_weight;  /* W = sum of fixed-point weights of kept tokens        */
  uint64_t probe_weight; /* w of probe_tokens[r] (0 if not kept / no probe)      */
  float cut_value;       /* smallest kept filter-space logit                     */
  float kept_mass;       /* sum exp(y - y_max) over kept tokens                  */
  float kept_entropy;    /* Shannon entropy (nats) of the kept, renormalized row */
  float probe_prob;      /* kept_weight-normalized probability of the probe      */
} lsamp_row_stats;

/* ---- the sampling step ---------------------------------------------------- */
typedef struct lsamp_sample_args {
  int32_t semantics;  /* lsamp_semantics                                        */
  int32_t rows;       /* B                                                      */
  int32_t vocab;      /* V (logit dimension)                                    */
  int32_t dtype;      /* lsamp_dtype of `logits`                                */
  int64_t row_stride; /* elements between consecutive rows (>= vocab)           */
  const void* logits; /* [rows, row_stride]                                     */
  const lsamp_row_params* params; /* [rows]                                     */

  const int32_t* penalty_row_ptr;             /* [rows + 1] or NULL              */
  const lsamp_penalty_entry* penalty_entries; /* [penalty_row_ptr[rows]]         */

  const uint32_t* bitmask; /* [rows, mask_words] packed LSB-first, or NULL      */
  int32_t mask_words;      /* words per row (>= ceil(mask_bits / 32))           */
  int32_t mask_bits;       /* valid bits per row (tokenizer vocab size)         */
  int32_t mask_tail;       /* lsamp_mask_tail                                   */

  const float* uniforms;       /* [rows] in [0, 1), or NULL to use philox_keys */
  const uint64_t* philox_keys; /* [rows] Philox4x32-10 keys (lsamp_rng_key)     */

  const int32_t* probe_tokens; /* [rows] or NULL: report their kept weight      */

  int32_t* tokens;        /* [rows] out                                         */
  uint32_t* row_flags;    /* [rows] out or NULL                                 */
  float* processed;       /* [rows, vocab] out or NULL: filter-space logits
                             after penalties, temperature (CBv2) and mask,
                             before top-k/top-p/min-p (parity mode)            */
  uint8_t* keep;          /* [rows, vocab] out or NULL: 1 where the token
                             survives the filters (parity mode)               */
  lsamp_row_stats* stats; /* [rows] out or NULL                                 */

  /* [rows] or NULL: row r's entries are penalty_entries[penalty_row_ptr[r] ..
   * penalty_row_ptr[r] + penalty_row_len[r]) instead of .. penalty_row_ptr[r+1]
   * (a fixed-capacity table that lsamp_commit keeps up to date)             */
  const int32_t* penalty_row_len;

  /* [n_suppress] or NULL: token ids masked to -inf in every row, after the
   * penalties and the bitmask (SuppressTokensProcessor.process,
   * Libraries/MLXLMCommon/SuppressTokens.swift:67-81, chained last by
   * GenerationComponents.swift:126-141).  Any order; negative ids and ids >=
   * vocab are ignored, as the reference drops them.  Applied at the bitmask's
   * position in both semantics (both write -inf, so the order between them
   * does not change a value).                                               */
  const int32_t* suppress_ids;
  int32_t n_suppress; /* 0 .. LSAMP_MAX_SUPPRESS                             */

  /* [rows] HOST copy of `params`, or NULL.  Used only to choose the kernel
   * arrangement: when every row is an argmax row, or a CBv2 row whose top-k is
   * active and at most LSAMP_TOPK_MAX_K, the step runs the one-pass top-k
   * kernel (lsamp_launch_info.fused = 2).  It must describe `params`; a row
   * of `params` that the top-k kernel cannot sample comes back as token -1
   * with LSAMP_ROW_OVERFLOW. */
  const lsamp_row_params* params_host;
} lsamp_sample_args;

#define LSAMP_TOPK_MAX_K 64

#define LSAMP_MAX_SUPPRESS 65536

/* ---- MTP verification ----------------------------------------------------- */
typedef enum lsamp_verify_mode {
  /* Textbook speculative sampling (Leviathan et al. 2023; Chen et al. 2023):
   * accept draft j iff u[j] < min(1, p_t(x_j) / p_d(x_j)); on the first
   * rejection draw from normalize(max(0, p_t - p_d)) with u[W-1]; if every
   * draft is accepted draw the bonus token from the last target position.  */
  LSAMP_VERIFY_RESIDUAL = 0,
  /* Reference exact mode (DefaultSamplerV2.swift:378-380): the target token at
   * every position is drawn with u[j]; accept iff it equals the draft.      */
  LSAMP_VERIFY_EXACT = 1,
  /* Reference typical mode (DefaultSamplerV2.swift:485-502): same draws;
   * accept iff p_t(draft) > min(1, delta * exp(-H)); greedy rows exact.      */
  LSAMP_VERIFY_TYPICAL = 2
} lsamp_verify_mode;

typedef struct lsamp_verify_args {
  int32_t mode;      /* lsamp_verify_mode                                      */
  int32_t sequences; /* S                                                      */
  int32_t window;    /* W = drafts + 1                                         */
  int32_t vocab;     /* V                                                      */
  int32_t dtype;     /* lsamp_dtype of both logit tensors                      */
  const void* target_logits;  /* [S, W, V] contiguous                          */
  const void* draft_logits;   /* [S, W-1, V] contiguous (RESIDUAL mode only)   */
  const int32_t* draft_tokens;/* [S, W-1]                                      */
  const lsamp_row_params* params; /* [S] CBv2-resolved, one per sequence       */
  const float* uniforms;      /* [S, W]                                        */
  float typical_delta;        /* TYPICAL mode, > 0                             */
  int32_t* accepted;          /* [S] out: number of accepted drafts            */
  int32_t* tokens;            /* [S, W] out: RESIDUAL mode emits accepted drafts
                                 then the correction / bonus token, -1 after;
                                 EXACT / TYPICAL write the target draw at every
                                 position                                      */
  uint8_t* accept_mask;       /* [S, W-1] out or NULL: per-position decision   */

  /* Penalty-aware verification (CBv2DefaultSampler.applyWindowPenalties,
   * DefaultSamplerV2.swift:503-580), EXACT and TYPICAL modes; NULL entries =
   * none.  Each sequence's confirmed output counts as sparse entries (token,
   * count; flags and bias are ignored: the reference's verify applies only
   * frequency / presence), in penalty_entries[penalty_row_ptr[s] ..
   * + penalty_row_len[s]) (or .. penalty_row_ptr[s+1] when row_len is NULL).
   * Position j of sequence s also counts the drafts that precede it: chain
   * positions [0, column_offset + j) of penalty_drafts ([S, drafts_stride];
   * NULL = draft_tokens with column_offset 0), as CBv2MTPVerifyPenalties
   * describes them (EngineLoopV2.swift:226-244).                            */
  const int32_t* penalty_row_ptr;
  const int32_t* penalty_row_len;
  const lsamp_penalty_entry* penalty_entries;
  const int32_t* penalty_drafts;
  int32_t penalty_drafts_stride;
  int32_t penalty_column_offset;
  lsamp_penalty_entry* penalty_scratch; /* [S * W, penalty_scratch_cap] device */
  int32_t penalty_scratch_cap;          /* entries per position, >= the longest
                                           sequence run + column_offset + W - 1 */
} lsamp_verify_args;

/* ---- context ------------------------------------------------------------- */
typedef struct lsamp_context lsamp_context;

/* Allocates the device workspace for up to `max_rows` rows of up to
 * `max_vocab` logits on `device` (and for MTP verification of up to
 * max_rows target+draft rows).  The step functions allocate nothing.
 *
 * Every entry point that takes a context uses its workspace (arrival
 * counters, candidate lists, slice summaries, the suppress bitmask, the mask
 * staging pair), so calls on one context must be ordered on ONE stream: two
 * calls in flight on different streams with the same context race.  Use one
 * context per concurrent stream.  The reference's caller is single-threaded
 * for the same reason (one engine queue). */
lsamp_status lsamp_context_create(int32_t device, int32_t max_rows, int32_t max_vocab,
                                  lsamp_context** out);
void lsamp_context_destroy(lsamp_context* ctx);

/* Enqueue one sampling step on `stream`. */
lsamp_status lsamp_sample(lsamp_context* ctx, const lsamp_sample_args* args, void* stream);

/* ---- the sampling step without a context -----------------------------------
 * No counterpart in the reference: an entry point for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  lsamp_sample on the CURRENT device with its workspace in
 * a file-scope device array of LSAMP_NOALLOC_SCRATCH_BYTES (12 MiB, held by
 * each GPU the library runs on until the process ends) instead of a context:
 * at most LSAMP_NOALLOC_MAX_ROWS rows of at most LSAMP_NOALLOC_MAX_VOCAB logits
 * (larger calls return LSAMP_ERR_CAPACITY).  Same arguments, results and
 * errors as lsamp_sample in the AUTO arrangement; allocates nothing and calls
 * no allocating routine.  Every call on one GPU shares that GPU's array: a
 * call clears its counters first (a fill kernel, capturable), and calls that
 * overlap on one GPU (unordered streams) race. */
#define LSAMP_NOALLOC_MAX_ROWS 64
#define LSAMP_NOALLOC_MAX_VOCAB 262144
#define LSAMP_NOALLOC_SCRATCH_BYTES (12u << 20)
lsamp_status lsamp_sample_noalloc(const lsamp_sample_args* args, void* stream);

/* Per-kernel timing hook, off by default (the role CBv2StepProfiler plays for
 * the reference, StepProfilerV2.swift:15-60).  While enabled, each
 * lsamp_sample call that is not under graph capture records three HIP events
 * on its stream: before the first kernel, after it, and after the second
 * kernel of a split step (a fused step has one kernel: its second interval is
 * empty), up to 4096 calls.  lsamp_context_read_timing waits for them,
 * returns the summed milliseconds of the two intervals and the number of
 * timed calls, and starts a new window. */
lsamp_status lsamp_context_set_timing(lsamp_context* ctx, int32_t enable);
lsamp_status lsamp_context_read_timing(lsamp_context* ctx, double* stats_ms, double* select_ms,
                                       int64_t* calls);

/* Kernel arrangement.  AUTO (default) runs the one-pass top-k kernel when
 * `params_host` shows every row is argmax or CBv2 top-k <= LSAMP_TOPK_MAX_K
 * (each slice of a row publishes its best keys; the slice that starts last
 * merges and draws; no co-residency needed), else one kernel whose grid fits
 * on the device at once (the slices of a row hand their results to each
 * other while the logits stay in registers).  FUSED never takes the top-k
 * kernel; SPLIT runs two kernels with no co-residency requirement (the
 * second re-reads each slice from L2).  All give identical results. */
#define LSAMP_MODE_AUTO 0
#define LSAMP_MODE_FUSED 1
#define LSAMP_MODE_SPLIT 2
lsamp_status lsamp_context_set_mode(lsamp_context* ctx, int32_t mode);

/* Sticky device-side status bits raised since the last read (waits for the
 * device); clears them.  LSAMP_STATUS_SPIN_TIMEOUT: a bounded wait for a
 * row's other slices gave up (another workload held the CUs).  In a top-k
 * step the affected rows carry LSAMP_ROW_TIMEOUT and token -1 in the same
 * step's outputs; in a fused step the slice that gave up left its work to
 * the row's last arriver, and every row is exact. */
#define LSAMP_STATUS_SPIN_TIMEOUT 1u
/* a penalty-aware verify position had more entries than penalty_scratch_cap
 * (its outputs are unreliable) */
#define LSAMP_STATUS_PENALTY_CAPACITY 2u
lsamp_status lsamp_context_read_status(lsamp_context* ctx, uint32_t* bits);

/* (The test hook of the bounded waits is declared apart, in lsamp_testing.h.) */

/* Launch shape of the context's last lsamp_sample call (diagnostics; no
 * device work): fused with raw log-probabilities (4, lsamp_step), top-k with
 * raw log-probabilities (3, lsamp_step), top-k (2), fused (1) or split (0),
 * slices per row, tokens per slice, rows per round of the fused grid,
 * work-groups per kernel launch. */
typedef struct lsamp_launch_info {
  int32_t fused;
  int32_t slices;
  int32_t slice_len;
  int32_t rows_per_round;
  int32_t grid;
} lsamp_launch_info;
lsamp_status lsamp_context_last_launch(lsamp_context* ctx, lsamp_launch_info* out);

/* Enqueue one MTP verification on `stream`. */
lsamp_status lsamp_verify(lsamp_context* ctx, const lsamp_verify_args* args, void* stream);

/* ---- coupled MTP proposal ---------------------------------------------------
 * CBv2DefaultSampler.mtpCoupledProposal (DefaultSamplerV2.swift:310-374): the
 * draft position's token drawn with the randomness the verifier will draw
 * that position with, so a draft distribution close to the target's proposes
 * the token the target draws.  The reference races exponential noise over the
 * draft's tempered probabilities and falls back to the mode when the winner
 * is outside top-k / top-p / min-p; the verifier here draws by inverse CDF
 * from one uniform (lsamp.h, draw rule), so the coupled proposal is the
 * inverse-CDF draw from the draft's filtered distribution with the same
 * uniform (greedy rows: the argmax).  Stateless transforms only, as in the
 * reference: no penalties, no mask.  Any proposal leaves verification exact. */
typedef struct lsamp_propose_args {
  int32_t rows;       /* sequences                                              */
  int32_t vocab;
  int32_t dtype;      /* lsamp_dtype                                           */
  int64_t row_stride; /* elements between rows (>= vocab)                       */
  const void* logits; /* [rows, row_stride] draft logits of one chain position  */
  const lsamp_row_params* params; /* [rows] CBv2-resolved                        */
  const float* uniforms;          /* [rows] the uniforms the verifier draws this
                                     position with, or NULL to use philox_keys */
  const uint64_t* philox_keys;    /* [rows] lsamp_rng_key(seed, id, stepBase + j) */
  int32_t* tokens;                /* [rows] out                                 */
} lsamp_propose_args;

lsamp_status lsamp_propose(lsamp_context* ctx, const lsamp_propose_args* args, void* stream);

/* ---- ranking of raw logits: exact top-2 and log-probabilities -------------
 * Both calls read a row's logits once (one kernel) and order tokens as the
 * reference's shared top-2 reduction does (CBv2TopTwo.swift:29-47): value
 * descending, token id ascending on exact ties (+0 and -0 tie), NaN last.
 * Strides are in elements and may describe any view (rows may overlap). */
typedef struct lsamp_top2_args {
  int32_t rows;       /* >= 1, <= the context's max_rows                       */
  int32_t vocab;      /* >= 2                                                  */
  int32_t dtype;      /* lsamp_dtype                                           */
  int64_t row_stride; /* elements between rows (>= 0)                          */
  int64_t col_stride; /* elements between tokens (>= 1; 1 = contiguous)        */
  const void* logits;
  int32_t* ids;       /* [rows, 2] out                                         */
  float* values;      /* [rows, 2] out: the logits converted to float32
                         (exact; NaN stays NaN)                                */
} lsamp_top2_args;

/* cbv2TopTwoRows (CBv2TopTwo.swift:191-212): ids and values of the two best
 * tokens of every row. */
lsamp_status lsamp_top2(lsamp_context* ctx, const lsamp_top2_args* args, void* stream);

typedef struct lsamp_logprobs_args {
  int32_t rows;       /* >= 1, <= the context's max_rows                       */
  int32_t vocab;      /* >= 1                                                  */
  int32_t dtype;      /* lsamp_dtype                                           */
  int64_t row_stride; /* elements between rows (>= 0)                          */
  int64_t col_stride; /* elements between tokens (>= 1)                        */
  const void* logits; /* RAW logits: before bias, penalties, temperature, mask */
  int32_t top_k;      /* 0 .. 32, <= vocab                                     */
  const int32_t* tokens; /* [rows] the sampled tokens, or NULL                 */
  float* chosen;      /* [rows] out (required with tokens): logprob of tokens[r] */
  float* top_values;  /* [rows, top_k] out: the top_k log-probabilities       */
  int32_t* top_ids;   /* [rows, top_k] out: their token ids                    */
  uint32_t* row_flags;/* [rows] out or NULL: LSAMP_ROW_NONFINITE, _TOKEN_RANGE */
} lsamp_logprobs_args;

/* Log-probabilities of the raw logits, x - logsumexp(x) in float32
 * (LogitsPipelineV2.process :307-314, Evaluate.swift:800-806), gathered for
 * the sampled token and the top_k best tokens (CBv2Logprobs.gather,
 * LogitsPipelineV2.swift:534-549; DeferredTokenLogProbabilities,
 * Evaluate.swift:818-853).  A row with a NaN or +inf logit, or with every
 * logit -inf, has no finite log-sum-exp and defines no log-probabilities: it
 * fails closed with LSAMP_ROW_NONFINITE, top_ids -1 and NaN values and chosen
 * log-probability, as the reference fails a non-finite row
 * (CBv2NonFiniteLogits.swift:8-34).  A row holding -inf beside finite logits
 * is flagged NONFINITE and keeps its (finite or -inf) log-probabilities. */
lsamp_status lsamp_logprobs(lsamp_context* ctx, const lsamp_logprobs_args* args, void* stream);

/* ---- the mlx-lm penalty processor on its own ------------------------------
 * PenaltyProcessor.process (Evaluate.swift:687-693) as a separate pass, for a
 * processor chain in which another processor runs between the penalties and
 * the sampler (GenerationComponents.swift:112-141 composes penalty, then the
 * custom processor, then suppression).  lsamp_sample applies the same
 * penalties inside the sampling pass; use this entry point only when the
 * penalized logits themselves are needed. */
typedef struct lsamp_penalize_args {
  int32_t rows;       /* >= 1                                                  */
  int32_t vocab;      /* >= 1                                                  */
  int32_t dtype;      /* lsamp_dtype of logits                                 */
  int64_t row_stride; /* elements between logits rows (>= vocab)              */
  const void* logits; /* [rows, vocab] device                                  */
  const lsamp_row_params* params; /* [rows] device: repetition / presence /
                                     frequency penalties (mlx-lm semantics)   */
  const int32_t* penalty_row_ptr; /* [rows + 1] device (CSR), or the row starts
                                     with penalty_row_len                     */
  const int32_t* penalty_row_len; /* [rows] device or NULL                     */
  const lsamp_penalty_entry* penalty_entries;
  int32_t out_dtype;  /* the logits' dtype, or LSAMP_DTYPE_F32: MLX promotes
                         to float32 when a frequency penalty is on
                         (FrequencyPenaltyContext's float32 histogram,
                         Evaluate.swift:649-658)                              */
  void* out;          /* [rows, vocab] device, contiguous, out_dtype           */
} lsamp_penalize_args;

/* RepetitionContext, then PresencePenaltyContext in the logits' dtype with the
 * penalty rounded to it, then FrequencyPenaltyContext in float32
 * (Evaluate.swift:586-658), every other logit copied unchanged.  Entries
 * follow lsamp_sample's rules (LSAMP_PEN_REPETITION, LSAMP_PEN_PRESENCE,
 * count = occurrences in the frequency window). */
lsamp_status lsamp_penalize(lsamp_context* ctx, const lsamp_penalize_args* args, void* stream);

/* ---- device-side penalty state ---------------------------------------------
 * The incremental state of LogitsPipelineV2 (outputCounts, repWindow,
 * repWindowCounts, ringPos; LogitsPipelineV2.swift:127-141) kept on the device
 * as a fixed-capacity sparse table that lsamp_sample reads directly
 * (penalty_row_ptr[r] = r * capacity, penalty_row_len = row_len).  Entries
 * hold {token, output count, LSAMP_PEN_REPETITION while the token is in the
 * repetition window, logit bias}; build the initial table from the request's
 * prompt / output history on the host once. */
#define LSAMP_STATE_COUNTS 1u     /* frequency or presence penalty on           */
#define LSAMP_STATE_REPETITION 2u /* repetition penalty on: keep the window ring */

typedef struct lsamp_penalty_table {
  int32_t rows;
  int32_t capacity;        /* entry slots per row                              */
  int32_t window_capacity; /* ring slots per row (>= every window_size)        */
  lsamp_penalty_entry* entries; /* [rows, capacity]; slots [0, row_len[r]) used */
  int32_t* row_len;        /* [rows]                                           */
  int32_t* window_count;   /* [rows, capacity]: occurrences of the entry's token
                              in the repetition window                         */
  int32_t* window;         /* [rows, window_capacity]: the ring, -1 = empty     */
  int32_t* ring_pos;       /* [rows]: the slot the next token overwrites       */
  const int32_t* window_size; /* [rows]: W >= 1 (repetitionContextSize)        */
  const uint32_t* mode;    /* [rows]: LSAMP_STATE_* bits                        */
} lsamp_penalty_table;

typedef struct lsamp_commit_args {
  lsamp_penalty_table table;
  int32_t vocab;
  const int32_t* tokens; /* [rows] the sampled tokens; ids outside [0, vocab)
                            (an EMPTY row's -1) commit nothing               */
  uint32_t* row_flags;   /* [rows] out or NULL: LSAMP_ROW_OVERFLOW when a new
                            entry did not fit in the row's capacity          */
} lsamp_commit_args;

/* LogitsPipelineV2.commit (LogitsPipelineV2.swift:357-384) for every row, on
 * the device: the sampled token's output count += 1 (COUNTS rows); the
 * repetition ring evicts the token at ring_pos (its window count -= 1, the
 * REPETITION flag cleared at 0) and takes the sampled token (window count
 * += 1, flag set), ring_pos = (ring_pos + 1) % W (REPETITION rows).  Entries
 * that end with no count, flag or bias are removed (the last entry of the
 * row takes the slot). */
lsamp_status lsamp_commit(lsamp_context* ctx, const lsamp_commit_args* args, void* stream);

/* ---- one decode step ----------------------------------------------------------
 * CBv2DefaultSampler.sample (DefaultSamplerV2.swift:84-181) as one call: the
 * draw (lsamp_sample), then the penalty commit of the drawn tokens into the
 * device table (lsamp_commit, :162), and the log-probabilities of the RAW
 * logits for the drawn tokens and the top k (lsamp_logprobs, :167-176), all
 * enqueued on `stream`.  The kernel that draws writes the log-probabilities
 * in the same pass over the logits: the one-pass top-k kernel (AUTO mode,
 * 16-bit logits, `sample.params_host` showing argmax or CBv2 top-k <=
 * LSAMP_TOPK_MAX_K rows; launch info `fused` = 3) or the fused sampling
 * kernel (every other step that fits its grid, fp32 included, fp32 top-k
 * batches too; `fused` = 4).  Only a step that runs the split kernels (an
 * fp32 batch larger than one round of the fused grid, or LSAMP_MODE_SPLIT)
 * takes a second pass (lsamp_logprobs).  Ids are the same either way and
 * values agree to float rounding of the log-sum-exp.  Graph-capturable like
 * its parts. */
typedef struct lsamp_step_args {
  lsamp_sample_args sample;          /* the draw; its penalty arguments usually
                                        point at `table` (row_ptr[r] = r * capacity,
                                        entries, row_len)                        */
  const lsamp_penalty_table* table;  /* or NULL: no commit                      */
  uint32_t* commit_flags;            /* [rows] or NULL: LSAMP_ROW_OVERFLOW        */
  int32_t logprobs_top_k;            /* -1: no log-probabilities; else 0 .. 32    */
  float* chosen_logprob;             /* [rows] (logprobs_top_k >= 0)             */
  float* top_logprobs;               /* [rows, logprobs_top_k]                   */
  int32_t* top_ids;                  /* [rows, logprobs_top_k]                   */
} lsamp_step_args;

lsamp_status lsamp_step(lsamp_context* ctx, const lsamp_step_args* args, void* stream);

/* ---- grammar masks: cached rows and the step's bitmask ---------------------
 * Replaces CBv2TokenConstraintSampler.mask (TokenConstraintSamplerV2.swift:
 * 131-182) and its deviceMask / open rows (:187-199): the reference builds a
 * [1, vocab] bool row per constrained request from its allowed ids (O(vocab)
 * host work and upload), keeps up to 8 per request in an LRU, and concatenates
 * the rows of a step.  Here a row's mask is a packed LSB-first bitmask row
 * ((vocab + 31) / 32 words, the lsamp_sample bitmask layout) in a device pool
 * the caller owns; one call assembles the step's [rows, words] bitmask:
 *   row_source[r] = -1  an open row (every token allowed: all bits set);
 *   row_source[r] = s   pool row s, built first from the row's allowed ids
 *                       when row_build[r] != 0 (a cache miss), else as cached.
 * A build with an id outside [0, vocab) yields an all-zero row (every logit
 * -inf, deviceMask :189-191) and sets LSAMP_MASK_ID_RANGE in row_flags.  The
 * impossible-state fallback (empty or out-of-range allowed ids -> the
 * fallback id, :160-163) is the caller's rule, made before the call.
 *
 * The descriptors (row_source, row_build, ids_ptr, ids) are HOST arrays.  The
 * call packs them into one of two pinned staging buffers the context owns,
 * copies it to the device on `stream` and launches the assembly, so the host
 * prepares step N+1's ids while step N's copy runs; it blocks only when the
 * copied or read.  A step with no builds and at most 256 rows skips the
 * staging: its pool rows travel in the kernel arguments.  Unlike the other
 * entry points it allocates: the staging
 * pair on first use and again when the descriptors outgrow it (after waiting
 * for both buffers).  Not capturable in a HIP graph (host staging).  A pool
 * row built by a call must not be read by another row of the same call. */
#define LSAMP_MASK_ID_RANGE 1u
#define LSAMP_MASK_MAX_WORDS 16000 /* vocab <= 512,000 (the row sits in LDS) */

typedef struct lsamp_mask_assemble_args {
  int32_t rows;
  int32_t vocab;
  int32_t words;              /* (vocab + 31) / 32                               */
  int32_t pool_rows;
  uint32_t* pool;             /* [pool_rows, words] device, caller-owned cache     */
  uint32_t* out;              /* [rows, words] device: the step's bitmask          */
  uint32_t* row_flags;        /* [rows] device out or NULL                         */
  const int32_t* row_source;  /* [rows] host: -1 open, else a pool row             */
  const uint8_t* row_build;   /* [rows] host: 1 = build the pool row from ids      */
  const int32_t* ids_ptr;     /* [rows + 1] host offsets into ids (build rows)     */
  const int32_t* ids;         /* [ids_ptr[rows]] host: allowed ids, any order      */
} lsamp_mask_assemble_args;

lsamp_status lsamp_mask_assemble(lsamp_context* ctx, const lsamp_mask_assemble_args* args,
                                 void* stream);

/* ---- host-side parameter resolution (no device work) ---------------------- */

/* GenerateParameters subset that drives the mlx-lm sampler/processor factory
 * (Evaluate.swift:127-289; defaults T=0.6, top-p 1, top-k 0, min-p 0,
 * context sizes 20).  `has_*` = 0 reproduces a nil optional. */
typedef struct lsamp_generate_parameters {
  float temperature;
  float top_p;
  int32_t top_k;
  float min_p;
  int32_t has_repetition_penalty;
  float repetition_penalty;
  int32_t repetition_context_size;
  int32_t has_presence_penalty;
  float presence_penalty;
  int32_t presence_context_size;
  int32_t has_frequency_penalty;
  float frequency_penalty;
  int32_t frequency_context_size;
} lsamp_generate_parameters;

/* GenerateParameters.sampler() / .processor() (Evaluate.swift:328-387).
 * Writes the resolved row, and in `*contexts` a bit set of the penalty
 * contexts the reference would build (1 repetition, 2 presence, 4 frequency;
 * 0 = processor() returns nil). */
lsamp_status lsamp_resolve_generate_parameters(const lsamp_generate_parameters* gp,
                                               lsamp_row_params* out, int32_t* contexts);

/* CBv2SamplingParams subset (CBv2Contracts.swift:37-75; defaults T=1,
 * repetition window 64). */
typedef struct lsamp_cbv2_params {
  float temperature;
  float top_p;
  int32_t top_k;
  float min_p;
  float repetition_penalty;
  int32_t repetition_context_size;
  float frequency_penalty;
  float presence_penalty;
} lsamp_cbv2_params;

/* LogitsPipelineV2.setRows resolution (LogitsPipelineV2.swift:188-227):
 * greedy iff T < 1e-5; top-k off unless 0 < k < vocab; top-p off (2.0) unless
 * 0 < p < 1, p <= 0 keeps the top token; min-p clamped to 1; repetition only
 * when p != 1 and the window is positive. */
lsamp_status lsamp_resolve_cbv2_params(const lsamp_cbv2_params* sp, int32_t vocab,
                                       lsamp_row_params* out);

/* SamplerV2.mix (SamplerV2.swift:183-191): SplitMix64 of (seed, id, step). */
uint64_t lsamp_rng_key(uint64_t seed, uint64_t request_id, uint64_t step);

/* The uniform the kernels draw for `key` when `uniforms` is NULL:
 * Philox4x32-10 (Salmon et al., SC'11) of counter {purpose, 0, 0, 0} and key
 * {lo32(key), hi32(key)}; u = (x0 >> 8) * 2^-24.  purpose 0 = token draw. */
float lsamp_rng_uniform(uint64_t key, uint32_t purpose);

/* ---- diagnostics ----------------------------------------------------------- */
const char* lsamp_last_error(void);
const char* lsamp_version(void);
/* sizeof of an ABI struct by name ("lsamp_row_params", ...), -1 if unknown;
 * lets bindings in other languages verify their layouts. */
int64_t lsamp_abi_sizeof(const char* type_name);

#ifdef __cplusplus
}
#endif

#endif /* LSAMP_H */
