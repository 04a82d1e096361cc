// lsamp_internal.h — device workspace layout and launch plan shared by the
// kernels (lsamp_kernels.hip) and the C ABI (lsamp_api.cpp).
#pragma once

#include <stdint.h>

#include "../../include/lsamp.h"

namespace lsamp {

// Work-group shape: one 512-thread work-group (8 wave64s, up to 256 VGPRs per
// lane) owns one slice of one row and holds the slice's logits in registers,
// 128 per thread at most (two 32-dword banks of 16-bit logits, four of fp32).
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kElemsPerThread = 128;
constexpr int kMaxSliceLen = kThreads * kElemsPerThread;  // 65536 tokens
constexpr int kChunk = 1024;                              // draw granularity (tokens)
constexpr int kMaxSlices = 8;                             // slices per row
constexpr int kMaxVocab = kMaxSlices * kMaxSliceLen;      // 524288
constexpr int kMaxRowChunks = kMaxVocab / kChunk;         // 512 <= one per thread
constexpr int kSliceChunks = kMaxSliceLen / kChunk;       // 64
// Histogram: bins of 1/32 nat of the filter-space logit, kBins of them below
// the slice's top bin (a 32-nat window), plus one tail bin for the rest.
constexpr int kBins = 1024;
constexpr int kTail = kBins;
constexpr int kHist = kBins + 1;
// Packed histogram word of a slice: count in bits 46..63, fixed-point mass in
// 0..45 (mass = sum exp(q - bin edge) * 2^29 <= 65536 * e^(1/32) * 2^29 < 2^46).
constexpr int kCountShift = 46;
constexpr uint64_t kMassMask = (1ull << kCountShift) - 1;
constexpr int kMassFracBits = 29;
// Candidates (tokens in the cut bin) per row, and per work-group in LDS.
constexpr int kCandCap = 4096;
constexpr int kWgCandCap = 2048;
// MTP verify residual draw: a work-group covers a part of kVerifyPart tokens
// of the rejected position's rows, a wave kVerifySpan of them.
constexpr int kVerifySpan = 2048;
constexpr int kVerifyPart = kWaves * kVerifySpan;  // 16,384
static_assert(kVerifySpan <= 65536, "queue entries are 16-bit offsets");
// Wave spans of a maximum-vocabulary row.
constexpr int kMaxVerifySpans = (kMaxVocab + kVerifyPart - 1) / kVerifyPart * kWaves;
// Short-list rows (argmax, or top-k <= kShortMaxK): each slice lists the
// tokens at or above a threshold taken from its threads' maxima (the quads
// holding them staged whole in LDS, at most kQStage per thread) and
// publishes them all (at most kShortPub, which the row's candidate area
// holds for every slice).
constexpr int kShortMaxK = 256;
constexpr int kQStage = 4;
constexpr int kShortPub = kCandCap / kMaxSlices;  // 512
constexpr int kTauBins = 1024;                    // thread-maximum histogram
// Kept tokens listed per slice (fast draw path); beyond this the draw scans.
constexpr int kKeptCap = 256;
// Penalty entries handled per slice (LDS).
constexpr int kSliceEntryCap = 2048;
// Fixed-point draw weights: 2^40 * dexp(d).
constexpr float kWeightScale = 1099511627776.0f;

// Cut position of a row (index into the row histogram, 0 = top bin).
constexpr int32_t kCutTail = kBins;      // cut inside the tail bin
constexpr int32_t kCutNone = kBins + 1;  // no filter cuts: every token kept
constexpr int32_t kCutList = kBins + 2;  // short-list row: kept iff in the kept list

// Row modes decided by the stats merge.
constexpr int32_t kModeNormal = 0;
constexpr int32_t kModeEmpty = 1;   // every logit masked / NaN
constexpr int32_t kModePosInf = 2;  // +inf logits present: keep exactly those

// Slice flags.
constexpr uint32_t kSlicePosInf = 0x100u;
constexpr uint32_t kSliceEntryOverflow = 0x200u;
constexpr uint32_t kSliceShortOverflow = 0x400u;  // short list did not fit
// Slice flags that send a short-list row down the histogram path.
constexpr uint32_t kSliceNoShort = kSlicePosInf | kSliceEntryOverflow | kSliceShortOverflow;

// Per-slice summary written by the stats phase.
struct SliceSummary {
  float x_max;       // largest finite transformed logit (pre-temperature)
  int32_t top_bin;   // bin of x_max
  uint32_t flags;    // LSAMP_ROW_NONFINITE | kSlice*
  int32_t n_finite;  // histogram token count; without a histogram, 1 when the
                     // slice holds a finite (or +inf) transformed logit
  double z;          // histogram mass relative to the top edge of bin top_bin
  double zs;         // short-list rows: sum exp((x - x_max) / T_f) over the slice
  int32_t npub;      // short-list rows: published keys (top-k plus ties)
  float ylo;         // short-list rows: no published key's value is below it
  uint64_t hist[kHist];
};

// Per-row decision of the stats merge.
struct RowInfo {
  float x_max;          // row max (pre-temperature space)
  float q_top;          // fast filter-space max that the masses are relative to
  int32_t top_bin;      // absolute bin of x_max
  int32_t cut;          // kCut* or bin index relative to top_bin
  int32_t mode;         // kMode*
  uint32_t flags;       // LSAMP_ROW_* accumulated so far
  int32_t count_above;  // tokens in bins above the cut
  int32_t n_finite;
  double mass_above;    // sum exp(q - q_top) of bins above the cut
  double z;             // sum exp(q - q_top) over every finite token
  double p_limit;       // top-p comparison bound (top_p * z), < 0 if off
  int32_t kept_cands;   // select finalize: kept candidates, listed first in cands[row]
  int32_t done;         // split mode: the stats kernel already drew this row's token
};

// Per-slice partial results of the select phase.
struct SelectPartial {
  double ent;        // sum over kept tokens of e * d (entropy numerator)
  float min_kept;    // smallest kept filter-space logit
  int32_t n_kept;
  int32_t n_cand;    // candidates this slice produced
  int32_t n_list;    // kept tokens listed (> kKeptCap: list incomplete)
  int32_t overflow;  // entry-table overflow in this slice
};

struct Candidate {
  float y;     // filter-space logit (exact)
  int32_t id;  // token id
};

struct KeptItem {
  uint64_t w;  // fixed-point draw weight
  int32_t id;
  int32_t pad;
};

static_assert(kMaxRowChunks <= kThreads, "the draw keeps one chunk per thread");
static_assert(kBins == 2 * kThreads, "the merge keeps two bins per thread");

// Ranking of raw logits (exact top-k and log-probabilities).  One 512-thread
// work-group per slice of a row; a slice is 16,384 / 32,768 / 65,536 tokens
// (option 0 / 1 / 2, whatever the dtype: 32 / 64 / 128 tokens per thread).
constexpr int kRankMaxK = 32;
constexpr int kRankMaxSlices = 16;
constexpr int kRankOptions = 3;
constexpr int rank_slice_len(int option) { return 16384 << option; }
// Slice flags of the ranking.
constexpr uint32_t kRankNaN = 1u;        // a NaN logit
constexpr uint32_t kRankPosInf = 2u;     // a +inf logit
constexpr uint32_t kRankNonfinite = 4u;  // a NaN or +-inf logit

// Per-slice result of the ranking: the slice's k largest sort keys (value
// descending, then token id ascending, NaN last), 0 past the slice's own
// tokens, and its log-sum-exp partial.
struct RankSlice {
  uint64_t top[kRankMaxK];
  double s;           // sum exp(x - m) over the slice's finite logits (m finite)
  float m;            // largest non-NaN logit of the slice (-inf if none)
  uint32_t flags;     // kRank*
  uint32_t tok_bits;  // the logit bits of the row's chosen token, if this slice holds it
  int32_t pad;
};

// A wave span's sums of the residual draw's two weights.
struct VerifySpan {
  uint64_t res;  // max(0, p_t - p_d) at 2^-52
  uint64_t tgt;  // the target's kept weight
};

constexpr int kRowSyncWords = 4;  // per-row synchronisation words of the sampling kernels
struct Workspace {
  int32_t max_rows;
  int32_t max_vocab;
  int32_t max_chunks;
  int32_t max_parts;        // verify parts per sequence (kVerifyPart tokens each)
  SliceSummary* summaries;  // [max_rows][kMaxSlices]
  RowInfo* rows;            // [max_rows]
  uint64_t* chunk_w;        // [max_rows][max_chunks]
  Candidate* cands;         // [max_rows][kCandCap]
  KeptItem* klist;          // [max_rows][kMaxSlices][kKeptCap]
  SelectPartial* partials;  // [max_rows][kMaxSlices]
  uint32_t* cand_count;     // [max_rows]
  uint32_t* arrive_stats;   // [max_rows][kRowSyncWords]: split mode's stats arrivals (word 0);
                            // the fused arrangement's arrivals, start tickets, claims, departures
  uint32_t* arrive_select;  // [max_rows]
  uint32_t* status;         // [1] sticky error bits (kStatus*)
  uint32_t* tasks;          // [1] fused kernel over several rounds: tasks taken
  // MTP verification: the sampled rows' outputs
  lsamp_row_stats* vstats;  // [max_rows]
  int32_t* vtokens;         // [max_rows]
  uint32_t* vflags;         // [max_rows]
  VerifySpan* vspan;        // [max_rows][max_parts][kWaves] per sequence
  uint32_t* vticket;        // [max_rows] per sequence: parts done (zeroed range)
};

// The one-pass top-k kernel (lsamp_topk.hip) takes steps whose rows are all
// argmax rows or CBv2 rows with 0 < top-k <= kTopkMaxK.  Each row has a
// ticket counter (taken when a slice starts; the slice with the last ticket
// finalizes the row and returns the counter to zero), an epoch (the tag of
// the step's payload words; the finalizer advances it) and, per slice, a
// payload of tagged 64-bit words: tag (epoch + 1) in the high half, data in
// the low half, so every word shows on its own whether it is this step's.
constexpr int kTopkMaxK = 64;
constexpr int kTopkMaxLp = 32;                     // raw log-probabilities per row
static_assert(kTopkMaxLp == kRankMaxK, "lsamp_step's log-prob limit either way");
constexpr int kTopkHead = 8;                       // header words per slice
constexpr int kTopkWordsBase = kTopkHead + 2 * kTopkMaxK;  // + (value, id) per key
// + (value, id) per raw key, written when the step also asks for raw
// log-probabilities (the payload stride is the larger size either way)
constexpr int kTopkRawWords = 2 * kTopkMaxLp;
constexpr int kTopkWords = kTopkWordsBase + kTopkRawWords;
// A slice's record of the fused sampling kernel's in-pass raw
// log-probabilities (FusedLp, below): its largest non-NaN raw logit, NaN /
// +inf flags, the sum of exp(x - max) over its raw logits, and its best
// raw keys in order.
struct RawRecord {
  float max;
  uint32_t flags;
  int32_t n;  // keys
  int32_t pad;
  double z;
  uint64_t keys[kTopkMaxLp];
};

struct TopkWs {
  uint64_t* pub;     // [max_rows][kMaxSlices][kTopkWords]
  uint32_t* ticket;  // [max_rows]
  uint32_t* epoch;   // [max_rows]
  uint32_t* status;  // the workspace's sticky status word
};

// Byte layout of a workspace for max_rows rows of up to max_vocab logits:
// offsets from its base, every part 256-byte aligned.  The words that must
// start at zero (the status word, candidate counts, arrival counters) form
// the one range [zero_begin, zero_end); the kernels return them to zero at
// the end of every step.
struct WorkspaceLayout {
  size_t sum, rows, chunk, cand, klist, part, status, tasks, cc, as, asel, tticket, vtick;
  size_t vstats, vtok, vfl, vspan, rpart, arank, vrp, vrl, smask, tpub, tepoch, rawrec;
  size_t zero_begin, zero_end, total;
};
constexpr size_t align256(size_t v) { return (v + 255) / 256 * 256; }
constexpr size_t verify_parts(size_t vocab) { return (vocab + kVerifyPart - 1) / kVerifyPart; }
constexpr WorkspaceLayout workspace_layout(size_t R, size_t max_vocab) {
  const size_t chunks = (max_vocab + kChunk - 1) / kChunk;
  const size_t words = (max_vocab + 31) / 32;
  WorkspaceLayout L{};
  size_t off = 0;
  L.sum = off;    off = align256(off + R * kMaxSlices * sizeof(SliceSummary));
  L.rows = off;   off = align256(off + R * sizeof(RowInfo));
  L.chunk = off;  off = align256(off + R * chunks * sizeof(uint64_t));
  L.cand = off;   off = align256(off + R * kCandCap * sizeof(Candidate));
  L.klist = off;  off = align256(off + R * kMaxSlices * kKeptCap * sizeof(KeptItem));
  L.part = off;   off = align256(off + R * kMaxSlices * sizeof(SelectPartial));
  L.zero_begin = off;
  L.status = off; off = align256(off + sizeof(uint32_t));
  L.tasks = off;  off = align256(off + sizeof(uint32_t));
  L.cc = off;     off = align256(off + R * sizeof(uint32_t));
  L.as = off;     off = align256(off + R * kRowSyncWords * sizeof(uint32_t));
  L.asel = off;   off = align256(off + R * sizeof(uint32_t));
  L.tticket = off; off = align256(off + R * sizeof(uint32_t));
  L.vtick = off;  off = align256(off + R * sizeof(uint32_t));
  L.zero_end = off;
  L.vstats = off; off = align256(off + R * sizeof(lsamp_row_stats));
  L.vtok = off;   off = align256(off + R * sizeof(int32_t));
  L.vfl = off;    off = align256(off + R * sizeof(uint32_t));
  L.vspan = off;  off = align256(off + R * verify_parts(max_vocab) * kWaves * sizeof(VerifySpan));
  L.rpart = off;  off = align256(off + R * kRankMaxSlices * sizeof(RankSlice));
  L.arank = off;  off = align256(off + R * sizeof(uint32_t));
  L.vrp = off;    off = align256(off + R * sizeof(int32_t));
  L.vrl = off;    off = align256(off + R * sizeof(int32_t));
  L.smask = off;  off = align256(off + R * words * sizeof(uint32_t));
  // (the epochs are outside the zeroed range: a payload word left by an
  // earlier step must never carry the current step's tag)
  L.tpub = off;   off = align256(off + R * kMaxSlices * kTopkWords * sizeof(uint64_t));
  L.tepoch = off; off = align256(off + R * sizeof(uint32_t));
  L.rawrec = off; off = align256(off + R * kMaxSlices * sizeof(RawRecord));
  L.total = off;
  return L;
}

struct RankPlan {
  int32_t rows;
  int32_t vocab;
  int32_t dtype;
  int32_t k;           // keys reported per row (0..kRankMaxK)
  int64_t row_stride;  // elements between rows
  int64_t col_stride;  // elements between tokens
  int32_t slices;      // per row
  int32_t option;      // slice option (rank_slice_len)
  int32_t vec;         // 16-byte vector loads (col_stride 1, aligned rows)
  int32_t lse;         // compute the log-sum-exp
  int32_t raw_values;  // values = raw logits (else log-probabilities)
  const void* logits;
  const int32_t* tokens;  // chosen token per row (NULL: no chosen output)
  float* chosen;          // [rows]
  float* values;          // [rows, k]
  int32_t* ids;           // [rows, k]
  uint32_t* row_flags;    // [rows] or NULL
  // the context's ranking workspace
  RankSlice* part;        // [max_rows][kRankMaxSlices]
  uint32_t* arrive;       // [max_rows]
};

// Sticky device status bits.
constexpr uint32_t kStatusSpinTimeout = 1u;  // a fused-kernel barrier wait timed out
// Test hook of the fused kernel's bounded waits (set by lsamp_test_set_spin_limit):
// 0 = normal; n > 0 = every wait's target is unreachable and it gives up after
// n polls, so the fail-closed path runs while every kernel still exits.
int set_spin_test(int32_t polls);
int set_topk_spin_test(int32_t polls);  // the same hook for the top-k kernel's finalizer
constexpr uint32_t kStatusPenaltyCapacity = 2u;  // a verify position's entries did not fit

// Launch description resolved on the host.
struct SamplePlan {
  int32_t semantics;
  int32_t rows;
  int32_t vocab;
  int32_t dtype;
  int64_t row_stride;
  int32_t slices;          // G
  int32_t slice_len;       // tokens per slice (multiple of kChunk)
  int32_t nchunks;
  int32_t aligned;         // 16-byte vector loads allowed
  int32_t fused;           // one co-resident kernel (1) or two kernels (0)
  int32_t rows_per_round;  // fused: rows processed per round of the grid
  const void* logits;
  const void* logits2;     // rows >= rows_split read logits2 (MTP draft rows)
  int32_t rows_split;
  // MTP verification layout (vwin = 0: a plain sampling step).  Rows below
  // rows_split are target positions (s, j), row = s * vwin + j; the others
  // are draft positions (s, j), row - rows_split = s * (vwin - 1) + j.  Each
  // row uses params[s], the uniform [s, j] of a [S, vwin] array, and probes
  // the draft token [s, j] of a [S, vwin - 1] array (none at j = vwin - 1).
  int32_t vwin;
  // MTP verify in RESIDUAL mode: only the last target position's draw is
  // read (the bonus token); the other rows report their weights, no token
  int32_t bonus_only;
  const lsamp_row_params* params;
  const int32_t* row_ptr;
  const int32_t* row_len;  // or NULL: rows end at row_ptr[row + 1]
  const lsamp_penalty_entry* entries;
  const uint32_t* bitmask;
  int32_t mask_words;
  int32_t mask_bits;
  int32_t mask_tail;
  int32_t stats_full;      // kept count, cut value and entropy wanted in stats
  const float* uniforms;
  const uint64_t* philox_keys;
  const int32_t* probe_tokens;
  int32_t* tokens;
  uint32_t* row_flags;
  float* processed;
  uint8_t* keep;
  lsamp_row_stats* stats;
};

// MTP verification outcome computation (after the sampling launch).
struct VerifyPlan {
  int32_t mode;        // lsamp_verify_mode
  int32_t sequences;   // S
  int32_t window;      // W
  int32_t vocab;
  int32_t dtype;
  int32_t semantics;   // LSAMP_SEM_CBV2
  float typical_delta;
  const void* target;  // [S, W, V]
  const void* draft;   // [S, W-1, V]
  const int32_t* draft_tokens;
  const lsamp_row_params* params;
  const float* uniforms;
  int32_t* accepted;
  int32_t* tokens;
  uint8_t* accept_mask;
  int32_t penalized;   // penalty-aware call: rows with a penalty accept exactly
  int32_t parts;       // work-groups per sequence (RESIDUAL: verify_parts(vocab))
};

// The one-pass top-k kernel over a plan whose rows all qualify (see TopkWs);
// `events` as launch_sample's.  Returns a hipError_t as int.
// Raw log-probabilities the top-k kernel can write in the same pass over the
// logits (lsamp_step's log-prob outputs; LogitsPipelineV2.process :307-314
// with CBv2Logprobs.gather :534-549): the chosen token's x - logsumexp(x) and
// the k best tokens' by the raw order (value descending, lower id on ties,
// NaN last).  k < 0: none.
struct TopkLp {
  int32_t k;       // -1, or 0 .. kTopkMaxLp
  float* chosen;   // [rows]
  float* values;   // [rows, k]
  int32_t* ids;    // [rows, k]
};
int launch_topk(const SamplePlan& plan, const TopkWs& tw, const TopkLp& lp, void* stream,
                void* const* events);

// Raw log-probabilities in the fused sampling kernel's own pass over the
// logits (lsamp_step): each slice publishes a record before its first
// exchange (its largest non-NaN raw logit, the sum of exp(x - max) over its
// raw logits, NaN / +inf flags, and its k best raw keys in order), and the
// row's finalizer merges the records once the token is drawn.
struct FusedLp {
  int32_t k;        // -1: none; else 0 .. kTopkMaxLp
  float* chosen;    // [rows]
  float* values;    // [rows, k]
  int32_t* ids;     // [rows, k]
  RawRecord* rec;   // [max_rows][kMaxSlices] (in the workspace)
};
// Work-groups of the top-k kernel that fit on one CU.
int topk_blocks_per_cu(int dtype);

// Kernel launchers (lsamp_kernels.hip).  Return a hipError_t as int.
// `events` (3 hipEvent_t or NULL) bracket the step: before, between the two
// kernels (split mode; same as before in fused mode), after.
// `lp` (or NULL): raw log-probabilities in the same pass (fused steps only).
int launch_sample(const Workspace& ws, const SamplePlan& plan, const FusedLp* lp, void* stream,
                  void* const* events);
// Work-groups of the fused kernel that fit on one CU (occupancy query).
int fused_blocks_per_cu(int dtype);
// Acceptance, residual / bonus draws and outputs of an MTP verification whose
// rows were sampled by launch_sample into ws.v* (one work-group per sequence).
int launch_verify_finish(const Workspace& ws, const VerifyPlan& plan, void* stream);
// Exact top-k of raw logits and their log-probabilities (lsamp_rank.hip).
int launch_rank(const RankPlan& plan, void* stream);
// Incremental penalty-state update after a draw (lsamp_commit.hip).
int launch_commit(const lsamp_commit_args& args, void* stream);

// lsamp_penalize (lsamp_penalize.hip): the mlx-lm penalty processor's output.
struct PenalizePlan {
  int32_t rows;
  int32_t vocab;
  int32_t dtype;
  int32_t out_dtype;
  int64_t row_stride;
  const void* logits;
  const lsamp_row_params* params;
  const int32_t* row_ptr;
  const int32_t* row_len;
  const lsamp_penalty_entry* entries;
  void* out;
};
int launch_penalize(const PenalizePlan& plan, void* stream);

// Per-position penalty entries of a penalty-aware verify window: row s * W + j
// = sequence s's confirmed counts plus the drafts before chain position
// column_offset + j (lsamp_commit.hip).
struct WindowEntriesPlan {
  int32_t sequences;
  int32_t window;
  int32_t vocab;
  int32_t cap;            // entries per position in `out`
  int32_t column_offset;
  int32_t drafts_stride;
  const int32_t* row_ptr;
  const int32_t* row_len;  // or NULL
  const lsamp_penalty_entry* entries;
  const int32_t* drafts;   // [S, drafts_stride]
  lsamp_penalty_entry* out;  // [S * W, cap]
  int32_t* out_ptr;        // [S * W]
  int32_t* out_len;        // [S * W]
  uint32_t* status;        // sticky status bits
};
int launch_window_entries(const WindowEntriesPlan& plan, void* stream);

constexpr int kMaskInlineRows = 256;

// Grammar bitmask assembly (lsamp_mask_assemble).  The descriptor arrays are
// device copies of the caller's host arrays; vec: words % 4 == 0 and the pool
// and output 16-byte aligned (cached and open rows copy whole vectors).
struct MaskAssemblePlan {
  int32_t rows;
  int32_t vocab;
  int32_t words;
  int32_t vec;
  uint32_t* pool;
  uint32_t* out;
  uint32_t* row_flags;
  const int32_t* row_source;
  const uint8_t* row_build;
  const int32_t* ids_ptr;
  const int32_t* ids;
  // a step with no builds and at most kMaskInlineRows rows carries its pool
  // rows here (no descriptor copy); inline_rows = 0 otherwise
  int32_t inline_rows;
  int32_t src_inline[kMaskInlineRows];
};
int launch_mask_assemble(const MaskAssemblePlan& plan, void* stream);

// Suppressed ids folded into a step's bitmask: out[r] = the caller's row r
// (its tail policy resolved; all ones without a bitmask) with the bits of the
// suppressed ids cleared, over (vocab + 31) / 32 words per row.
struct SuppressPlan {
  int32_t rows;
  int32_t vocab;
  int32_t words;            // (vocab + 31) / 32
  const uint32_t* bitmask;  // caller's [rows, mask_words] or NULL
  int32_t mask_words;
  int32_t mask_bits;
  int32_t mask_tail;
  const int32_t* ids;       // [n]
  int32_t n;
  uint32_t* out;            // [rows, words]
};
int launch_suppress_mask(const SuppressPlan& plan, void* stream);

// Device views of a workspace laid out by workspace_layout at `base`.
struct WorkspaceViews {
  Workspace ws;
  RankSlice* rank_part;   // [max_rows][kRankMaxSlices]
  uint32_t* arrive_rank;  // [max_rows]
  int32_t* vrow_ptr;      // [max_rows] penalty-aware verify: per-position runs
  int32_t* vrow_len;      // [max_rows]
  uint32_t* smask;        // [max_rows][smask_words]: bitmask with suppressed ids
  int32_t smask_words;
  TopkWs topk;            // the one-pass top-k kernel's exchange
  RawRecord* rawrec;      // [max_rows][kMaxSlices]: in-pass raw log-probability records
  char* zero_begin;       // the words that must start at zero
  size_t zero_bytes;
};
inline WorkspaceViews bind_workspace(char* b, int32_t max_rows, int32_t max_vocab) {
  const WorkspaceLayout L = workspace_layout((size_t)max_rows, (size_t)max_vocab);
  WorkspaceViews v{};
  Workspace& ws = v.ws;
  ws.max_rows = max_rows;
  ws.max_vocab = max_vocab;
  ws.max_chunks = (max_vocab + kChunk - 1) / kChunk;
  ws.summaries = reinterpret_cast<SliceSummary*>(b + L.sum);
  ws.rows = reinterpret_cast<RowInfo*>(b + L.rows);
  ws.chunk_w = reinterpret_cast<uint64_t*>(b + L.chunk);
  ws.cands = reinterpret_cast<Candidate*>(b + L.cand);
  ws.klist = reinterpret_cast<KeptItem*>(b + L.klist);
  ws.partials = reinterpret_cast<SelectPartial*>(b + L.part);
  ws.status = reinterpret_cast<uint32_t*>(b + L.status);
  ws.tasks = reinterpret_cast<uint32_t*>(b + L.tasks);
  ws.cand_count = reinterpret_cast<uint32_t*>(b + L.cc);
  ws.arrive_stats = reinterpret_cast<uint32_t*>(b + L.as);
  ws.arrive_select = reinterpret_cast<uint32_t*>(b + L.asel);
  ws.vstats = reinterpret_cast<lsamp_row_stats*>(b + L.vstats);
  ws.vtokens = reinterpret_cast<int32_t*>(b + L.vtok);
  ws.vflags = reinterpret_cast<uint32_t*>(b + L.vfl);
  ws.max_parts = (int32_t)verify_parts((size_t)max_vocab);
  ws.vspan = reinterpret_cast<VerifySpan*>(b + L.vspan);
  ws.vticket = reinterpret_cast<uint32_t*>(b + L.vtick);
  v.rank_part = reinterpret_cast<RankSlice*>(b + L.rpart);
  v.arrive_rank = reinterpret_cast<uint32_t*>(b + L.arank);
  v.vrow_ptr = reinterpret_cast<int32_t*>(b + L.vrp);
  v.vrow_len = reinterpret_cast<int32_t*>(b + L.vrl);
  v.smask = reinterpret_cast<uint32_t*>(b + L.smask);
  v.smask_words = (max_vocab + 31) / 32;
  v.topk.pub = reinterpret_cast<uint64_t*>(b + L.tpub);
  v.topk.ticket = reinterpret_cast<uint32_t*>(b + L.tticket);
  v.topk.epoch = reinterpret_cast<uint32_t*>(b + L.tepoch);
  v.rawrec = reinterpret_cast<RawRecord*>(b + L.rawrec);
  v.topk.status = ws.status;
  v.zero_begin = b + L.zero_begin;
  v.zero_bytes = L.zero_end - L.zero_begin;
  return v;
}

// What the planner needs to know about a device: its CUs and how many
// work-groups of each sampling kernel fit on one (per dtype).
struct DeviceShape {
  int32_t cus;
  int32_t fused_bpc[3];
  int32_t topk_bpc[3];
};
inline DeviceShape query_device_shape(int32_t cus) {
  DeviceShape d{};
  d.cus = cus;
  for (int dt = 0; dt < 3; ++dt) {
    d.fused_bpc[dt] = fused_blocks_per_cu(dt);
    d.topk_bpc[dt] = topk_blocks_per_cu(dt);
  }
  return d;
}

// Validation, planning and launch of one sampling step (lsamp_sample) over a
// workspace; records the launch shape in *last.  Sets the thread's last
// error and returns its status.
// `lp` (or NULL): raw log-probabilities wanted with the draw.  When the step
// runs the top-k kernel it writes them in the same launch and *lp_done is
// set; otherwise the caller computes them with lsamp_logprobs.
lsamp_status sample_step(const WorkspaceViews& v, const DeviceShape& d, int32_t mode,
                         const lsamp_sample_args* a, void* stream, void* const* events,
                         lsamp_launch_info* last, const TopkLp* lp = nullptr,
                         bool* lp_done = nullptr);
// The thread's last-error string (xgrammar_c.h:63-69 convention).
lsamp_status set_error(lsamp_status st, const char* fmt, ...);
lsamp_status clear_error();
// Zero `bytes` (a multiple of 4) at `p` on `stream` with a fill kernel (no
// memset node, so the call can be captured in a HIP graph).
int launch_zero_words(void* p, size_t bytes, void* stream);

}  // namespace lsamp
