// lsamp_internal.h — device workspace layout and launch plan shared by the
// kernels (lsamp_kernels.hip) and the C ABI (lsamp_api.cpp).
#pragma once

#include <stdint.h>

#include "../../include/lsamp.h"

namespace lsamp {

// Work-group shape.  One work-group owns one slice of one row.
constexpr int kThreads = 512;            // 8 wave64s
constexpr int kWaves = kThreads / 64;
constexpr int kElemsPerThread = 64;      // register budget per thread (logits)
constexpr int kMaxSliceLen = kThreads * kElemsPerThread;  // 32768 tokens
constexpr int kChunk = 1024;             // draw granularity (tokens)
constexpr int kMaxSlices = 16;           // slices per row
// Histogram: bins of 1/32 nat of the filter-space logit, kBins of them below
// the slice's top bin (a 32-nat window), plus one tail bin for the rest.
constexpr int kBinScale = 32;
constexpr int kBins = 1024;
constexpr int kTail = kBins;             // index of the tail bin
constexpr int kHist = kBins + 1;
// Packed histogram word: count in bits 46..63, fixed-point mass in 0..45.
constexpr int kCountShift = 46;
constexpr uint64_t kMassMask = (1ull << kCountShift) - 1;
constexpr int kMassFracBits = 30;        // mass = sum(exp(q - edge)) * 2^30
// Candidates (tokens in the cut bin) per row, and per work-group in LDS.
constexpr int kCandCap = 4096;
constexpr int kWgCandCap = 2048;
// Penalty entries handled per slice (LDS).
constexpr int kSliceEntryCap = 2048;
// Fixed-point draw weights: 2^40 * dexp(d).
constexpr float kWeightScale = 1099511627776.0f;

// Cut position of a row (index into the row histogram, 0 = top bin).
constexpr int32_t kCutTail = kBins;      // cut inside the tail bin
constexpr int32_t kCutNone = kBins + 1;  // no filter cuts: every token kept

// Row modes decided by the stats merge.
constexpr int32_t kModeNormal = 0;
constexpr int32_t kModeEmpty = 1;   // every logit masked / NaN
constexpr int32_t kModePosInf = 2;  // +inf logits present: keep exactly those

// Per-slice summary written by the stats kernel.
struct SliceSummary {
  float x_max;         // largest finite transformed logit (pre-temperature)
  int32_t top_bin;     // bin of x_max
  uint32_t flags;      // LSAMP_ROW_NONFINITE | kSliceOverflow | kSlicePosInf
  int32_t n_finite;    // tokens with a finite transformed logit
  uint64_t hist[kHist];
};
constexpr uint32_t kSlicePosInf = 0x100u;
constexpr uint32_t kSliceEntryOverflow = 0x200u;

// Per-row decision written by the last stats work-group of the row.
struct RowInfo {
  float x_max;       // row max (pre-temperature space)
  float q_top;       // s_max / 32: fast filter-space max used by the masses
  int32_t top_bin;   // absolute bin of x_max
  int32_t cut;       // kCut* or bin index relative to top_bin
  int32_t mode;      // kMode*
  uint32_t flags;    // LSAMP_ROW_* accumulated so far
  int32_t count_above;  // tokens in bins above the cut
  int32_t n_finite;
  double mass_above;    // sum exp(q - q_top) of bins above the cut
  double z;             // sum exp(q - q_top) over every finite token
  double p_limit;       // top_p * z (top-p comparison bound), < 0 if off
  float t_min_p;        // min-p threshold in filter space (-inf if off)
  int32_t kept_cands;   // select finalize: kept candidates, listed first in cands[row]
};

// Per-slice partial results of the select kernel.
struct SelectPartial {
  double ent;       // sum over kept tokens of e * d (entropy numerator)
  float min_kept;   // smallest kept filter-space logit
  int32_t n_kept;
  int32_t n_cand;   // candidates this slice produced (for overflow)
  int32_t pad;
};

struct Candidate {
  float y;     // filter-space logit (exact)
  int32_t id;  // token id
};

struct Workspace {
  int32_t max_rows;
  int32_t max_vocab;
  int32_t max_chunks;
  SliceSummary* summaries;   // [max_rows][kMaxSlices]
  RowInfo* rows;             // [max_rows]
  uint64_t* chunk_w;         // [max_rows][max_chunks]
  Candidate* cands;          // [max_rows][kCandCap]
  SelectPartial* partials;   // [max_rows][kMaxSlices]
  uint32_t* cand_count;      // [max_rows]
  uint32_t* arrive_stats;    // [max_rows]
  uint32_t* arrive_select;   // [max_rows]
  // MTP verification scratch
  lsamp_row_stats* vstats;   // [max_rows]
  int32_t* vtokens;          // [max_rows]
  uint32_t* vflags;          // [max_rows]
  int32_t* vprobe;           // [max_rows]
  float* vuniform;           // [max_rows]
  lsamp_row_params* vparams; // [max_rows]
  uint64_t* vres_chunk;      // [max_rows][max_chunks] residual chunk sums
  uint32_t* arrive_resid;    // [max_rows]
};

// Launch description resolved on the host.
struct SamplePlan {
  int32_t semantics;
  int32_t rows;
  int32_t vocab;
  int32_t dtype;
  int64_t row_stride;
  int32_t slices;        // G
  int32_t slice_len;     // tokens per slice (multiple of kChunk)
  int32_t nchunks;
  int32_t aligned;       // 16-byte vector loads allowed
  const void* logits;
  const void* logits2;   // rows >= rows_split read logits2 (MTP draft rows)
  int32_t rows_split;
  const lsamp_row_params* params;
  const int32_t* row_ptr;
  const lsamp_penalty_entry* entries;
  const uint32_t* bitmask;
  int32_t mask_words;
  int32_t mask_bits;
  int32_t mask_tail;
  const float* uniforms;
  const uint64_t* philox_keys;
  const int32_t* probe_tokens;
  int32_t* tokens;
  uint32_t* row_flags;
  float* processed;
  uint8_t* keep;
  lsamp_row_stats* stats;
};

// Kernel launchers (lsamp_kernels.hip).  Return a hipError_t as int.
// `events` (3 hipEvent_t or NULL) are recorded before, between and after the
// two kernels.
int launch_sample(const Workspace& ws, const SamplePlan& plan, void* stream, void* const* events);
int launch_verify_residual(const Workspace& ws, const lsamp_verify_args& va, int32_t slices,
                           int32_t slice_len, int32_t nchunks, int32_t aligned, void* stream);
int launch_verify_gather(const Workspace& ws, const lsamp_verify_args& va, int32_t nchunks,
                         void* stream);

}  // namespace lsamp
