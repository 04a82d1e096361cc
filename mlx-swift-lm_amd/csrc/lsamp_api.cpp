// lsamp_api.cpp — the C ABI of include/lsamp.h: context (device workspace),
// argument validation, launch planning, host-side parameter resolution.
//
// Conventions follow Libraries/MLXCXGrammar/include/xgrammar_c.h:28-69:
// int32 status codes and a thread-local last-error message; a failed call
// leaves every output untouched.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "lsamp_internal.h"
#include "../../include/lsamp_testing.h"

using namespace lsamp;

namespace {

thread_local std::string g_last_error;

lsamp_status fail(lsamp_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

lsamp_status ok() {
  g_last_error.clear();
  return LSAMP_OK;
}

}  // namespace

lsamp_status lsamp::set_error(lsamp_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

lsamp_status lsamp::clear_error() { return ok(); }

namespace {

// Restores the caller's current device on scope exit.
struct DeviceGuard {
  int prev = -1;
  bool changed = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) == hipSuccess && prev != dev) {
      changed = hipSetDevice(dev) == hipSuccess;
    }
  }
  ~DeviceGuard() {
    if (changed) (void)hipSetDevice(prev);
  }
};

}  // namespace

struct lsamp_context {
  int32_t device;
  int32_t cus;
  int32_t mode = LSAMP_MODE_AUTO;
  DeviceShape shape{};  // CUs and kernel occupancies
  Workspace ws;
  RankSlice* rank_part;  // [max_rows][kRankMaxSlices] (in `block`)
  uint32_t* arrive_rank; // [max_rows] (in `block`)
  int32_t* vrow_ptr;     // [max_rows] penalty-aware verify: per-position runs (in `block`)
  int32_t* vrow_len;     // [max_rows] (in `block`)
  WorkspaceViews views;  // every part of `block`
  void* block;  // single device allocation backing the workspace
  size_t bytes;
  // timing hook
  static constexpr int kTimedCalls = 4096;
  bool timing = false;
  int timed = 0;
  hipEvent_t* events = nullptr;  // [kTimedCalls * 3]
  lsamp_launch_info last{};      // shape of the last sample launch
  // grammar mask descriptors: two pinned staging buffers and their device
  // copies; done[i] follows the last assembly that read buffer i
  struct MaskStage {
    void* host[2] = {nullptr, nullptr};
    void* dev[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    size_t cap = 0;
    int next = 0;
  } mstage;
};

namespace {

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Number of slices per row: about one work-group per resident slot of the
// device, slices of whole 1024-token chunks, at most kMaxSliceLen tokens each.
void plan_slices(int32_t rows, int32_t vocab, int32_t slots, int32_t* slices, int32_t* slice_len,
                 int32_t* nchunks) {
  const int32_t nch = (vocab + kChunk - 1) / kChunk;
  const int32_t g_min = (vocab + kMaxSliceLen - 1) / kMaxSliceLen;
  int32_t target = slots > 0 ? slots : 256;
  int32_t g = (target + rows - 1) / rows;
  if (g < g_min) g = g_min;
  if (g > kMaxSlices) g = kMaxSlices;
  if (g > nch) g = nch;
  if (g < 1) g = 1;
  const int32_t cps = (nch + g - 1) / g;
  *slice_len = cps * kChunk;
  *slices = (nch + cps - 1) / cps;
  *nchunks = nch;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Slice option of a ranking launch: the smallest slices (more work-groups)
// that keep a row within kRankMaxSlices slices and the grid within about two
// work-groups per CU.
void plan_rank(int32_t rows, int32_t vocab, int32_t cus, int32_t* option, int32_t* slices) {
  int32_t o = 0;
  for (; o < kRankOptions - 1; ++o) {
    const int32_t g = (vocab + rank_slice_len(o) - 1) / rank_slice_len(o);
    if (g <= kRankMaxSlices && (int64_t)rows * g <= 2 * (int64_t)cus) break;
  }
  *option = o;
  *slices = (vocab + rank_slice_len(o) - 1) / rank_slice_len(o);
}

// Shared checks and launch of lsamp_top2 / lsamp_logprobs.
lsamp_status rank_common(lsamp_context* ctx, RankPlan& P, int32_t min_vocab, void* stream) {
  if (P.dtype != LSAMP_DTYPE_F32 && P.dtype != LSAMP_DTYPE_BF16 && P.dtype != LSAMP_DTYPE_F16)
    return fail(LSAMP_ERR_DTYPE, "unsupported dtype %d", P.dtype);
  if (P.rows <= 0 || P.rows > ctx->ws.max_rows)
    return fail(P.rows <= 0 ? LSAMP_ERR_SHAPE : LSAMP_ERR_CAPACITY, "rows %d outside [1, %d]",
                P.rows, ctx->ws.max_rows);
  if (P.vocab < min_vocab || P.vocab > ctx->ws.max_vocab)
    return fail(P.vocab < min_vocab ? LSAMP_ERR_SHAPE : LSAMP_ERR_CAPACITY,
                "vocab %d outside [%d, %d]", P.vocab, min_vocab, ctx->ws.max_vocab);
  if (P.row_stride < 0 || P.col_stride < 1)
    return fail(LSAMP_ERR_SHAPE, "row_stride %lld / col_stride %lld invalid",
                (long long)P.row_stride, (long long)P.col_stride);
  if (!P.logits) return fail(LSAMP_ERR_INVALID_ARGUMENT, "logits is NULL");
  const size_t es = P.dtype == LSAMP_DTYPE_F32 ? 4 : 2;
  P.vec = P.col_stride == 1 && aligned16(P.logits) && ((size_t)P.row_stride * es) % 16 == 0;
  plan_rank(P.rows, P.vocab, ctx->cus, &P.option, &P.slices);
  P.part = ctx->rank_part;
  P.arrive = ctx->arrive_rank;
  DeviceGuard guard(ctx->device);
  const int err = launch_rank(P, stream);
  if (err != 0)
    return fail(LSAMP_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString((hipError_t)err));
  return ok();
}

}  // namespace

// Can the one-pass top-k kernel sample every row (the host copy of the
// parameters says so)?  Argmax rows (a sampled row whose temperature defines
// no distribution draws the argmax too), and CBv2 rows with an active top-k
// of at most kTopkMaxK.
static bool topk_eligible(const lsamp_sample_args* a) {
  if (!a->params_host) return false;
  for (int32_t r = 0; r < a->rows; ++r) {
    const lsamp_row_params& p = a->params_host[r];
    const bool argmax = p.kind == LSAMP_KIND_ARGMAX ||
                        !(p.temperature > 0.0f && p.temperature < INFINITY);
    if (argmax) continue;
    if (a->semantics != LSAMP_SEM_CBV2 || p.kind != LSAMP_KIND_FILTERED) return false;
    if (!(p.top_k > 0 && p.top_k < a->vocab && p.top_k <= kTopkMaxK)) return false;
  }
  return true;
}

lsamp_status lsamp::sample_step(const WorkspaceViews& v, const DeviceShape& d, int32_t mode,
                                const lsamp_sample_args* a, void* stream, void* const* ev,
                                lsamp_launch_info* last, const TopkLp* lp, bool* lp_done) {
  if (lp_done) *lp_done = false;
  if (!a) return fail(LSAMP_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->semantics != LSAMP_SEM_MLXLM && a->semantics != LSAMP_SEM_CBV2)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "unknown semantics %d", a->semantics);
  if (a->dtype != LSAMP_DTYPE_F32 && a->dtype != LSAMP_DTYPE_BF16 && a->dtype != LSAMP_DTYPE_F16)
    return fail(LSAMP_ERR_DTYPE, "unsupported dtype %d", a->dtype);
  if (a->rows <= 0 || a->rows > v.ws.max_rows)
    return fail(a->rows <= 0 ? LSAMP_ERR_SHAPE : LSAMP_ERR_CAPACITY,
                "rows %d outside [1, %d]", a->rows, v.ws.max_rows);
  if (a->vocab <= 0 || a->vocab > v.ws.max_vocab)
    return fail(a->vocab <= 0 ? LSAMP_ERR_SHAPE : LSAMP_ERR_CAPACITY,
                "vocab %d outside [1, %d]", a->vocab, v.ws.max_vocab);
  if (a->row_stride < a->vocab)
    return fail(LSAMP_ERR_SHAPE, "row_stride %lld < vocab %d", (long long)a->row_stride, a->vocab);
  if (!a->logits || !a->params || !a->tokens)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "logits, params and tokens are required");
  if (!a->uniforms && !a->philox_keys)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "either uniforms or philox_keys is required");
  if ((a->penalty_row_ptr == nullptr) != (a->penalty_entries == nullptr))
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "penalty_row_ptr and penalty_entries go together");
  if (a->penalty_row_len && !a->penalty_row_ptr)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "penalty_row_len needs penalty_row_ptr");
  if (a->bitmask) {
    if (a->mask_words <= 0 || a->mask_bits < 0)
      return fail(LSAMP_ERR_SHAPE, "mask_words %d / mask_bits %d invalid", a->mask_words,
                  a->mask_bits);
    // xgrammar: vocab_size <= bitmask words * 32 (grammar_matcher.cc:219-222)
    if ((int64_t)a->mask_bits > (int64_t)a->mask_words * 32)
      return fail(LSAMP_ERR_SHAPE, "mask_bits %d exceed %d words", a->mask_bits, a->mask_words);
    if (a->mask_tail != LSAMP_MASK_TAIL_KEEP && a->mask_tail != LSAMP_MASK_TAIL_FORBID)
      return fail(LSAMP_ERR_INVALID_ARGUMENT, "unknown mask_tail %d", a->mask_tail);
  }
  if (a->n_suppress < 0 || a->n_suppress > LSAMP_MAX_SUPPRESS)
    return fail(LSAMP_ERR_SHAPE, "n_suppress %d outside [0, %d]", a->n_suppress,
                LSAMP_MAX_SUPPRESS);
  if (a->n_suppress > 0 && !a->suppress_ids)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "suppress_ids is NULL");
  SamplePlan P{};
  P.semantics = a->semantics;
  P.rows = a->rows;
  P.vocab = a->vocab;
  P.dtype = a->dtype;
  P.row_stride = a->row_stride;
  bool topk = mode == LSAMP_MODE_AUTO && d.topk_bpc[a->dtype] > 0 && topk_eligible(a);
  if (topk && lp && lp->k >= 0 && a->dtype == LSAMP_DTYPE_F32 && d.fused_bpc[a->dtype] > 0) {
    // raw log-probabilities of fp32 logits: the top-k kernel has no variant
    // that ranks them and the fused sampling kernel does, in one round, so
    // a batch that fits one round takes it (no second pass)
    const int32_t fslots = d.cus * d.fused_bpc[a->dtype];
    int32_t fs = 0, fl = 0, fc = 0;
    plan_slices(a->rows, a->vocab, fslots, &fs, &fl, &fc);
    if ((int64_t)a->rows * fs <= fslots) topk = false;
  }
  const int32_t bpc = topk ? d.topk_bpc[a->dtype] : d.fused_bpc[a->dtype];
  const int32_t slots = d.cus * (bpc > 0 ? bpc : 1);
  // (the top-k kernel: one work-group per CU is enough, and fewer slices per
  // row mean a shorter merge)
  plan_slices(a->rows, a->vocab, topk ? d.cus : slots, &P.slices, &P.slice_len, &P.nchunks);
  // (fp32 steps run fused in one round only: the fused kernel's several-rounds
  // form is not built for the fp32 slab)
  P.fused = !topk && mode != LSAMP_MODE_SPLIT && bpc > 0 && slots >= P.slices &&
            (a->dtype != LSAMP_DTYPE_F32 || (int64_t)a->rows * P.slices <= slots);
  P.rows_per_round = P.fused ? slots / P.slices : a->rows;
  const size_t es = a->dtype == LSAMP_DTYPE_F32 ? 4 : 2;
  P.aligned = aligned16(a->logits) && ((size_t)a->row_stride * es) % 16 == 0;
  P.logits = a->logits;
  P.logits2 = a->logits;
  P.rows_split = a->rows;
  P.params = a->params;
  P.row_ptr = a->penalty_row_ptr;
  P.row_len = a->penalty_row_len;
  P.entries = a->penalty_entries;
  P.bitmask = a->bitmask;
  P.mask_words = a->mask_words;
  P.mask_bits = a->mask_bits;
  P.mask_tail = a->mask_tail;
  P.uniforms = a->uniforms;
  P.philox_keys = a->philox_keys;
  P.probe_tokens = a->probe_tokens;
  P.tokens = a->tokens;
  P.row_flags = a->row_flags;
  P.processed = a->processed;
  P.keep = a->keep;
  P.stats = a->stats;
  P.stats_full = a->stats != nullptr;
  if (a->n_suppress > 0) {
    // the suppressed ids and the caller's bitmask become one bitmask over
    // the whole vocabulary, which the sampling kernels apply as any other
    SuppressPlan S{};
    S.rows = a->rows;
    S.vocab = a->vocab;
    S.words = (a->vocab + 31) / 32;
    S.bitmask = a->bitmask;
    S.mask_words = a->mask_words;
    S.mask_bits = a->mask_bits;
    S.mask_tail = a->mask_tail;
    S.ids = a->suppress_ids;
    S.n = a->n_suppress;
    S.out = v.smask;
    const int err = launch_suppress_mask(S, stream);
    if (err != 0)
      return fail(LSAMP_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString((hipError_t)err));
    P.bitmask = v.smask;
    P.mask_words = S.words;
    P.mask_bits = a->vocab;
    P.mask_tail = LSAMP_MASK_TAIL_KEEP;
  }
  // raw log-probabilities in the same launch: the top-k kernel (16-bit
  // logits), or the fused sampling kernel (any dtype)
  const bool lp_fused = topk && lp && lp->k >= 0 && a->dtype != LSAMP_DTYPE_F32;
  const bool lp_sample = !topk && P.fused && lp && lp->k >= 0;
  TopkLp lpk{};
  lpk.k = -1;
  if (lp_fused) lpk = *lp;
  FusedLp flp{};
  flp.k = -1;
  if (lp_sample) {
    flp.k = lp->k;
    flp.chosen = lp->chosen;
    flp.values = lp->values;
    flp.ids = lp->ids;
    flp.rec = v.rawrec;
  }
  last->fused = topk ? (lp_fused ? 3 : 2) : (lp_sample ? 4 : P.fused);
  last->slices = P.slices;
  last->slice_len = P.slice_len;
  last->rows_per_round = P.rows_per_round;
  last->grid = topk ? (P.rows + 7) / 8 * 8 * P.slices
                    : P.fused ? (P.rows < P.rows_per_round ? P.rows : P.rows_per_round) * P.slices
                              : P.rows * P.slices;
  const int err =
      topk ? launch_topk(P, v.topk, lpk, stream, ev)
           : launch_sample(v.ws, P, lp_sample ? &flp : nullptr, stream, ev);
  if (err != 0) return fail(LSAMP_ERR_DEVICE, "kernel launch failed: %s",
                            hipGetErrorString((hipError_t)err));
  if (lp_done) *lp_done = lp_fused || lp_sample;
  return ok();
}


extern "C" {

const char* lsamp_last_error(void) { return g_last_error.c_str(); }

const char* lsamp_version(void) { return "lsamp 0.1.0 (gfx950, abi 1)"; }

int64_t lsamp_abi_sizeof(const char* name) {
  if (!name) return -1;
  if (!strcmp(name, "lsamp_row_params")) return (int64_t)sizeof(lsamp_row_params);
  if (!strcmp(name, "lsamp_penalty_entry")) return (int64_t)sizeof(lsamp_penalty_entry);
  if (!strcmp(name, "lsamp_row_stats")) return (int64_t)sizeof(lsamp_row_stats);
  if (!strcmp(name, "lsamp_sample_args")) return (int64_t)sizeof(lsamp_sample_args);
  if (!strcmp(name, "lsamp_verify_args")) return (int64_t)sizeof(lsamp_verify_args);
  if (!strcmp(name, "lsamp_generate_parameters")) return (int64_t)sizeof(lsamp_generate_parameters);
  if (!strcmp(name, "lsamp_cbv2_params")) return (int64_t)sizeof(lsamp_cbv2_params);
  if (!strcmp(name, "lsamp_launch_info")) return (int64_t)sizeof(lsamp_launch_info);
  if (!strcmp(name, "lsamp_top2_args")) return (int64_t)sizeof(lsamp_top2_args);
  if (!strcmp(name, "lsamp_propose_args")) return (int64_t)sizeof(lsamp_propose_args);
  if (!strcmp(name, "lsamp_step_args")) return (int64_t)sizeof(lsamp_step_args);
  if (!strcmp(name, "lsamp_penalty_table")) return (int64_t)sizeof(lsamp_penalty_table);
  if (!strcmp(name, "lsamp_commit_args")) return (int64_t)sizeof(lsamp_commit_args);
  if (!strcmp(name, "lsamp_mask_assemble_args")) return (int64_t)sizeof(lsamp_mask_assemble_args);
  if (!strcmp(name, "lsamp_logprobs_args")) return (int64_t)sizeof(lsamp_logprobs_args);
  if (!strcmp(name, "lsamp_penalize_args")) return (int64_t)sizeof(lsamp_penalize_args);
  return -1;
}

lsamp_status lsamp_context_create(int32_t device, int32_t max_rows, int32_t max_vocab,
                                  lsamp_context** out) {
  if (!out) return fail(LSAMP_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  if (max_rows <= 0 || max_rows > (1 << 20))
    return fail(LSAMP_ERR_SHAPE, "max_rows %d out of range [1, 1048576]", max_rows);
  if (max_vocab <= 0 || max_vocab > kMaxVocab)
    return fail(LSAMP_ERR_SHAPE, "max_vocab %d out of range [1, %d]", max_vocab, kMaxVocab);
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
    return fail(LSAMP_ERR_DEVICE, "device %d not available (%d devices)", device, ndev);
  DeviceGuard guard(device);
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess)
    return fail(LSAMP_ERR_DEVICE, "hipGetDeviceProperties failed");

  const size_t total = workspace_layout((size_t)max_rows, (size_t)max_vocab).total;
  void* block = nullptr;
  if (hipMalloc(&block, total) != hipSuccess)
    return fail(LSAMP_ERR_DEVICE, "hipMalloc(%zu) failed", total);
  // Arrival counters and candidate counts must start at zero; the kernels
  // return them to zero at the end of every step.
  if (hipMemset(block, 0, total) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
    (void)hipFree(block);
    return fail(LSAMP_ERR_DEVICE, "hipMemset of the workspace failed");
  }
  lsamp_context* ctx = new lsamp_context();
  ctx->device = device;
  ctx->cus = prop.multiProcessorCount;
  ctx->shape = query_device_shape(prop.multiProcessorCount);
  ctx->block = block;
  ctx->bytes = total;
  ctx->views = bind_workspace(reinterpret_cast<char*>(block), max_rows, max_vocab);
  ctx->ws = ctx->views.ws;
  ctx->rank_part = ctx->views.rank_part;
  ctx->arrive_rank = ctx->views.arrive_rank;
  ctx->vrow_ptr = ctx->views.vrow_ptr;
  ctx->vrow_len = ctx->views.vrow_len;
  *out = ctx;
  return ok();
}

void lsamp_context_destroy(lsamp_context* ctx) {
  if (!ctx) return;
  {
    DeviceGuard guard(ctx->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(ctx->block);
    for (int i = 0; i < 2; ++i) {
      if (ctx->mstage.host[i]) (void)hipHostFree(ctx->mstage.host[i]);
      if (ctx->mstage.dev[i]) (void)hipFree(ctx->mstage.dev[i]);
      if (ctx->mstage.done[i]) (void)hipEventDestroy(ctx->mstage.done[i]);
    }
    if (ctx->events) {
      for (int i = 0; i < lsamp_context::kTimedCalls * 3; ++i) (void)hipEventDestroy(ctx->events[i]);
      delete[] ctx->events;
    }
  }
  delete ctx;
}

lsamp_status lsamp_context_set_mode(lsamp_context* ctx, int32_t mode) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  if (mode != LSAMP_MODE_AUTO && mode != LSAMP_MODE_FUSED && mode != LSAMP_MODE_SPLIT)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "unknown mode %d", mode);
  ctx->mode = mode;
  return ok();
}

lsamp_status lsamp_context_read_status(lsamp_context* ctx, uint32_t* bits) {
  if (!ctx || !bits) return fail(LSAMP_ERR_INVALID_ARGUMENT, "NULL argument");
  DeviceGuard guard(ctx->device);
  uint32_t v = 0, zero = 0;
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(&v, ctx->ws.status, sizeof v, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(ctx->ws.status, &zero, sizeof zero, hipMemcpyHostToDevice) != hipSuccess)
    return fail(LSAMP_ERR_DEVICE, "reading the device status failed");
  *bits = v;
  return ok();
}

lsamp_status lsamp_test_set_spin_limit(int32_t device, int32_t polls) {
  if (polls < 0) return fail(LSAMP_ERR_INVALID_ARGUMENT, "polls %d is negative", polls);
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
    return fail(LSAMP_ERR_DEVICE, "device %d not available (%d devices)", device, ndev);
  DeviceGuard guard(device);
  if (set_spin_test(polls) != 0 || set_topk_spin_test(polls) != 0 ||
      hipDeviceSynchronize() != hipSuccess)
    return fail(LSAMP_ERR_DEVICE, "setting the wait test hook failed");
  return ok();
}

lsamp_status lsamp_context_last_launch(lsamp_context* ctx, lsamp_launch_info* out) {
  if (!ctx || !out) return fail(LSAMP_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = ctx->last;
  return ok();
}

lsamp_status lsamp_context_set_timing(lsamp_context* ctx, int32_t enable) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  DeviceGuard guard(ctx->device);
  if (enable && !ctx->events) {
    ctx->events = new hipEvent_t[lsamp_context::kTimedCalls * 3];
    for (int i = 0; i < lsamp_context::kTimedCalls * 3; ++i) {
      if (hipEventCreate(&ctx->events[i]) != hipSuccess) {
        for (int j = 0; j < i; ++j) (void)hipEventDestroy(ctx->events[j]);
        delete[] ctx->events;
        ctx->events = nullptr;
        return fail(LSAMP_ERR_DEVICE, "hipEventCreate failed");
      }
    }
  }
  ctx->timing = enable != 0;
  ctx->timed = 0;
  return ok();
}

lsamp_status lsamp_context_read_timing(lsamp_context* ctx, double* stats_ms, double* select_ms,
                                       int64_t* calls) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  DeviceGuard guard(ctx->device);
  double a = 0.0, b = 0.0;
  for (int i = 0; i < ctx->timed; ++i) {
    hipEvent_t* e = ctx->events + 3 * i;
    if (hipEventSynchronize(e[2]) != hipSuccess) return fail(LSAMP_ERR_DEVICE, "hipEventSynchronize failed");
    float t01 = 0.0f, t12 = 0.0f;
    if (hipEventElapsedTime(&t01, e[0], e[1]) != hipSuccess ||
        hipEventElapsedTime(&t12, e[1], e[2]) != hipSuccess)
      return fail(LSAMP_ERR_DEVICE, "hipEventElapsedTime failed");
    a += t01;
    b += t12;
  }
  if (stats_ms) *stats_ms = a;
  if (select_ms) *select_ms = b;
  if (calls) *calls = ctx->timed;
  ctx->timed = 0;
  return ok();
}

// lsamp_sample, and lsamp_step's draw with its raw log-probabilities (`lp`,
// done in the same launch when *lp_done comes back true).
static lsamp_status sample_call(lsamp_context* ctx, const lsamp_sample_args* a, void* stream,
                                const TopkLp* lp, bool* lp_done) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  DeviceGuard guard(ctx->device);
  void* const* ev = nullptr;
  if (ctx->timing && ctx->timed < lsamp_context::kTimedCalls) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(reinterpret_cast<hipStream_t>(stream), &cs) == hipSuccess &&
        cs == hipStreamCaptureStatusNone)
      ev = reinterpret_cast<void* const*>(ctx->events + 3 * ctx->timed);
  }
  const lsamp_status st =
      sample_step(ctx->views, ctx->shape, ctx->mode, a, stream, ev, &ctx->last, lp, lp_done);
  if (st == LSAMP_OK && ev) ++ctx->timed;
  return st;
}

lsamp_status lsamp_sample(lsamp_context* ctx, const lsamp_sample_args* a, void* stream) {
  return sample_call(ctx, a, stream, nullptr, nullptr);
}

lsamp_status lsamp_step(lsamp_context* ctx, const lsamp_step_args* a, void* stream) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  if (!a) return fail(LSAMP_ERR_INVALID_ARGUMENT, "args is NULL");
  const lsamp_sample_args& sa = a->sample;
  if (a->table && a->table->rows != sa.rows)
    return fail(LSAMP_ERR_SHAPE, "table rows %d != sample rows %d", a->table->rows, sa.rows);
  if (a->logprobs_top_k >= 0 && !a->chosen_logprob)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "log-probabilities need chosen_logprob");
  // validate the later calls before enqueueing anything
  lsamp_logprobs_args la{};
  if (a->logprobs_top_k >= 0) {
    la.rows = sa.rows;
    la.vocab = sa.vocab;
    la.dtype = sa.dtype;
    la.row_stride = sa.row_stride;
    la.col_stride = 1;
    la.logits = sa.logits;
    la.top_k = a->logprobs_top_k;
    la.tokens = sa.tokens;
    la.chosen = a->chosen_logprob;
    la.top_values = a->top_logprobs;
    la.top_ids = a->top_ids;
    if (la.top_k > kRankMaxK || la.top_k > la.vocab)
      return fail(LSAMP_ERR_SHAPE, "logprobs_top_k %d outside [0, min(%d, vocab)]", la.top_k,
                  kRankMaxK);
    if (la.top_k > 0 && (!la.top_values || !la.top_ids))
      return fail(LSAMP_ERR_INVALID_ARGUMENT, "top_logprobs and top_ids are required");
  }
  // the top-k kernel writes the raw log-probabilities in the same pass over
  // the logits when it takes the step; otherwise they are a second pass
  TopkLp lp{};
  lp.k = a->logprobs_top_k;
  lp.chosen = la.chosen;
  lp.values = la.top_values;
  lp.ids = la.top_ids;
  bool lp_done = false;
  lsamp_status st =
      sample_call(ctx, &sa, stream, a->logprobs_top_k >= 0 ? &lp : nullptr, &lp_done);
  if (st != LSAMP_OK) return st;
  if (a->table) {
    lsamp_commit_args c{};
    c.table = *a->table;
    c.vocab = sa.vocab;
    c.tokens = sa.tokens;
    c.row_flags = a->commit_flags;
    st = lsamp_commit(ctx, &c, stream);
    if (st != LSAMP_OK) return st;
  }
  if (a->logprobs_top_k >= 0 && !lp_done) return lsamp_logprobs(ctx, &la, stream);
  return ok();
}

lsamp_status lsamp_propose(lsamp_context* ctx, const lsamp_propose_args* a, void* stream) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  if (!a) return fail(LSAMP_ERR_INVALID_ARGUMENT, "args is NULL");
  // the draft row's own draw: one CBv2 sampling step, no penalties, no mask
  lsamp_sample_args s{};
  s.semantics = LSAMP_SEM_CBV2;
  s.rows = a->rows;
  s.vocab = a->vocab;
  s.dtype = a->dtype;
  s.row_stride = a->row_stride;
  s.logits = a->logits;
  s.params = a->params;
  s.uniforms = a->uniforms;
  s.philox_keys = a->philox_keys;
  s.tokens = a->tokens;
  return lsamp_sample(ctx, &s, stream);
}

lsamp_status lsamp_top2(lsamp_context* ctx, const lsamp_top2_args* a, void* stream) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  if (!a) return fail(LSAMP_ERR_INVALID_ARGUMENT, "args is NULL");
  if (!a->ids || !a->values) return fail(LSAMP_ERR_INVALID_ARGUMENT, "ids and values are required");
  RankPlan P{};
  P.rows = a->rows;
  P.vocab = a->vocab;
  P.dtype = a->dtype;
  P.k = 2;
  P.row_stride = a->row_stride;
  P.col_stride = a->col_stride;
  P.lse = 0;
  P.raw_values = 1;
  P.logits = a->logits;
  P.ids = a->ids;
  P.values = a->values;
  // precondition(rows > 0 && vocabularySize >= 2), CBv2TopTwo.swift:195
  return rank_common(ctx, P, 2, stream);
}

lsamp_status lsamp_logprobs(lsamp_context* ctx, const lsamp_logprobs_args* a, void* stream) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  if (!a) return fail(LSAMP_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->top_k < 0 || a->top_k > kRankMaxK || a->top_k > a->vocab)
    return fail(LSAMP_ERR_SHAPE, "top_k %d outside [0, min(%d, vocab)]", a->top_k, kRankMaxK);
  if (a->top_k > 0 && (!a->top_values || !a->top_ids))
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "top_values and top_ids are required when top_k > 0");
  if ((a->tokens == nullptr) != (a->chosen == nullptr))
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "tokens and chosen go together");
  RankPlan P{};
  P.rows = a->rows;
  P.vocab = a->vocab;
  P.dtype = a->dtype;
  P.k = a->top_k;
  P.row_stride = a->row_stride;
  P.col_stride = a->col_stride;
  P.lse = 1;
  P.raw_values = 0;
  P.logits = a->logits;
  P.tokens = a->tokens;
  P.chosen = a->chosen;
  P.values = a->top_values;
  P.ids = a->top_ids;
  P.row_flags = a->row_flags;
  return rank_common(ctx, P, 1, stream);
}

lsamp_status lsamp_commit(lsamp_context* ctx, const lsamp_commit_args* a, void* stream) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  if (!a) return fail(LSAMP_ERR_INVALID_ARGUMENT, "args is NULL");
  const lsamp_penalty_table& t = a->table;
  if (t.rows <= 0 || t.capacity <= 0 || t.window_capacity <= 0)
    return fail(LSAMP_ERR_SHAPE, "rows %d / capacity %d / window_capacity %d must be positive",
                t.rows, t.capacity, t.window_capacity);
  if (a->vocab <= 0) return fail(LSAMP_ERR_SHAPE, "vocab %d must be positive", a->vocab);
  if (!t.entries || !t.row_len || !t.window_count || !t.window || !t.ring_pos ||
      !t.window_size || !t.mode || !a->tokens)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "every table array and tokens are required");
  DeviceGuard guard(ctx->device);
  const int err = launch_commit(*a, stream);
  if (err != 0)
    return fail(LSAMP_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString((hipError_t)err));
  return ok();
}

// ------------------------------------------------------- penalty processor

lsamp_status lsamp_penalize(lsamp_context* ctx, const lsamp_penalize_args* a, void* stream) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  if (!a) return fail(LSAMP_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->rows <= 0 || a->vocab <= 0)
    return fail(LSAMP_ERR_SHAPE, "rows %d / vocab %d must be positive", a->rows, a->vocab);
  if (a->row_stride < a->vocab)
    return fail(LSAMP_ERR_SHAPE, "row_stride %lld is below vocab %d", (long long)a->row_stride,
                a->vocab);
  if (a->dtype < LSAMP_DTYPE_F32 || a->dtype > LSAMP_DTYPE_F16)
    return fail(LSAMP_ERR_DTYPE, "dtype %d is not a logits dtype", a->dtype);
  if (a->out_dtype != a->dtype && a->out_dtype != LSAMP_DTYPE_F32)
    return fail(LSAMP_ERR_DTYPE, "out_dtype %d must be the logits dtype %d or float32",
                a->out_dtype, a->dtype);
  if (!a->logits || !a->params || !a->out)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "logits, params and out are required");
  if ((a->penalty_entries != nullptr) != (a->penalty_row_ptr != nullptr))
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "penalty_row_ptr and penalty_entries go together");
  PenalizePlan P{};
  P.rows = a->rows;
  P.vocab = a->vocab;
  P.dtype = a->dtype;
  P.out_dtype = a->out_dtype;
  P.row_stride = a->row_stride;
  P.logits = a->logits;
  P.params = a->params;
  P.row_ptr = a->penalty_row_ptr;
  P.row_len = a->penalty_row_len;
  P.entries = a->penalty_entries;
  P.out = a->out;
  DeviceGuard guard(ctx->device);
  const int err = launch_penalize(P, stream);
  if (err != 0)
    return fail(LSAMP_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString((hipError_t)err));
  return ok();
}

// ------------------------------------------------------------- grammar masks

lsamp_status lsamp_mask_assemble(lsamp_context* ctx, const lsamp_mask_assemble_args* a,
                                 void* stream) {
  if (!ctx) return fail(LSAMP_ERR_INVALID_ARGUMENT, "context is NULL");
  if (!a) return fail(LSAMP_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->rows <= 0 || a->vocab <= 0)
    return fail(LSAMP_ERR_SHAPE, "rows %d / vocab %d must be positive", a->rows, a->vocab);
  if (a->words != (a->vocab + 31) / 32 || a->words > LSAMP_MASK_MAX_WORDS)
    return fail(LSAMP_ERR_SHAPE, "words %d must be (vocab + 31) / 32 = %d and at most %d",
                a->words, (a->vocab + 31) / 32, LSAMP_MASK_MAX_WORDS);
  if (!a->out || !a->row_source || !a->row_build || !a->ids_ptr)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "out, row_source, row_build and ids_ptr are required");
  if (a->pool_rows < 0) return fail(LSAMP_ERR_SHAPE, "pool_rows %d is negative", a->pool_rows);
  if (a->ids_ptr[0] != 0) return fail(LSAMP_ERR_SHAPE, "ids_ptr[0] must be 0");
  for (int32_t r = 0; r < a->rows; ++r) {
    const int32_t s = a->row_source[r];
    if (s < -1 || s >= a->pool_rows)
      return fail(LSAMP_ERR_SHAPE, "row %d: pool row %d outside [-1, %d)", r, s, a->pool_rows);
    if (s >= 0 && !a->pool) return fail(LSAMP_ERR_INVALID_ARGUMENT, "pool is NULL");
    if (a->row_build[r] && s < 0)
      return fail(LSAMP_ERR_SHAPE, "row %d: a build needs a pool row", r);
    if (a->ids_ptr[r + 1] < a->ids_ptr[r])
      return fail(LSAMP_ERR_SHAPE, "ids_ptr decreases at row %d", r);
  }
  const int32_t nids = a->ids_ptr[a->rows];
  if (nids > 0 && !a->ids) return fail(LSAMP_ERR_INVALID_ARGUMENT, "ids is NULL");
  DeviceGuard guard(ctx->device);
  MaskAssemblePlan P{};
  P.rows = a->rows;
  P.vocab = a->vocab;
  P.words = a->words;
  P.vec = (a->words % 4 == 0 && ((uintptr_t)a->out % 16) == 0 && ((uintptr_t)a->pool % 16) == 0)
              ? 1 : 0;
  P.pool = a->pool;
  P.out = a->out;
  P.row_flags = a->row_flags;
  bool any_build = false;
  for (int32_t r = 0; r < a->rows; ++r) any_build |= a->row_build[r] != 0;
  if (!any_build && a->rows <= kMaskInlineRows) {
    // every row cached or open: the pool rows travel in the kernel arguments
    P.inline_rows = a->rows;
    memcpy(P.src_inline, a->row_source, (size_t)a->rows * 4);
    const int err = launch_mask_assemble(P, stream);
    if (err != 0)
      return fail(LSAMP_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString((hipError_t)err));
    return ok();
  }
  // staging layout: row_source | ids_ptr | ids | row_build, 16-byte aligned parts
  const size_t b_src = align_up((size_t)a->rows * 4, 16);
  const size_t b_ptr = align_up(((size_t)a->rows + 1) * 4, 16);
  const size_t b_ids = align_up((size_t)nids * 4, 16);
  const size_t bytes = b_src + b_ptr + b_ids + align_up((size_t)a->rows, 16);
  auto& m = ctx->mstage;
  if (bytes > m.cap) {
    // growth: wait for both buffers' readers, then reallocate
    for (int i = 0; i < 2; ++i) {
      if (m.pending[i]) (void)hipEventSynchronize(m.done[i]);
      m.pending[i] = false;
      if (m.host[i]) (void)hipHostFree(m.host[i]);
      if (m.dev[i]) (void)hipFree(m.dev[i]);
      m.host[i] = m.dev[i] = nullptr;
    }
    const size_t cap = align_up(bytes * 2 > 65536 ? bytes * 2 : 65536, 4096);
    m.cap = 0;
    for (int i = 0; i < 2; ++i) {
      if (!m.done[i] && hipEventCreateWithFlags(&m.done[i], hipEventDisableTiming) != hipSuccess)
        return fail(LSAMP_ERR_DEVICE, "hipEventCreateWithFlags failed");
      if (hipHostMalloc(&m.host[i], cap, hipHostMallocDefault) != hipSuccess ||
          hipMalloc(&m.dev[i], cap) != hipSuccess)
        return fail(LSAMP_ERR_DEVICE, "mask staging allocation of %zu bytes failed", cap);
    }
    m.cap = cap;
  }
  const int slot = m.next;
  m.next ^= 1;
  // the buffer's previous copy and assembly (two calls ago) must be over
  if (m.pending[slot] && hipEventSynchronize(m.done[slot]) != hipSuccess)
    return fail(LSAMP_ERR_DEVICE, "waiting for the mask staging buffer failed");
  char* h = static_cast<char*>(m.host[slot]);
  memcpy(h, a->row_source, (size_t)a->rows * 4);
  memcpy(h + b_src, a->ids_ptr, ((size_t)a->rows + 1) * 4);
  if (nids > 0) memcpy(h + b_src + b_ptr, a->ids, (size_t)nids * 4);
  memcpy(h + b_src + b_ptr + b_ids, a->row_build, (size_t)a->rows);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (hipMemcpyAsync(m.dev[slot], h, bytes, hipMemcpyHostToDevice, st) != hipSuccess)
    return fail(LSAMP_ERR_DEVICE, "mask descriptor copy failed");
  const char* d = static_cast<const char*>(m.dev[slot]);
  P.row_source = reinterpret_cast<const int32_t*>(d);
  P.ids_ptr = reinterpret_cast<const int32_t*>(d + b_src);
  P.ids = reinterpret_cast<const int32_t*>(d + b_src + b_ptr);
  P.row_build = reinterpret_cast<const uint8_t*>(d + b_src + b_ptr + b_ids);
  const int err = launch_mask_assemble(P, stream);
  if (err != 0)
    return fail(LSAMP_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString((hipError_t)err));
  if (hipEventRecord(m.done[slot], st) != hipSuccess)
    return fail(LSAMP_ERR_DEVICE, "hipEventRecord failed");
  m.pending[slot] = true;
  return ok();
}

// ---------------------------------------------------------------- resolution

lsamp_status lsamp_resolve_generate_parameters(const lsamp_generate_parameters* gp,
                                               lsamp_row_params* out, int32_t* contexts) {
  if (!gp || !out) return fail(LSAMP_ERR_INVALID_ARGUMENT, "NULL argument");
  lsamp_row_params r{};
  // GenerateParameters.sampler() (Evaluate.swift:328-341)
  const bool uses_top_p = gp->top_p > 0.0f && gp->top_p < 1.0f;
  const bool uses_top_k = gp->top_k > 0;
  const bool uses_min_p = gp->min_p > 0.0f;
  if (gp->temperature == 0.0f) {
    r.kind = LSAMP_KIND_ARGMAX;
  } else if (uses_top_p || uses_top_k || uses_min_p) {
    r.kind = LSAMP_KIND_FILTERED;
  } else {
    r.kind = LSAMP_KIND_CATEGORICAL;
  }
  r.temperature = gp->temperature;
  // TopPSampler.init keeps each filter only when enabled (Evaluate.swift:420-427)
  r.top_p = uses_top_p ? gp->top_p : 1.0f;
  r.top_k = uses_top_k ? gp->top_k : 0;
  r.min_p = uses_min_p ? gp->min_p : 0.0f;
  // GenerateParameters.processor() (Evaluate.swift:343-387)
  int32_t ctxs = 0;
  r.repetition_penalty = 1.0f;
  if (gp->has_repetition_penalty && gp->repetition_penalty != 0.0f &&
      gp->repetition_penalty != 1.0f && gp->repetition_context_size > 0) {
    r.repetition_penalty = gp->repetition_penalty;
    ctxs |= 1;
  }
  r.presence_penalty = 0.0f;
  if (gp->has_presence_penalty && gp->presence_penalty != 0.0f && gp->presence_context_size > 0) {
    r.presence_penalty = gp->presence_penalty;
    ctxs |= 2;
  }
  r.frequency_penalty = 0.0f;
  if (gp->has_frequency_penalty && gp->frequency_penalty != 0.0f &&
      gp->frequency_context_size > 0) {
    r.frequency_penalty = gp->frequency_penalty;
    ctxs |= 4;
  }
  *out = r;
  if (contexts) *contexts = ctxs;
  return ok();
}

lsamp_status lsamp_resolve_cbv2_params(const lsamp_cbv2_params* sp, int32_t vocab,
                                       lsamp_row_params* out) {
  if (!sp || !out) return fail(LSAMP_ERR_INVALID_ARGUMENT, "NULL argument");
  if (vocab <= 0) return fail(LSAMP_ERR_SHAPE, "vocab %d must be positive", vocab);
  lsamp_row_params r{};
  // LogitsPipelineV2.setRows (LogitsPipelineV2.swift:188-227)
  const bool greedy = sp->temperature < 1e-5f;  // greedyEpsilon (:79)
  r.kind = greedy ? LSAMP_KIND_ARGMAX : LSAMP_KIND_FILTERED;
  r.temperature = greedy ? 1.0f : sp->temperature;
  r.top_k = 0;
  r.top_p = 2.0f;
  r.min_p = 0.0f;
  if (!greedy) {
    if (sp->top_k > 0 && sp->top_k < vocab) r.top_k = sp->top_k;
    if (sp->top_p > 0.0f && sp->top_p < 1.0f)
      r.top_p = sp->top_p;
    else if (sp->top_p <= 0.0f)
      r.top_p = 0.0f;  // top_p == 0 keeps only the most probable token (:204-207)
    if (sp->min_p > 0.0f) r.min_p = sp->min_p < 1.0f ? sp->min_p : 1.0f;
  }
  const bool windowed = sp->repetition_penalty != 1.0f && sp->repetition_context_size > 0;
  r.repetition_penalty = windowed ? sp->repetition_penalty : 1.0f;
  if (sp->frequency_penalty != 0.0f || sp->presence_penalty != 0.0f) {
    r.frequency_penalty = sp->frequency_penalty;
    r.presence_penalty = sp->presence_penalty;
  }
  *out = r;
  return ok();
}

// SamplerV2.mix (SamplerV2.swift:183-191).
static uint64_t splitmix64(uint64_t v) {
  uint64_t z = v + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t lsamp_rng_key(uint64_t seed, uint64_t request_id, uint64_t step) {
  return splitmix64(splitmix64(splitmix64(seed) ^ request_id) ^ step);
}

float lsamp_rng_uniform(uint64_t key, uint32_t purpose) {
  uint32_t c0 = purpose, c1 = 0, c2 = 0, c3 = 0;
  uint32_t k0 = (uint32_t)key, k1 = (uint32_t)(key >> 32);
  for (int round = 0; round < 10; ++round) {
    if (round > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    c1 = (uint32_t)p1;
    c3 = (uint32_t)p0;
    c0 = n0;
    c2 = n2;
  }
  return (float)(c0 >> 8) * 5.9604644775390625e-08f;
}

lsamp_status lsamp_verify(lsamp_context* ctx, const lsamp_verify_args* a, void* stream) {
  if (!ctx || !a) return fail(LSAMP_ERR_INVALID_ARGUMENT, "NULL argument");
  if (a->mode != LSAMP_VERIFY_RESIDUAL && a->mode != LSAMP_VERIFY_EXACT &&
      a->mode != LSAMP_VERIFY_TYPICAL)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "unknown verify mode %d", a->mode);
  if (a->dtype != LSAMP_DTYPE_F32 && a->dtype != LSAMP_DTYPE_BF16 && a->dtype != LSAMP_DTYPE_F16)
    return fail(LSAMP_ERR_DTYPE, "unsupported dtype %d", a->dtype);
  if (a->sequences <= 0 || a->window < 2 || a->vocab <= 0)
    return fail(LSAMP_ERR_SHAPE, "sequences %d / window %d / vocab %d invalid", a->sequences,
                a->window, a->vocab);
  if (a->vocab > ctx->ws.max_vocab)
    return fail(LSAMP_ERR_CAPACITY, "vocab %d above the context's %d", a->vocab,
                ctx->ws.max_vocab);
  if (!a->target_logits || !a->draft_tokens || !a->params || !a->uniforms || !a->accepted ||
      !a->tokens)
    return fail(LSAMP_ERR_INVALID_ARGUMENT,
                "target_logits, draft_tokens, params, uniforms, accepted and tokens are required");
  const bool residual = a->mode == LSAMP_VERIFY_RESIDUAL;
  if (residual && !a->draft_logits)
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "RESIDUAL mode needs draft_logits");
  if (a->mode == LSAMP_VERIFY_TYPICAL && !(a->typical_delta > 0.0f))
    return fail(LSAMP_ERR_INVALID_ARGUMENT, "TYPICAL mode needs typical_delta > 0");
  const int64_t S = a->sequences, W = a->window, D = W - 1;
  const int64_t rows = S * W + (residual ? S * D : 0);
  if (rows > ctx->ws.max_rows)
    return fail(LSAMP_ERR_CAPACITY, "verify needs %lld rows, the context holds %d",
                (long long)rows, ctx->ws.max_rows);
  const bool penalized = a->penalty_entries != nullptr;
  WindowEntriesPlan E{};
  if (penalized) {
    if (residual)
      return fail(LSAMP_ERR_INVALID_ARGUMENT,
                  "penalty-aware verification is for the EXACT and TYPICAL modes");
    if (!a->penalty_row_ptr || !a->penalty_scratch || a->penalty_scratch_cap <= 0)
      return fail(LSAMP_ERR_INVALID_ARGUMENT,
                  "penalty_entries needs penalty_row_ptr, penalty_scratch and a positive cap");
    const int32_t off = a->penalty_drafts ? a->penalty_column_offset : 0;
    const int32_t stride = a->penalty_drafts ? a->penalty_drafts_stride : (int32_t)D;
    if (off < 0 || (int64_t)off + D > 64 || (a->penalty_drafts && stride < off + D))
      return fail(LSAMP_ERR_SHAPE,
                  "column_offset %d / drafts_stride %d: at most 64 drafts precede a position",
                  off, stride);
    E.sequences = a->sequences;
    E.window = a->window;
    E.vocab = a->vocab;
    E.cap = a->penalty_scratch_cap;
    E.column_offset = off;
    E.drafts_stride = stride;
    E.row_ptr = a->penalty_row_ptr;
    E.row_len = a->penalty_row_len;
    E.entries = a->penalty_entries;
    E.drafts = a->penalty_drafts ? a->penalty_drafts : a->draft_tokens;
    E.out = a->penalty_scratch;
    E.out_ptr = ctx->vrow_ptr;
    E.out_len = ctx->vrow_len;
    E.status = ctx->ws.status;
  }

  // every target (and, for RESIDUAL, draft) position is one sampling row
  SamplePlan P{};
  P.semantics = LSAMP_SEM_CBV2;
  P.rows = (int32_t)rows;
  P.vocab = a->vocab;
  P.dtype = a->dtype;
  P.row_stride = a->vocab;
  const int32_t bpc = ctx->shape.fused_bpc[a->dtype];
  const int32_t slots = ctx->cus * (bpc > 0 ? bpc : 1);
  plan_slices(P.rows, P.vocab, slots, &P.slices, &P.slice_len, &P.nchunks);
  P.fused = ctx->mode != LSAMP_MODE_SPLIT && bpc > 0 && slots >= P.slices &&
            (a->dtype != LSAMP_DTYPE_F32 || (int64_t)P.rows * P.slices <= slots);
  P.rows_per_round = P.fused ? slots / P.slices : P.rows;
  const size_t es = a->dtype == LSAMP_DTYPE_F32 ? 4 : 2;
  P.aligned = aligned16(a->target_logits) && (!residual || aligned16(a->draft_logits)) &&
              ((size_t)a->vocab * es) % 16 == 0;
  P.logits = a->target_logits;
  P.logits2 = residual ? a->draft_logits : a->target_logits;
  P.rows_split = (int32_t)(S * W);
  P.vwin = (int32_t)W;
  P.bonus_only = residual ? 1 : 0;
  P.params = a->params;
  P.uniforms = a->uniforms;
  P.probe_tokens = a->draft_tokens;
  if (penalized) {
    P.row_ptr = ctx->vrow_ptr;
    P.row_len = ctx->vrow_len;
    P.entries = a->penalty_scratch;
  }
  P.tokens = ctx->ws.vtokens;
  P.row_flags = ctx->ws.vflags;
  P.stats = ctx->ws.vstats;
  // the outcome reads the kept weight and the probe's; TYPICAL also the entropy
  P.stats_full = a->mode == LSAMP_VERIFY_TYPICAL;
  VerifyPlan Q{};
  Q.mode = a->mode;
  Q.sequences = a->sequences;
  Q.window = a->window;
  Q.vocab = a->vocab;
  Q.dtype = a->dtype;
  Q.semantics = LSAMP_SEM_CBV2;
  Q.typical_delta = a->typical_delta;
  Q.target = a->target_logits;
  Q.draft = a->draft_logits;
  Q.draft_tokens = a->draft_tokens;
  Q.params = a->params;
  Q.uniforms = a->uniforms;
  Q.accepted = a->accepted;
  Q.tokens = a->tokens;
  Q.accept_mask = a->accept_mask;
  Q.penalized = penalized ? 1 : 0;
  Q.parts = a->mode == LSAMP_VERIFY_RESIDUAL ? (int32_t)verify_parts((size_t)a->vocab) : 1;
  DeviceGuard guard(ctx->device);
  int err = penalized ? launch_window_entries(E, stream) : 0;
  if (err == 0) err = launch_sample(ctx->ws, P, nullptr, stream, nullptr);
  if (err == 0) err = launch_verify_finish(ctx->ws, Q, stream);
  if (err != 0)
    return fail(LSAMP_ERR_DEVICE, "kernel launch failed: %s", hipGetErrorString((hipError_t)err));
  return ok();
}

}  // extern "C"
