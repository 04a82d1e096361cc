// lsamp_kernels.hip — gfx950 kernels of the logits-to-token stage.
//
// A sampling step runs over tasks (row, slice): one 512-thread work-group
// owns one slice (<= 65536 tokens) of one row and keeps the slice's logits in
// registers from the moment they arrive from HBM until the token is drawn.
//
//  stats phase   16-byte vector loads of the slice, the grammar mask and the
//                sparse penalties applied exactly as the reference orders
//                them, then a histogram of the filter-space logit in 1/32-nat
//                bins (count + fixed-point mass, one packed 64-bit LDS atomic
//                per token).  The slices' histograms are merged on the
//                absolute bin grid and the bin holding the top-k / top-p /
//                min-p cut is located.
//  select phase  every work-group keeps the tokens above the cut bin (fixed-
//                point draw weight per 1024-token chunk, and a short list of
//                them) and lists the tokens inside it.  The last work-group of
//                the row sorts those candidates, applies the exact keep rule of
//                the row's semantics and draws the token by inverse CDF in
//                token-id order.
//
// Fused mode runs both phases in one kernel and assumes nothing about which
// work-groups are resident.  Each slice takes a start ticket on its row.  At
// the exchange a slice waits for the others' histograms only when every slice
// of the row has started (those finish their stats without waiting for
// anyone); otherwise, or when its bounded wait runs out, it leaves.  The
// slice that arrives last merges at once, does its own select, and then
// claims the select of every slice that left and does it from a re-read of
// that slice; a slice claims its own select before doing it, so each select
// runs exactly once.  The short-list rows' first exchange works the same way
// (the fallback's histograms of slices that left are claimed by the first
// exchange's last arriver).  Split mode runs the phases as two kernels (the
// last stats work-group of a row merges; the second kernel re-reads its slice
// from L2).  Neither mode uses MFMA: the stage is a bandwidth- and
// reduction-bound pass, not a contraction.
#include <hip/hip_runtime.h>

#include "lsamp_device.h"
#include "lsamp_internal.h"
#include "lsamp_row.h"

namespace lsamp {
namespace {

using namespace dev;
using namespace rowops;

constexpr int kSpinLimit = 1 << 20;                   // ~0.2 s of polling
// lsamp_test_set_spin_limit: > 0 makes every bounded wait's target unreachable and
// its limit this many polls (the waits' fail-closed path, under test)
__device__ int32_t g_spin_test = 0;

// The fused arrangement's per-row synchronisation words (in the arrive_stats
// array): arrivals at the exchange in the low half of word 0 and start
// tickets in its high half (an arrival's atomic returns both counts), claims
// (bit s: slice s's select; bit kClaimStats + s: its fallback histogram) and
// departures.  The last slice to leave returns them to zero.  (Split mode
// counts its arrivals in word 0 alone.)
constexpr int kSyncArrive = 0, kSyncClaims = 2, kSyncOut = 3;
constexpr uint32_t kStartOne = 1u << 16, kArriveMask = 0xffffu;
constexpr uint32_t kClaimStats = 8;
static_assert(kMaxSlices <= (int)kClaimStats, "claim bits of both kinds fit one word");
__device__ __forceinline__ uint32_t* row_sync(const Workspace& ws, int row) {
  return ws.arrive_stats + (size_t)kRowSyncWords * (size_t)row;
}

// Thread 0: set bit `bit` of the row's claims; true for the one caller that
// set it.
__device__ __forceinline__ bool claim_bit(uint32_t* sync, uint32_t bit) {
  const uint32_t old = __hip_atomic_fetch_or(sync + kSyncClaims, 1u << bit, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
  return ((old >> bit) & 1u) == 0u;
}

// Thread 0: the first slice from `from` on, other than `own`, whose claim
// bit `base + s` this work-group sets (and `from` moves past it); -1 when
// none is left.
__device__ __forceinline__ int claim_next(uint32_t* sync, int G, int own, uint32_t base,
                                          int& from) {
  for (; from < G; ++from) {
    if (from == own) continue;
    if (claim_bit(sync, base + (uint32_t)from)) return from++;
  }
  return -1;
}

// A bounded wait of the fused kernel (thread 0) for the row's exchange: 1
// when the arrivals reach `target`; -1 when another work-group set claim bit
// `bit` (it does that work itself, so this slice can leave); 0 when the wait
// gave up (the sticky status bit is raised, and the slice leaves).  Callers
// wait only when every slice of the row has started, so the arrivals come
// from work-groups that are running.
__device__ __forceinline__ int wait_exchange(const Workspace& ws, const uint32_t* sync,
                                             uint32_t target, uint32_t bit) {
  const int32_t test = __hip_atomic_load(&g_spin_test, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t tgt = test > 0 ? 0xffffffffu : target;
  const int lim = test > 0 ? test : kSpinLimit;
  for (int it = 0;;) {
    if ((ld_coherent(sync + kSyncArrive) & kArriveMask) >= tgt) return 1;
    // (claims are rare: every 16th poll looks)
    if ((it & 15) == 15 && ((ld_coherent(sync + kSyncClaims) >> bit) & 1u)) return -1;
    if (++it >= lim) {
      atomicOr(ws.status, kStatusSpinTimeout);
      return 0;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// A slice's last act on its row (fused arrangement, thread 0): count it out.
// Thread 0 has the results of all its other operations on the row's words
// by now (the start ticket's included), so none of them can land after a
// clear.  The old count is checked later (clear_if_last), so the round trip
// overlaps the next task's take.
__device__ __forceinline__ uint32_t leave_row(const Workspace& ws, int row) {
  return __hip_atomic_fetch_add(row_sync(ws, row) + kSyncOut, 1u, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0: the last of the row's G slices to leave clears its
// synchronisation words for the next step (every slice is done with them).
__device__ __forceinline__ void clear_if_last(const Workspace& ws, int row, int G, uint32_t out) {
  if (out + 1u == (uint32_t)G) {
    uint32_t* sync = row_sync(ws, row);
    st_coherent(sync + kSyncArrive, 0u);
    st_coherent(sync + kSyncClaims, 0u);
    st_coherent(sync + kSyncOut, 0u);
  }
}
// Buckets of the short-list finalize's counting sort (by a key's high word);
// their counts and starts live in the thread-maximum histogram.
constexpr int kRankBuckets = 512;
// The publish's LDS list holds at most kShortPub raw pairs; threads write the
// tokens that are not candidates to their own slot from here on.
constexpr int kExpandDump = kShortPub;
static_assert(kExpandDump + kThreads <= kCandCap, "dump slots fit the list area");
static_assert(2 * kRankBuckets <= kTauBins, "bucket counts and starts fit");

enum TaskMode { kFused = 0, kStatsOnly = 1, kSelectOnly = 2 };

// Token classes relative to the row's cut.
constexpr int kDrop = 0, kKept = 1, kCand = 2;

// Classification rule of a row, resolved once per task: with
// j = top - floor(x * c32) (clamped at 0), a finite token is kept when
// j < kc and a candidate when kc <= j < kd; in +inf mode exactly the +inf
// tokens are kept.
struct ClassRule {
  int32_t top, kc, kd;
  float c32;
  float screen;  // x * c32 < screen: neither kept nor candidate
  bool posinf;
  int32_t pinf_cls;  // class of a +inf token in +inf mode: kept, or (argmax
                     // rows: the first one wins) candidate
};

__device__ __forceinline__ ClassRule make_rule(const RowInfo& info, const RowCtx& c) {
  ClassRule r;
  r.top = info.top_bin;
  r.c32 = c.c32;
  r.posinf = info.mode == kModePosInf;
  r.pinf_cls = c.kind == LSAMP_KIND_ARGMAX ? kCand : kKept;
  if (info.mode != kModeNormal) {
    r.kc = r.kd = -1;
  } else if (info.cut == kCutList) {
    r.kc = 0;  // every finite token is a candidate; the kept list decides
    r.kd = 0x7fffffff;
  } else if (info.cut == kCutNone) {
    r.kc = r.kd = 0x7fffffff;
  } else if (info.cut == kCutTail) {
    r.kc = kBins;
    r.kd = 0x7fffffff;
  } else {
    r.kc = info.cut;
    r.kd = info.cut + 1;
  }
  // j < kd  <=>  floor(clamp(s)) >= top - kd + 1 =: n, implied by s >= n when
  // n > -1e9; the threshold is n rounded up to a float (s is a float).
  const int64_t n = (int64_t)r.top - (int64_t)r.kd + 1;
  if (r.posinf)
    r.screen = kPosInf;
  else if (r.kd < 0)
    r.screen = __builtin_nanf("");
  else if (n <= -1000000000ll)
    r.screen = -__FLT_MAX__;
  else
    r.screen = __int2float_ru((int)(n > 1000000001ll ? 1000000001ll : n));
  return r;
}

__device__ __forceinline__ int classify(const ClassRule& r, float x) {
  if (r.posinf) return x == kPosInf ? r.pinf_cls : kDrop;
  if (!__builtin_isfinite(x)) return kDrop;
  int j = r.top - bin_of(x, r.c32);
  j = j < 0 ? 0 : j;
  return j < r.kc ? kKept : (j < r.kd ? kCand : kDrop);
}

// ----------------------------------------------------------------- LDS
struct MergeLds {
  uint64_t mass[kBins];  // row-aligned fixed-point mass per bin
  uint32_t cnt[kBins];
};
struct SelectLds {
  Candidate cand[kWgCandCap];
  KeptItem klist[kKeptCap];
  uint64_t chunk[kSliceChunks];
};
struct FinalLds {
  uint64_t keys[kCandCap];
  uint8_t keep[kCandCap];
  uint64_t rowchunk[kMaxRowChunks];
  uint64_t dw[kChunk + kChunk / 16];  // draw slots (padded), or rank-sort scratch
  float cx[kChunk];
  uint8_t cent[kChunk];
  uint8_t cflag[kChunk];
  uint16_t qoff[kChunk];  // chunk re-read: the slots the bin screen passes
};
union PhaseLds {
  uint64_t hist[kHist + 64];  // + one discard word per lane
  MergeLds m;
  SelectLds s;
  FinalLds f;
};
// Short-list slice phase: thread-maximum histogram and the slice's candidates.
struct ShortLds {
  uint32_t tcnt[kTauBins];
  uint4 squad[(kQStage + 1) * kThreads];  // slot k of thread t at k * kThreads + t; k = kQStage discards
};
struct TaskLds {
  PhaseLds u;
  ShortLds sh;
  uint64_t ssrc[kCandCap];  // short-list finalize: the slices' published keys
  int32_t soff[kMaxSlices + 1];
  uint32_t pen[kSliceWords];
  int32_t etok[kSliceEntryCap];
  float ex[kSliceEntryCap];
  RowInfo info;
  SelectPartial part[kMaxSlices];
  float hx[kMaxSlices];
  int32_t htop[kMaxSlices];
  uint32_t hfl[kMaxSlices];
  int32_t hn[kMaxSlices];
  double hz[kMaxSlices];
  float redf[kWaves];
  float redf2[kWaves];
  int32_t redi[kWaves];
  double redd[kWaves];
  uint64_t redu[kWaves];
  uint64_t misc64[4];
  int32_t misc[8];
  int32_t ecount;
  int32_t ncand;
  int32_t nlist;
  int32_t nitems;
  int32_t last;
  // the fused arrangement's hand-off (thread 0 writes, the work-group reads)
  int32_t wait;         // the first exchange's wait: 1 reached, 0 gave up / not started, -1 claimed
  int32_t won;          // a claim of this work-group's own work succeeded
  int32_t x1;           // first exchange's last arriver of a row that fell back
  int32_t xlast;        // this work-group made the exchange's last arrival
  int32_t job;          // the slice of the claimed job, or -1
  int32_t nraw;         // raw log-probability candidates listed
  int32_t from_stats;   // claim scans: the next slice to try
  int32_t from_select;
  uint32_t flags;
  uint32_t task;  // fused kernel over several rounds: the task taken
};
// Select pass: each wave's queue of screened tokens (offset in the slice,
// value bits) lives in the short-list area, idle in that phase.
constexpr int kSelQueue = (int)(sizeof(TaskLds::ssrc) / sizeof(uint2) / kWaves);  // 512
static_assert(kSelQueue >= kThreads / kWaves * 8, "a quad step of a wave fits the queue");



// ============================================================ merge (stats)
// Merges the G slice histograms of a row (integer sums on the absolute bin
// grid) and locates the cut bin; result in L.info.  Split mode runs it in the
// last stats work-group of the row; fused mode in every work-group of the row
// once all slices have published (each computes the same result).
//
// One wave does the work with wave-level scans (no work-group barriers): one
// round trip fetches the slice headers and the top 256 bins of every slice,
// which are aligned through LDS; the bins are scanned from the top in blocks
// of 64 and the scan stops at the block holding the cut.  Deeper cuts read
// further bins, already aligned, 256 at a time.  Slices publish their own
// total mass, so the scan never needs the bins below the cut.
// The merge's first round trip, spread over the work-group: every wave reads
// the slices' top bins and counts, wave 0 the rest of the heads (kept in LDS
// for merge_wave), and wave s < G the top bins of slice s, which it adds,
// aligned to the row's top bin, into the merge arrays: 512 bins a slice when
// the row has more than 4 slices (a batch below them would cost two round
// trips), else 256 (one).  A cut in those bins needs no further round trip.
// Whole work-group.
constexpr int kMergeStageBins = 512;
__device__ __forceinline__ int merge_stage_batches(int slices) { return slices > 4 ? 2 : 1; }
__device__ __forceinline__ void merge_stage(const Workspace& ws, const SamplePlan& P, int row,
                                            const RowCtx& c, TaskLds& L) {
  constexpr int kPer = kMergeStageBins / 64;
  static_assert(kMergeStageBins <= kBins, "the staged bins fit the merge arrays");
  static_assert(kWaves >= kMaxSlices, "a wave per slice");
  const int tid = fresh_tid(), l = tid & 63, wv = tid >> 6;
  const int G = P.slices;
  const SliceSummary* summ = ws.summaries + (size_t)row * kMaxSlices;
  const bool hist_row = c.kind != LSAMP_KIND_ARGMAX;
  int32_t ht = 0, hn = 0;
  if (l < G) {
    ht = ld_coherent(&summ[l].top_bin);
    hn = ld_coherent(&summ[l].n_finite);
  }
  float hx = kNegInf;
  uint32_t hfl = 0u;
  double hz = 0.0;
  if (wv == 0 && l < G) {
    hx = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&summ[l].x_max)));
    hfl = ld_coherent(&summ[l].flags);
    hz = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&summ[l].z)));
  }
  const int per = 4 * merge_stage_batches(G);  // blocks of 64 bins staged
  uint64_t w[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    w[k] = (hist_row && wv < G && k < per) ? ld_coherent(&summ[wv].hist[64 * k + l]) : 0ull;
  for (int i = tid; i < 64 * per; i += kThreads) {
    L.u.m.cnt[i] = 0u;
    L.u.m.mass[i] = 0ull;
  }
  __syncthreads();
  // the row's top bin over the slices with a finite token (as merge_wave)
  const int32_t rt = wave_max(l < G && hn > 0 ? ht : INT32_MIN);
  const int32_t hn_w = __shfl(hn, wv < G ? wv : 0, 64);
  if (wv < G && hn_w > 0) {
    const int32_t off = rt - __shfl(ht, wv, 64);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int j = 64 * k + l + off;
      if (w[k] != 0ull && j < 64 * per) {
        atomicAdd(&L.u.m.cnt[j], (uint32_t)(w[k] >> kCountShift));
        atomicAdd(reinterpret_cast<unsigned long long*>(&L.u.m.mass[j]),
                  (unsigned long long)(w[k] & kMassMask));
      }
    }
  }
  if (wv == 0 && l < G) {
    L.hx[l] = hx;
    L.htop[l] = ht;
    L.hfl[l] = hfl;
    L.hn[l] = hn;
    L.hz[l] = hz;
  }
  __syncthreads();
}

template <bool STAGED>
__device__ __forceinline__ void merge_wave(const Workspace& ws, const SamplePlan& P, int row,
                                           const RowCtx& c, const lsamp_row_params& prm, TaskLds& L) {
  const int l = fresh_tid();  // lane, wave 0
  const int G = P.slices;
  const int64_t V = P.vocab;
  const SliceSummary* summ = ws.summaries + (size_t)row * kMaxSlices;
  const bool hist_row = c.kind != LSAMP_KIND_ARGMAX;
  constexpr int kBlk = 4;  // blocks of 64 bins per batch
  // (STAGED: merge_stage has the heads in LDS and the top staged_batches
  // batches of bins aligned there)
  const int staged_batches = STAGED ? merge_stage_batches(G) : 1;
  float hx = kNegInf;
  int32_t htop = 0, hn = 0;
  uint32_t hfl = 0u;
  double hz = 0.0;
  if (l < G) {
    if constexpr (STAGED) {
      hx = L.hx[l];
      htop = L.htop[l];
      hfl = L.hfl[l];
      hn = L.hn[l];
      hz = L.hz[l];
    } else {
      hx = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&summ[l].x_max)));
      htop = ld_coherent(&summ[l].top_bin);
      hfl = ld_coherent(&summ[l].flags);
      hn = ld_coherent(&summ[l].n_finite);
      hz = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&summ[l].z)));
    }
  }
  uint64_t w[STAGED ? 1 : kMaxSlices][kBlk];
  if constexpr (!STAGED) {
#pragma unroll
    for (int s = 0; s < kMaxSlices; ++s)
#pragma unroll
      for (int k = 0; k < kBlk; ++k)
        w[s][k] = (hist_row && s < G) ? ld_coherent(&summ[s].hist[64 * k + l]) : 0ull;
  }

  float row_max = kNegInf;
  int32_t row_top = 0, n_total = 0;
  uint32_t rflags = 0u;
  bool first = true;
  for (int s = 0; s < G; ++s) {
    const float xs = __shfl(hx, s, 64);
    const int32_t ts = __shfl(htop, s, 64);
    const int32_t ns = __shfl(hn, s, 64);
    rflags |= (uint32_t)__shfl((int)hfl, s, 64);
    n_total += ns;
    if (ns > 0) {
      if (first || xs > row_max) row_max = xs;
      if (first || ts > row_top) row_top = ts;
      first = false;
    }
  }
  RowInfo info;
  info.x_max = row_max;
  info.top_bin = row_top;
  info.flags = rflags & LSAMP_ROW_NONFINITE;
  if (rflags & kSliceEntryOverflow) info.flags |= LSAMP_ROW_OVERFLOW;
  info.n_finite = n_total;
  info.mode = (rflags & kSlicePosInf) ? kModePosInf : (n_total == 0 ? kModeEmpty : kModeNormal);
  info.cut = kCutNone;
  info.count_above = n_total;
  info.mass_above = 0.0;
  info.z = 0.0;
  info.p_limit = -1.0;
  info.kept_cands = 0;
  info.done = 0;
  const float s_top = bin_pos(row_max, c.c32);
  // masses are relative to e^q_top, q_top the row's top in filter units
  info.q_top = (float)((double)s_top / (32.0 * c.tf));
  const double q_ref = (double)info.q_top;
  const double bin_t = 1.0 / (32.0 * c.tf);  // filter units per bin

  if (c.kind == LSAMP_KIND_ARGMAX && info.mode != kModeEmpty) {
    // the first maximum: every token of the top bin (in +inf mode every +inf
    // token) is a candidate and the finalize keeps the first in id order
    info.cut = 0;
    info.count_above = 0;
  } else if (info.mode == kModeNormal) {
    const double inv_frac = 1.0 / (double)(1ull << kMassFracBits);
    // total mass relative to the row top: each slice's total is relative to
    // its own top bin
    const double z = wave_sum((l < G && hn > 0) ? hz * fexp((double)(htop + 1) * bin_t - q_ref)
                                                : 0.0);
    info.z = z;
    const int32_t k_lim = (prm.top_k > 0 && (int64_t)prm.top_k < V) ? prm.top_k : 0;
    const double P_lim = top_p_limit(P, c, prm, z);
    const bool p_on = P_lim >= 0.0;
    // CBv2 keeps exclusive mass <= P; mlx-lm keeps mass-before < P
    const bool strict = P.semantics != LSAMP_SEM_CBV2;
    const bool k_on = c.kind == LSAMP_KIND_FILTERED && k_lim > 0;
    const float mp = prm.min_p > 1.0f ? 1.0f : prm.min_p;
    const bool m_on = c.kind == LSAMP_KIND_FILTERED && mp > 0.0f;
    int32_t j_t = kBins + 1;
    if (m_on) {
      const float st = s_top + (float)(32.0 * c.tf) * __builtin_logf(mp);
      j_t = row_top - (int32_t)__builtin_floorf(__builtin_fmaxf(st, -1.0e9f));
      if (j_t < 0) j_t = 0;
      if (j_t > kBins) j_t = kBins;
    }
    info.p_limit = P_lim;

    if constexpr (!STAGED) {
      // batch 0: align the top 256 bins of every slice in LDS
#pragma unroll
      for (int k = 0; k < kBlk; ++k) {
        L.u.m.cnt[64 * k + l] = 0u;
        L.u.m.mass[64 * k + l] = 0ull;
      }
#pragma unroll
      for (int s = 0; s < kMaxSlices; ++s) {
        if (s >= G) break;
        const int32_t off = row_top - __shfl(htop, s, 64);
#pragma unroll
        for (int k = 0; k < kBlk; ++k) {
          const int j = 64 * k + l + off;
          if (w[s][k] != 0ull && j < 64 * kBlk) {
            atomicAdd(&L.u.m.cnt[j], (uint32_t)(w[s][k] >> kCountShift));
            atomicAdd(reinterpret_cast<unsigned long long*>(&L.u.m.mass[j]),
                      (unsigned long long)(w[s][k] & kMassMask));
          }
        }
      }
    }
    int32_t carry_c = 0;
    double carry_m = 0.0;
    int cut = -1;
    int32_t cut_c = 0;
    double cut_m = 0.0;
    for (int b = 0; b < kBins / (64 * kBlk) && cut < 0; ++b) {
      uint32_t cnt[kBlk];
      uint64_t msum[kBlk];
      if (b < staged_batches) {
#pragma unroll
        for (int k = 0; k < kBlk; ++k) {
          cnt[k] = L.u.m.cnt[64 * kBlk * b + 64 * k + l];
          msum[k] = L.u.m.mass[64 * kBlk * b + 64 * k + l];
        }
      } else {
        // deeper batch: read the slices' bins already aligned, four slices'
        // requests out before the first is used (one round trip a batch up
        // to four slices)
#pragma unroll
        for (int k = 0; k < kBlk; ++k) {
          cnt[k] = 0u;
          msum[k] = 0ull;
        }
        constexpr int kGrp = 4;
        for (int s0 = 0; s0 < G; s0 += kGrp) {
          uint64_t wg[kGrp][kBlk];
#pragma unroll
          for (int d = 0; d < kGrp; ++d) {
            const int s = s0 + d;
            const bool live = s < G && __shfl(hn, s, 64) > 0;
            const int32_t off = row_top - __shfl(htop, s, 64);
#pragma unroll
            for (int k = 0; k < kBlk; ++k) {
              const int i = 64 * kBlk * b + 64 * k + l - off;
              wg[d][k] = (live && i >= 0 && i < kBins) ? ld_coherent(&summ[s].hist[i]) : 0ull;
            }
          }
#pragma unroll
          for (int d = 0; d < kGrp; ++d)
#pragma unroll
            for (int k = 0; k < kBlk; ++k) {
              cnt[k] += (uint32_t)(wg[d][k] >> kCountShift);
              msum[k] += wg[d][k] & kMassMask;
            }
        }
      }
#pragma unroll
      for (int k = 0; k < kBlk; ++k) {
        if (cut >= 0) break;
        const int j = 64 * kBlk * b + 64 * k + l;
        const int32_t cj = (int32_t)cnt[k];
        const double mj = cj ? (double)msum[k] * inv_frac *
                                   fexp((double)(row_top - j + 1) * bin_t - q_ref)
                             : 0.0;
        const int32_t ic = wave_incl_scan(cj);
        const double im = wave_incl_scan(mj);
        const int32_t C = carry_c + ic - cj;
        const double M = carry_m + im - mj;
        bool hit = false;
        if (cj > 0 || (m_on && j == j_t)) {
          const bool tk = k_on && C + cj >= k_lim;
          const bool tp = p_on && cj > 0 && (strict ? (M + mj >= P_lim) : (M + mj > P_lim));
          const bool tm = m_on && j >= j_t;
          hit = tk || tp || tm;
        }
        const uint64_t hits = __ballot(hit);
        if (hits) {
          const int f = __builtin_ctzll(hits);
          cut = 64 * kBlk * b + 64 * k + f;
          cut_c = __shfl(C, f, 64);
          cut_m = __shfl(M, f, 64);
        } else {
          carry_c += __shfl(ic, 63, 64);
          carry_m += __shfl(im, 63, 64);
        }
      }
    }
    if (cut >= 0) {
      info.cut = cut;
      info.count_above = cut_c;
      info.mass_above = cut_m;
    } else {
      // carry_* now hold the whole window; the rest of the row is the tail
      const bool tk = k_on && n_total >= k_lim;
      const bool tp = p_on && n_total > carry_c && (strict ? (z >= P_lim) : (z > P_lim));
      const bool tm = m_on && j_t >= kBins;
      if (tk || tp || tm) {
        info.cut = kCutTail;
        info.count_above = carry_c;
        info.mass_above = carry_m;
      } else {
        info.cut = kCutNone;
        info.count_above = n_total;
        info.mass_above = z;
      }
    }
  }
  if (l == 0) L.info = info;
}

__device__ __forceinline__ void merge_row(const Workspace& ws, const SamplePlan& P, int row, const RowCtx& c,
                          const lsamp_row_params& prm, TaskLds& L) {
  if (threadIdx.x < 64) merge_wave<false>(ws, P, row, c, prm, L);
  __syncthreads();
}

// ========================================================= finalize (select)
// Last select work-group of a row: exact cut among the candidates, kept
// weights per chunk, and the inverse-CDF draw.  Only the sort of more than 64
// candidates uses the whole work-group; everything else runs in wave 0 with
// wave-level scans (no work-group barriers), and the other waves leave.
constexpr int kChunksPerLane = kMaxRowChunks / 64;  // chunk sums held per lane
constexpr int kSlotsPerLane = kChunk / 64;           // draw slots per lane

// LDS slot of offset o (0..1023) within the drawn chunk: lane-contiguous runs
// of kSlotsPerLane with one pad word per run (no bank conflicts).
__device__ __forceinline__ int draw_slot(int o) { return o + (o >> 4); }

// The row's raw log-probabilities, once its token is drawn (defined with
// the rest of the in-pass log-probabilities below).
template <int DT>
__device__ __forceinline__ void raw_chosen(const SamplePlan& P, const FusedLp& lp, int row,
                                           int32_t tok, const char* rowp);
template <int DT>
__device__ __forceinline__ void raw_lists(const SamplePlan& P, const FusedLp& lp, int row,
                                          uint64_t* lists);

// What the finalize tail needs besides the sorted candidates in F.keys.
struct TailIn {
  int nc;           // candidates in F.keys, sorted by cand_key descending
  bool overflow;    // the row's keep set could not be resolved
  double ent_all;   // kept tokens outside the candidates: entropy numerator,
  float min_all;    //   smallest kept value,
  int32_t kept_all; //   count
  float u_draw;
  int32_t probe;
  bool probe_x_set; // probe_x holds the probe's logit (loaded early)
  float probe_x;
  int32_t n_list;   // lane s < G: kept tokens slice s listed (> kKeptCap: incomplete)
  bool reset;       // clear the row's select counters (histogram path)
  int32_t done;     // RowInfo.done of the written row decision
};

// Keep rule over the sorted candidates, the draw, the probe and the outputs
// (wave 0 of the finalizing work-group).
template <int DT>
__device__ __forceinline__ void finalize_tail(const Workspace& ws, const SamplePlan& P, int row,
                                              const RowCtx& c, const lsamp_row_params& prm,
                                              const RowInfo& info, TaskLds& L, const char* rowp,
                                              const uint32_t* mrow, const TailIn& t,
                                              uint64_t (&rch)[kChunksPerLane],
                                              const FusedLp* lp) {
  const int l = fresh_tid() & 63;
  const int64_t V = P.vocab;
  const float y_max = info.mode == kModePosInf ? kPosInf : to_filter(c, info.x_max);
  const bool active = info.mode != kModeEmpty;
  Candidate* rc = ws.cands + (size_t)row * kCandCap;
  FinalLds& F = L.u.f;
  const int nc = t.nc;
  const bool overflow = t.overflow;
  const float u_draw = t.u_draw;
  const int32_t probe = t.probe;
  // ---- keep rule over the sorted candidates, 64 at a time
  const double P_lim = info.p_limit;
  const bool p_on = P_lim >= 0.0;
  const int32_t k_lim = (c.kind == LSAMP_KIND_FILTERED && prm.top_k > 0 && (int64_t)prm.top_k < V)
                            ? prm.top_k
                            : (c.kind == LSAMP_KIND_ARGMAX ? 1 : 0);
  const float mp = prm.min_p > 1.0f ? 1.0f : prm.min_p;
  const bool m_on = c.kind == LSAMP_KIND_FILTERED && mp > 0.0f;
  const float ln_mp = m_on ? __builtin_logf(mp) : 0.0f;
  const bool mlx = P.semantics == LSAMP_SEM_MLXLM;
#pragma unroll
  for (int i = 0; i < kChunksPerLane; ++i) F.rowchunk[kChunksPerLane * l + i] = rch[i];
  __builtin_amdgcn_wave_barrier();
  double carry_e = 0.0;
  int32_t carry_s = 0, carry_k = 0;
  double cent = 0.0;
  float cmin = kPosInf;
  for (int r0 = 0; r0 < nc; r0 += 64) {
    const int r = r0 + l;
    const bool in = r < nc;
    const uint64_t key = in ? F.keys[r] : 0ull;
    const uint32_t kr = (uint32_t)(key >> 32);
    const float y = key_to_float(kr);
    const double e = in ? (double)__builtin_expf(y - info.q_top) : 0.0;
    const double ie = wave_incl_scan(e);
    const double e_excl = carry_e + ie - e;
    bool keep_p = true, keep_m = true;
    if (mlx) {
      // tie group [g0, g1) of equal values (sorted by id ascending): its
      // edges inside the block from the lanes' neighbours (two ballots);
      // a group that crosses the block's edge is searched in LDS
      // (the lane moves run on every lane: a lane move inside a branch
      // would read the lanes the branch leaves out)
      const uint32_t up = (uint32_t)__shfl_up((int)kr, 1, 64);
      const uint32_t dn = (uint32_t)__shfl_down((int)kr, 1, 64);
      const uint32_t kprev = l > 0 ? up : (r0 > 0 ? (uint32_t)(F.keys[r0 - 1] >> 32) : ~kr);
      const uint32_t knext = l < 63 ? dn : (r0 + 64 < nc ? (uint32_t)(F.keys[r0 + 64] >> 32) : ~kr);
      const uint64_t starts = __ballot(in && (r == 0 || kprev != kr));
      const uint64_t ends = __ballot(in && (r == nc - 1 || knext != kr));
      if (in) {
        const uint64_t below = starts & (~0ull >> (63 - l));  // starts at lanes <= l
        const uint64_t above = ends & (~0ull << l);           // ends at lanes >= l
        int g0, g1;
        if (below) {
          g0 = r0 + 63 - __builtin_clzll(below);
        } else {
          int lo = 0, hi = r;
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if ((uint32_t)(F.keys[mid] >> 32) == kr) hi = mid; else lo = mid + 1;
          }
          g0 = lo;
        }
        if (above) {
          g1 = r0 + __builtin_ctzll(above) + 1;
        } else {
          int lo = r, hi = nc - 1;
          while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if ((uint32_t)(F.keys[mid] >> 32) == kr) lo = mid; else hi = mid - 1;
          }
          g1 = lo + 1;
        }
        // mass ranked strictly before r when equal values put higher ids first
        // (ascending stable argsort, Evaluate.swift:463-469)
        const double sp = info.mass_above + e_excl - (double)(r - g0) * e + (double)(g1 - 1 - r) * e;
        if (p_on) keep_p = sp < P_lim;
        if (m_on) keep_m = (y - y_max) >= ln_mp;
      }
    } else {
      const double sr = info.mass_above + e_excl;
      if (p_on) keep_p = sr <= P_lim;
      if (m_on) keep_m = __builtin_expf(y - y_max) >= mp;
      const int64_t rank = (int64_t)info.count_above + r;
      if (k_lim > 0 && rank >= k_lim) keep_p = false;
    }
    const int32_t surv = (in && keep_p && keep_m) ? 1 : 0;
    const int32_t is = wave_incl_scan(surv);
    bool keep = surv != 0;
    if (keep && mlx && k_lim > 0) keep = ((int64_t)info.count_above + carry_s + is - 1) < k_lim;
    const int32_t kk = keep ? 1 : 0;
    const int32_t ik = wave_incl_scan(kk);
    if (in) F.keep[r] = keep ? 1 : 0;
    if (keep) {
      const int32_t id = key_id(key);
      const uint64_t wgt = weight(y, y_max, c.scale);
      atomicAdd(reinterpret_cast<unsigned long long*>(&F.rowchunk[id / kChunk]), (unsigned long long)wgt);
      cent += (double)wgt * (1.0 / 1099511627776.0) * (double)weight_arg(y, y_max, c.scale);
      cmin = __builtin_fminf(cmin, y);
      // kept candidates persist (sorted) for the MTP residual pass
      const int32_t slot = carry_k + ik - 1;
      rc[slot].y = y;
      rc[slot].id = id;
    }
    if (in && P.keep) P.keep[(size_t)row * (size_t)V + key_id(key)] = keep ? 1 : 0;
    carry_e += read_lane(ie, 63);
    carry_s += read_lane(is, 63);
    carry_k += read_lane(ik, 63);
  }
  cent = wave_sum(cent);
  cmin = wave_min(cmin);
  const int32_t kept_c = carry_k;
  __builtin_amdgcn_wave_barrier();

  // ---- total weight and the chunk holding the target
  uint64_t lane_w = 0ull;
#pragma unroll
  for (int i = 0; i < kChunksPerLane; ++i) {
    rch[i] = F.rowchunk[kChunksPerLane * l + i];
    lane_w += rch[i];
  }
  const uint64_t iw = wave_incl_scan(lane_w);
  const uint64_t W = read_lane(iw, 63);
  const uint64_t target = W ? scaled_target(uniform_u32(u_draw), W) : 0ull;
  int my_c = -1;
  uint64_t my_t = 0ull;
  {
    uint64_t pre = iw - lane_w;
#pragma unroll
    for (int i = 0; i < kChunksPerLane; ++i) {
      if (rch[i] && pre <= target && target < pre + rch[i]) {
        my_c = kChunksPerLane * l + i;
        my_t = target - pre;
      }
      pre += rch[i];
    }
  }
  const uint64_t hitc = __ballot(my_c >= 0);
  int cstar = -1;
  uint64_t ltarget = 0ull;
  // (a verify row whose draw nobody reads keeps only its weights)
  const bool draw = !P.bonus_only || (row < P.rows_split && row % P.vwin == P.vwin - 1);
  if (W && hitc && !overflow && active && draw) {
    const int f = __builtin_ctzll(hitc);
    cstar = read_lane(my_c, f);
    ltarget = read_lane(my_t, f);
  }

  // ---- the token inside the chunk: inverse CDF in id order over draw slots
  int token = -1;
  if (cstar >= 0) {
    const int32_t cb = cstar * kChunk;
    const int32_t ce = cb + kChunk < V ? cb + kChunk : (int32_t)V;
    const int cps = P.slice_len / kChunk;
    const int sc = cstar / cps;
    const int32_t n_list = __shfl(t.n_list, sc, 64);
#pragma unroll
    for (int i = 0; i < kSlotsPerLane; ++i) F.dw[draw_slot(kSlotsPerLane * l + i)] = 0ull;
    __builtin_amdgcn_wave_barrier();
    if (n_list <= kKeptCap) {
      // fast path: the kept tokens of this chunk are all listed
      const KeptItem* kl = ws.klist + ((size_t)row * kMaxSlices + sc) * kKeptCap;
#pragma unroll
      for (int k = 0; k < kKeptCap / 64; ++k) {
        const int i = 64 * k + l;
        if (i < n_list) {
          const int32_t id = ld_coherent(&kl[i].id);
          if (id >= cb && id < ce) F.dw[draw_slot(id - cb)] = ld_coherent(&kl[i].w);
        }
      }
      for (int r = l; r < nc; r += 64) {
        if (!F.keep[r]) continue;
        const int32_t id = key_id(F.keys[r]);
        if (id >= cb && id < ce) F.dw[draw_slot(id - cb)] = weight(key_y(F.keys[r]), y_max, c.scale);
      }
    } else {
      // re-read the chunk: every token's transformed value and class
      for (int i = l; i < kChunk / 4; i += 64) {
        reinterpret_cast<uint32_t*>(F.cent)[i] = 0u;
        reinterpret_cast<uint32_t*>(F.cflag)[i] = 0u;
      }
      __builtin_amdgcn_wave_barrier();
      for (int r = l; r < nc; r += 64) {
        if (!F.keep[r]) continue;
        const int32_t id = key_id(F.keys[r]);
        if (id >= cb && id < ce) F.cflag[id - cb] = 1;
      }
      int32_t e0 = 0, e1 = 0;
      if (P.row_ptr && P.entries) {
        e0 = P.row_ptr[row];
        e1 = P.row_len ? e0 + P.row_len[row] : P.row_ptr[row + 1];
      }
      // (the lane's kSlotsPerLane contiguous tokens, requested at once with
      // the entries, ahead of the patches that need them)
      constexpr int NV = kSlotsPerLane / Vec<DT>::N;
      const int64_t i0 = cb + kSlotsPerLane * l;
      uint4 lv[NV];
#pragma unroll
      for (int v = 0; v < NV; ++v) lv[v] = load_vec<DT>(rowp, i0 + v * Vec<DT>::N, ce, P.aligned != 0);
#pragma unroll 4
      for (int32_t e = e0 + l; e < e1; e += 64) {
        const lsamp_penalty_entry ent = P.entries[e];
        if (ent.token < cb || ent.token >= ce) continue;
        float x = load_scalar<DT>(rowp, ent.token);
        x = patch_value(c, prm, x, ent, DT);
        if (!mask_allows(mrow, P.mask_words, P.mask_bits, P.mask_tail, ent.token)) x = kNegInf;
        if (x != x) x = kNegInf;
        F.cx[ent.token - cb] = x;
        F.cent[ent.token - cb] = 1;
      }
      __builtin_amdgcn_wave_barrier();
      const ClassRule rule = make_rule(info, c);
      const uint32_t allow =
          mask_allow_bits(mrow, P.mask_words, P.mask_bits, P.mask_tail, (int32_t)i0, kSlotsPerLane);
      // every slot's value to LDS; the slots the bin screen passes (kept and
      // cut-bin tokens) are listed, then classified and weighed a slot per
      // lane, so the wave does not run the weight once per lane holding one
      uint32_t m = 0u;
#pragma unroll
      for (int i = 0; i < kSlotsPerLane; ++i) {
        const int o = kSlotsPerLane * l + i;
        float x = F.cent[o] ? F.cx[o]
                            : (((allow >> i) & 1u) ? vec_elem<DT>(lv[i / Vec<DT>::N], i % Vec<DT>::N)
                                                   : kNegInf);
        if (x != x) x = kNegInf;
        F.cx[o] = x;
        m |= (cb + o < ce && x * rule.c32 >= rule.screen ? 1u : 0u) << i;
      }
      static_assert(kSlotsPerLane <= 16, "slot counts take five ballots");
      const int cnt = __builtin_popcount(m);
      int off = 0, tot = 0;
#pragma unroll
      for (int b = 0; b < 5; ++b) {
        const uint64_t bl = __ballot((cnt >> b) & 1);
        off += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bl >> 32),
                                              __builtin_amdgcn_mbcnt_lo((uint32_t)bl, 0u))
               << b;
        tot += __builtin_popcountll(bl) << b;
      }
#pragma unroll
      for (int i = 0; i < kSlotsPerLane; ++i)
        if ((m >> i) & 1u) F.qoff[off++] = (uint16_t)(kSlotsPerLane * l + i);
      __builtin_amdgcn_wave_barrier();
      for (int j = l; j < tot; j += 64) {
        const int o = F.qoff[j];
        const float x = F.cx[o];
        const int cls = classify(rule, x);
        if (cls == kKept || (cls == kCand && F.cflag[o]))
          F.dw[draw_slot(o)] = weight(to_filter(c, x), y_max, c.scale);
      }
    }
    __builtin_amdgcn_wave_barrier();
    uint64_t sw[kSlotsPerLane];
    uint64_t lane_s = 0ull;
#pragma unroll
    for (int i = 0; i < kSlotsPerLane; ++i) {
      sw[i] = F.dw[draw_slot(kSlotsPerLane * l + i)];
      lane_s += sw[i];
    }
    const uint64_t is = wave_incl_scan(lane_s);
    uint64_t pre = is - lane_s;
    int my_tok = -1;
#pragma unroll
    for (int i = 0; i < kSlotsPerLane; ++i) {
      if (sw[i] && pre <= ltarget && ltarget < pre + sw[i]) my_tok = cb + kSlotsPerLane * l + i;
      pre += sw[i];
    }
    const uint64_t hitt = __ballot(my_tok >= 0);
    if (hitt) token = read_lane(my_tok, __builtin_ctzll(hitt));
  }

  // ---- probe token (MTP acceptance): its kept weight
  uint64_t probe_w = 0ull;
  if (probe >= 0 && probe < V && !overflow && active) {
    bool kc = false;
    for (int r = l; r < nc; r += 64)
      if (F.keep[r] && key_id(F.keys[r]) == probe) kc = true;
    const bool kept_cand = __ballot(kc) != 0ull;
    int32_t e0 = 0, e1 = 0;
    if (P.row_ptr && P.entries) {
      e0 = P.row_ptr[row];
      e1 = P.row_len ? e0 + P.row_len[row] : P.row_ptr[row + 1];
    }
    int32_t pe = -1;
    for (int32_t e = e0 + l; e < e1; e += 64)
      if (P.entries[e].token == probe) pe = e;
    const uint64_t hp = __ballot(pe >= 0);
    float x;
    const float xr = t.probe_x_set ? t.probe_x : load_scalar<DT>(rowp, probe);
    if (hp) {
      const int32_t e = read_lane(pe, __builtin_ctzll(hp));
      x = patch_value(c, prm, xr, P.entries[e], DT);
    } else {
      x = xr;
    }
    if (!mask_allows(mrow, P.mask_words, P.mask_bits, P.mask_tail, probe) || x != x) x = kNegInf;
    const int cls = classify(make_rule(info, c), x);
    probe_w = (cls == kKept || (cls == kCand && kept_cand)) ? weight(to_filter(c, x), y_max, c.scale)
                                                             : 0ull;
  }

  if (l == 0) {
    uint32_t flags = info.flags;
    if (overflow) flags |= LSAMP_ROW_OVERFLOW;
    if (!overflow && ((draw && token < 0) || W == 0ull)) flags |= LSAMP_ROW_EMPTY;
    const int tok = overflow ? -1 : token;
    P.tokens[row] = tok;
    if (P.row_flags) P.row_flags[row] = flags;
    if (P.stats) {
      lsamp_row_stats st;
      st.max_value = y_max;
      st.log_normalizer =
          info.z > 0.0 ? __builtin_logf((float)info.z) + (info.q_top - y_max) : 0.0f;
      st.kept = t.kept_all + kept_c;
      st.token = tok;
      st.kept_weight = W;
      st.probe_weight = probe_w;
      st.cut_value = __builtin_fminf(t.min_all, cmin);
      const double zk = (double)W * (1.0 / 1099511627776.0);
      st.kept_mass = (float)zk;
      st.kept_entropy = zk > 0.0 ? __builtin_logf((float)zk) - (float)((t.ent_all + cent) / zk) : 0.0f;
      st.probe_prob = W ? (float)((double)probe_w / (double)W) : 0.0f;
      P.stats[row] = st;
    }
    RowInfo out = info;
    out.kept_cands = overflow ? 0 : kept_c;
    out.done = t.done;
    ws.rows[row] = out;
    if (t.reset) {
      // (every select of the row has arrived: nothing counts on these any
      // more this step; the exchange's words are cleared by the last slice
      // to leave the row, or, in split mode, by the stats kernel)
      ws.cand_count[row] = 0u;
      ws.arrive_select[row] = 0u;
    }
  }
  if (lp) raw_chosen<DT>(P, *lp, row, overflow ? -1 : token, rowp);
}


template <int DT>
__device__ __forceinline__ void finalize_row(const Workspace& ws, const SamplePlan& P, int row, const RowCtx& c,
                             const lsamp_row_params& prm, const RowInfo& info, TaskLds& L,
                             const char* rowp, const uint32_t* mrow, const FusedLp* lp) {
  const int tid = fresh_tid();
  const int l = tid & 63;
  const bool wave0 = tid < 64;
  const int G = P.slices;
  const int nch_row = P.nchunks;
  const bool active = info.mode != kModeEmpty;
  uint64_t* rowchunks = ws.chunk_w + (size_t)row * (size_t)ws.max_chunks;
  Candidate* rc = ws.cands + (size_t)row * kCandCap;
  FinalLds& F = L.u.f;

  // ---- wave 0 issues every independent load at once
  SelectPartial part{};
  uint64_t rch[kChunksPerLane];
  // candidate tid, read before the count is known (slots past it are ignored)
  uint64_t key0;
  {
    const float cy = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&rc[tid].y)));
    key0 = cand_key(cy, ld_coherent(&rc[tid].id));
  }
  float u_draw = 0.0f;
  int32_t probe = -1, total_cand = 0;
  float probe_x = kNegInf;
  if (wave0) {
    if (l < G) {
      const SelectPartial* sp = ws.partials + (size_t)row * kMaxSlices + l;
      part.ent = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&sp->ent)));
      part.min_kept = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&sp->min_kept)));
      part.n_kept = ld_coherent(&sp->n_kept);
      part.n_cand = ld_coherent(&sp->n_cand);
      part.n_list = ld_coherent(&sp->n_list);
      part.overflow = ld_coherent(&sp->overflow);
    }
#pragma unroll
    for (int i = 0; i < kChunksPerLane; ++i) {
      const int ci = kChunksPerLane * l + i;
      rch[i] = ci < nch_row ? ld_coherent(&rowchunks[ci]) : 0ull;
    }
    int32_t tc = 0;
    float u = 0.0f;
    int32_t pr = -1;
    if (l == 0) {
      tc = (int32_t)ld_coherent(&ws.cand_count[row]);
      if (P.uniforms)
        u = P.uniforms[uniform_index(P, row)];
      else if (P.philox_keys)
        u = philox_uniform(P.philox_keys[row], 0u);
      const int pi = probe_index(P, row);
      pr = (P.probe_tokens && pi >= 0) ? P.probe_tokens[pi] : -1;
    }
    total_cand = read_lane(tc, 0);
    u_draw = read_lane(u, 0);
    probe = read_lane(pr, 0);
    // the probe's logit, requested now: it is needed only at the end
    if (probe >= 0 && probe < P.vocab) probe_x = load_scalar<DT>(rowp, probe);
  }
  // ---- row-wide partials (wave 0), shared through LDS with the other waves
  double ent_all = 0.0;
  float min_all = kPosInf;
  int32_t kept_all = 0;
  bool overflow = false;
  int nc = 0;
  if (wave0) {
    const bool in = l < G;
    ent_all = wave_sum(in ? part.ent : 0.0);
    min_all = wave_min(in ? part.min_kept : kPosInf);
    kept_all = wave_sum(in ? part.n_kept : 0);
    const int32_t ov = wave_max(in && (part.n_cand > kWgCandCap || part.overflow) ? 1 : 0);
    overflow = (info.flags & LSAMP_ROW_OVERFLOW) != 0 || ov != 0 || total_cand > kCandCap;
    nc = (overflow || !active) ? 0 : total_cand;
    if (l == 0) L.misc[1] = nc;
  }
  __syncthreads();
  nc = L.misc[1];

  // ---- sort candidates: value descending, id ascending (-0 == +0)
  if (nc > 64 && nc <= kThreads) {
    // rank by counting (keys are distinct: ids are): one barrier
    if (tid < nc) F.dw[tid] = key0;
    __syncthreads();
    if (tid < nc) {
      int rank = 0;
      for (int i = 0; i < nc; ++i) rank += F.dw[i] > key0 ? 1 : 0;
      F.keys[rank] = key0;
    }
    __syncthreads();
  } else if (nc > 64) {
    int n2 = 1;
    while (n2 < nc) n2 <<= 1;
    for (int i = tid; i < n2; i += kThreads) {
      uint64_t key = 0ull;
      if (i < nc) {
        const float y = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&rc[i].y)));
        key = cand_key(y, ld_coherent(&rc[i].id));
      }
      F.keys[i] = key;
    }
    __syncthreads();
    for (int kk = 2; kk <= n2; kk <<= 1) {
      for (int jj = kk >> 1; jj > 0; jj >>= 1) {
        for (int i = tid; i < n2; i += kThreads) {
          const int ixj = i ^ jj;
          if (ixj > i) {
            const uint64_t a = F.keys[i], b = F.keys[ixj];
            const bool desc = (i & kk) == 0;
            if (desc ? (a < b) : (a > b)) {
              F.keys[i] = b;
              F.keys[ixj] = a;
            }
          }
        }
        __syncthreads();
      }
    }
  }
  if (!wave0) {
    // (wave 1: the raw log-probability lists, beside wave 0's draw, in the
    // staging area no finalize uses)
    if (lp && tid < 128) raw_lists<DT>(P, *lp, row, reinterpret_cast<uint64_t*>(L.sh.squad));
    return;
  }
  if (nc > 0 && nc <= 64) {
    // rank sort of the wave's own keys (keys are distinct: ids are)
    const uint64_t key = l < nc ? key0 : 0ull;
    F.dw[l] = key;
    __builtin_amdgcn_wave_barrier();
    int rank = 0;
    for (int i = 0; i < nc; ++i) rank += F.dw[i] > key ? 1 : 0;
    __builtin_amdgcn_wave_barrier();
    if (l < nc) F.keys[rank] = key;
    __builtin_amdgcn_wave_barrier();
  }

  TailIn t;
  t.nc = nc;
  t.overflow = overflow;
  t.ent_all = ent_all;
  t.min_all = min_all;
  t.kept_all = kept_all;
  t.u_draw = u_draw;
  t.probe = probe;
  t.probe_x_set = true;
  t.probe_x = probe_x;
  t.n_list = part.n_list;
  t.reset = true;
  t.done = 0;
  finalize_tail<DT>(ws, P, row, c, prm, info, L, rowp, mrow, t, rch, lp);
}

// Single-wave tail of a short-list row with at most 64 candidates (lane r
// holds F.keys[r]): the keep rule of finalize_tail with nothing kept above
// the candidates, the same integer inverse-CDF draw in token-id order, the
// probe and the outputs.
template <int DT>
__device__ __forceinline__ void short_tail(const Workspace& ws, const SamplePlan& P, int row,
                                           const RowCtx& c, const lsamp_row_params& prm,
                                           const RowInfo& info, TaskLds& L, int nc, float u_draw,
                                           int32_t probe, const char* rowp, const FusedLp* lp) {
  const int l = fresh_tid() & 63;
  const int64_t V = P.vocab;
  FinalLds& F = L.u.f;
  const float y_max = to_filter(c, info.x_max);
  const bool in = l < nc;
  const uint64_t key = in ? F.keys[l] : 0ull;
  const float y = key_y(key);
  const int32_t id = key_id(key);
  const double P_lim = info.p_limit;
  const bool p_on = P_lim >= 0.0;
  const int32_t k_lim = (c.kind == LSAMP_KIND_FILTERED && prm.top_k > 0 && (int64_t)prm.top_k < V)
                            ? prm.top_k
                            : (c.kind == LSAMP_KIND_ARGMAX ? 1 : 0);
  const float mp = prm.min_p > 1.0f ? 1.0f : prm.min_p;
  const bool m_on = c.kind == LSAMP_KIND_FILTERED && mp > 0.0f;
  const float ln_mp = m_on ? __builtin_logf(mp) : 0.0f;
  const bool mlx = P.semantics == LSAMP_SEM_MLXLM;
  const double e = in ? (double)__builtin_expf(y - info.q_top) : 0.0;
  const double e_excl = wave_incl_scan(e) - e;
  bool keep_p = true, keep_m = true;
  if (mlx) {
    if (in) {
      // tie group [g0, g1) of equal values; the reference's ascending stable
      // argsort ranks higher ids of a tie first (Evaluate.swift:463-469)
      const uint32_t kr = (uint32_t)(key >> 32);
      int g0 = l, g1 = l + 1;
      while (g0 > 0 && (uint32_t)(F.keys[g0 - 1] >> 32) == kr) --g0;
      while (g1 < nc && (uint32_t)(F.keys[g1] >> 32) == kr) ++g1;
      const double sp = e_excl - (double)(l - g0) * e + (double)(g1 - 1 - l) * e;
      if (p_on) keep_p = sp < P_lim;
      if (m_on) keep_m = (y - y_max) >= ln_mp;
    }
  } else {
    if (p_on) keep_p = e_excl <= P_lim;
    if (m_on) keep_m = __builtin_expf(y - y_max) >= mp;
    if (k_lim > 0 && l >= k_lim) keep_p = false;
  }
  const int32_t surv = (in && keep_p && keep_m) ? 1 : 0;
  bool keep = surv != 0;
  int32_t ik, kept_c;  // this lane's place among the kept (1-based), their count
  if (mlx) {
    const int32_t is = wave_incl_scan(surv);
    if (keep && k_lim > 0) keep = (is - 1) < k_lim;
    ik = wave_incl_scan(keep ? 1 : 0);
    kept_c = read_lane(ik, 63);
  } else {
    // each rule keeps a prefix of the sorted candidates, so the kept are one
    kept_c = (int32_t)__popcll(__ballot(keep));
    ik = l + 1;
  }
  const uint64_t w = keep ? weight(y, y_max, c.scale) : 0ull;
  // the kept tokens in id order (each kept lane counts the kept ids below
  // its own), then a running sum: the token is the one whose run crosses the
  // target
  int32_t* sid = reinterpret_cast<int32_t*>(F.cx);
  int32_t* sid2 = sid + 64;
  if (keep) sid[ik - 1] = id;  // kept ids, compacted
  if (l >= kept_c) sid[l] = 0x7fffffff;
  __builtin_amdgcn_wave_barrier();
  int pos = 0;
  for (int j0 = 0; j0 < kept_c; j0 += 16) {
    int32_t ij[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) ij[q] = sid[j0 + q];
#pragma unroll
    for (int q = 0; q < 16; ++q) pos += ij[q] < id ? 1 : 0;
  }
  __builtin_amdgcn_wave_barrier();
  if (keep) {
    F.dw[pos] = w;
    sid2[pos] = id;
  }
  __builtin_amdgcn_wave_barrier();
  const uint64_t wo = l < kept_c ? F.dw[l] : 0ull;
  const int32_t io = l < kept_c ? sid2[l] : -1;
  const uint64_t cum = wave_incl_scan(wo);
  const uint64_t W = read_lane(cum, 63);  // the kept weights, in any order
  const uint64_t target = W ? scaled_target(uniform_u32(u_draw), W) : 0ull;
  const uint64_t hm = __ballot(wo != 0ull && cum > target && cum - wo <= target);
  const int32_t token = hm ? read_lane(io, __builtin_ctzll(hm)) : -1;
  const uint64_t hp = __ballot(keep && probe >= 0 && id == probe);
  const uint64_t probe_w = hp ? read_lane(w, __builtin_ctzll(hp)) : 0ull;
  double cent = 0.0;  // statistics only
  float cmin = kPosInf;
  if (P.stats) {
    cent = wave_sum(keep ? (double)w * (1.0 / 1099511627776.0) * (double)weight_arg(y, y_max, c.scale)
                         : 0.0);
    cmin = wave_min(keep ? y : kPosInf);
  }
  // kept candidates persist, in key order, for the MTP residual pass
  Candidate* rc = ws.cands + (size_t)row * kCandCap;
  if (keep) {
    rc[ik - 1].y = y;
    rc[ik - 1].id = id;
  }
  if (in && P.keep) P.keep[(size_t)row * (size_t)V + id] = keep ? 1 : 0;
  if (l == 0) {
    uint32_t flags = info.flags;
    if (token < 0 || W == 0ull) flags |= LSAMP_ROW_EMPTY;
    P.tokens[row] = token;
    if (P.row_flags) P.row_flags[row] = flags;
    if (P.stats) {
      lsamp_row_stats st;
      st.max_value = y_max;
      st.log_normalizer = info.z > 0.0 ? __builtin_logf((float)info.z) : 0.0f;
      st.kept = kept_c;
      st.token = token;
      st.kept_weight = W;
      st.probe_weight = probe_w;
      st.cut_value = cmin;
      const double zk = (double)W * (1.0 / 1099511627776.0);
      st.kept_mass = (float)zk;
      st.kept_entropy = zk > 0.0 ? __builtin_logf((float)zk) - (float)(cent / zk) : 0.0f;
      st.probe_prob = W ? (float)((double)probe_w / (double)W) : 0.0f;
      P.stats[row] = st;
    }
    RowInfo out = info;
    out.kept_cands = kept_c;
    out.done = 1;
    ws.rows[row] = out;
  }
  if (lp) raw_chosen<DT>(P, *lp, row, token, rowp);
}

// Short-list finalize (the last work-group of a short-list row to publish).
// Every slice published the tokens at or above its own k-th largest filter-
// space value, sorted by cand_key descending; every token of the row's top-k
// (and every token tied with the k-th) is among them.  The lists are merged
// by rank into F.keys, cut after the row's top-k plus ties, and drawn from.
// The row's total mass comes from the slices' sums.  Returns false, having
// changed nothing, when a slice asks for the histogram path instead.
template <int DT>
__device__ __forceinline__ bool short_gather(const Workspace& ws, const SamplePlan& P, int row,
                                             const RowCtx& c, const lsamp_row_params& prm,
                                             TaskLds& L) {
  const int tid = fresh_tid();
  const int l = tid & 63;
  const bool wave0 = tid < 64;
  const int G = P.slices;
  const SliceSummary* summ = ws.summaries + (size_t)row * kMaxSlices;
  const uint64_t* pub = reinterpret_cast<const uint64_t*>(ws.cands + (size_t)row * kCandCap);
  // one round trip: thread t fetches key t % 64 of slice t / 64 (lists are
  // short), wave 0 also the slices' headers, the row's uniform and probe
  const int ks = tid >> 6, kj = tid & 63;
  const uint64_t kspec = ks < G ? ld_coherent(pub + (size_t)ks * kShortPub + kj) : 0ull;
  if (wave0) {
    float hx = kNegInf;
    int32_t hn = 0, hp = 0;
    uint32_t hf = 0u;
    double hz = 0.0;
    float hl = kPosInf;
    if (l < G) {
      hx = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&summ[l].x_max)));
      hn = ld_coherent(&summ[l].n_finite);
      hp = ld_coherent(&summ[l].npub);
      hf = ld_coherent(&summ[l].flags);
      hz = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&summ[l].zs)));
      hl = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&summ[l].ylo)));
    }
    float u = 0.0f;
    int32_t pr = -1;
    if (l == 0) {
      if (P.uniforms)
        u = P.uniforms[uniform_index(P, row)];
      else if (P.philox_keys)
        u = philox_uniform(P.philox_keys[row], 0u);
      const int pi = probe_index(P, row);
      pr = (P.probe_tokens && pi >= 0) ? P.probe_tokens[pi] : -1;
    }
    const bool fallback = __ballot(l < G && (hf & kSliceNoShort) != 0u) != 0ull;
    const bool live = l < G && hn > 0;
    const bool any = __ballot(live) != 0ull;
    const float row_max = wave_max(live ? hx : kNegInf);
    const bool nonfinite = __ballot(l < G && (hf & LSAMP_ROW_NONFINITE) != 0u) != 0ull;
    const int32_t hpv = live ? hp : 0;
    const int32_t ip = wave_incl_scan(hpv);
    const int32_t npmax = wave_max(hpv);
    if (l < G) L.soff[l] = ip - hpv;
    if (l == G - 1) L.soff[G] = ip;
    const float y_max = any ? to_filter(c, row_max) : 0.0f;
    // buckets of the finalize's counting sort: equal widths in value from
    // the row's largest down to the lowest slice bound
    const float y_low = wave_min(live && hpv > 0 ? hl : kPosInf);
    const float span = y_max - y_low;
    const float bscale = span > 0.0f && span < kPosInf ? (float)kRankBuckets / span : 0.0f;
    // slice s summed exp((x - x_s) / T_f); rescaled to e^y_max
    double z = 0.0;
    if (any && c.kind != LSAMP_KIND_ARGMAX)
      z = wave_sum(live ? hz * (double)__builtin_expf((hx - row_max) / (float)c.tf) : 0.0);
    RowInfo info;
    info.x_max = row_max;
    info.q_top = y_max;
    info.top_bin = any ? bin_of(row_max, c.c32) : 0;
    info.cut = kCutList;
    info.mode = any ? kModeNormal : kModeEmpty;
    info.flags = nonfinite ? LSAMP_ROW_NONFINITE : 0u;
    info.count_above = 0;
    info.n_finite = any ? 1 : 0;
    info.mass_above = 0.0;
    info.z = z;
    info.p_limit = top_p_limit(P, c, prm, z);
    {
      // (made here: the constant pair (0, 1) hoisted out of the fused
      // kernel's task loop was held across it and spilled)
      int zero = 0, one = 1;
      asm volatile("" : "+v"(zero), "+v"(one));
      info.kept_cands = zero;
      info.done = one;
    }
    if (l == 0) {
      L.info = info;
      L.misc[5] = fallback ? 1 : 0;
      L.misc[7] = npmax;
      L.misc64[0] = __float_as_uint(u);
      L.misc[4] = pr;
      L.misc[0] = (int32_t)__float_as_uint(y_max);
      L.misc[1] = (int32_t)__float_as_uint(bscale);
    }
  }
  for (int i = tid; i < kRankBuckets; i += kThreads) L.sh.tcnt[i] = 0u;
  __syncthreads();
  if (L.misc[5]) return false;
  if (ks < G && kj < L.soff[ks + 1] - L.soff[ks]) L.ssrc[L.soff[ks] + kj] = kspec;
  return true;
}

// The rest of a short-list row's finalize, once short_gather has accepted it:
// the keys past the 64th of a slice, the merge by rank, the cut after the
// row's top-k plus ties, and the tail.
template <int DT>
__device__ __forceinline__ void short_finish(const Workspace& ws, const SamplePlan& P, int row,
                                             const RowCtx& c, const lsamp_row_params& prm,
                                             TaskLds& L, const char* rowp, const uint32_t* mrow,
                                             int K, const FusedLp* lp) {
  const int tid = fresh_tid();
  const bool wave0 = tid < 64;
  const int G = P.slices;
  const int64_t V = P.vocab;
  FinalLds& F = L.u.f;
  const uint64_t* pub = reinterpret_cast<const uint64_t*>(ws.cands + (size_t)row * kCandCap);
  const int n_tot = L.soff[G];
  const int npmax = L.misc[7];
  if (npmax > 64) {
    // keys past the 64th of a slice: a second round trip
    for (int s2 = 0; s2 < G; ++s2) {
      const int np = L.soff[s2 + 1] - L.soff[s2];
      for (int j = 64 + tid; j < np; j += kThreads)
        L.ssrc[L.soff[s2] + j] = ld_coherent(pub + (size_t)s2 * kShortPub + j);
    }
  }
  if (P.keep) {
    // the tail writes the bytes of the listed tokens; every other token of
    // the row is dropped
    uint8_t* kr = P.keep + (size_t)row * (size_t)V;
    for (int64_t i = tid; i < V; i += kThreads) kr[i] = 0;
    __syncthreads();  // (these stores land before the tail's)
  } else {
    lds_barrier();
  }
  // rank of each key in the union (keys are distinct: token ids are): the
  // keys above it.  The comparisons of a key are split over `parts` threads
  // (the whole work-group works), each reading its share of the keys 16 at a
  // time, and the partial counts meet in LDS.
  int32_t* racc = reinterpret_cast<int32_t*>(F.dw);  // [n_tot] partial ranks (n_tot <= kCandCap)
  int32_t* rk = racc;
  const int parts = n_tot > 0 && n_tot <= kThreads / 2 ? kThreads / n_tot : 1;
  if (n_tot <= kThreads) {
    // counting sort by the key's high word (bucket 0: the largest keys), then
    // the rank within the bucket: the bucket's start plus its keys above
    uint32_t* bcnt = L.sh.tcnt;                  // [kRankBuckets], zeroed
    uint32_t* bstart = L.sh.tcnt + kRankBuckets;  // [kRankBuckets]
    uint64_t* tmp = reinterpret_cast<uint64_t*>(F.dw);  // keys grouped by bucket
    const float y_top = __uint_as_float((uint32_t)L.misc[0]);
    const float bscale = __uint_as_float((uint32_t)L.misc[1]);
    if (tid == 0) L.misc[6] = n_tot;
    const bool have = tid < n_tot;
    uint64_t key = 0ull;
    int b = 0, slot = 0;
    if (have) {
      key = L.ssrc[tid];
      // (monotone in the key: a larger value never lands in a later bucket)
      const float d = (y_top - key_y(key)) * bscale;
      b = d < (float)(kRankBuckets - 1) ? (int)d : kRankBuckets - 1;
      b = b > 0 ? b : 0;
      slot = (int)atomicAdd(&bcnt[b], 1u);
    }
    lds_barrier();
    if (tid < 64) {
      constexpr int kPer = kRankBuckets / 64;
      uint32_t cb[kPer];
      uint32_t cs = 0u;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        cb[i] = bcnt[kPer * tid + i];
        cs += cb[i];
      }
      uint32_t acc = wave_incl_scan(cs) - cs;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        bstart[kPer * tid + i] = acc;
        acc += cb[i];
      }
    }
    lds_barrier();
    int s0 = 0, cnt = 0;
    if (have) {
      s0 = (int)bstart[b];
      cnt = (int)bcnt[b];
      tmp[s0 + slot] = key;
    }
    lds_barrier();
    if (have) {
      int r = s0;
      int j = s0;
      const int je = s0 + cnt;
      for (; j + 4 <= je; j += 4) {
        uint64_t k4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) k4[q] = tmp[j + q];
#pragma unroll
        for (int q = 0; q < 4; ++q) r = add_gt_u64(r, k4[q], key);
      }
      for (; j < je; ++j) r = add_gt_u64(r, tmp[j], key);
      F.keys[r] = key;
    }
  } else if (parts > 1) {
    for (int i = tid; i < n_tot; i += kThreads) racc[i] = 0;
    if (tid == 0) L.misc[6] = n_tot;
    lds_barrier();
    const int i = tid % n_tot, part = tid / n_tot;
    if (part < parts) {
      const uint64_t key = L.ssrc[i];
      const int j0 = (n_tot * part) / parts, j1 = (n_tot * (part + 1)) / parts;
      int r = 0;
      int j = j0;
      for (; j + 16 <= j1; j += 16) {
        uint64_t kk[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) kk[q] = L.ssrc[j + q];
#pragma unroll
        for (int q = 0; q < 16; ++q) r += kk[q] > key ? 1 : 0;
      }
      for (; j < j1; ++j) r += L.ssrc[j] > key ? 1 : 0;
      atomicAdd(&racc[i], r);
    }
    lds_barrier();
    for (int i2 = tid; i2 < n_tot; i2 += kThreads) F.keys[rk[i2]] = L.ssrc[i2];
  } else {
    if (tid == 0) L.misc[6] = n_tot;
    for (int i = tid; i < n_tot; i += kThreads) {
      const uint64_t key = L.ssrc[i];
      int r = 0;
      int j = 0;
      for (; j + 16 <= n_tot; j += 16) {
        uint64_t kk[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) kk[q] = L.ssrc[j + q];
#pragma unroll
        for (int q = 0; q < 16; ++q) r += kk[q] > key ? 1 : 0;
      }
      for (; j < n_tot; ++j) r += L.ssrc[j] > key ? 1 : 0;
      F.keys[r] = key;
    }
  }
  lds_barrier();
  // the row's top-k and every token tied with the k-th: the first position
  // past K - 1 whose value is below the k-th's
  if (n_tot > K) {
    const uint32_t kv = (uint32_t)(F.keys[K - 1] >> 32);
    for (int i = K + tid; i < n_tot; i += kThreads)
      if ((uint32_t)(F.keys[i] >> 32) < kv && (uint32_t)(F.keys[i - 1] >> 32) >= kv) L.misc[6] = i;
  }
  lds_barrier();
  if (!wave0) {
    // (wave 1: the raw log-probability lists, beside wave 0's draw, in the
    // staging area no finalize uses)
    if (lp && tid < 128) raw_lists<DT>(P, *lp, row, reinterpret_cast<uint64_t*>(L.sh.squad));
    return;
  }
  int nc = L.misc[6];
  const RowInfo info = L.info;
  if (info.mode != kModeNormal) nc = 0;
  const float u_draw = __uint_as_float((uint32_t)L.misc64[0]);
  const int32_t probe = L.misc[4];
  if (nc <= 64) {
    short_tail<DT>(ws, P, row, c, prm, info, L, nc, u_draw, probe, rowp, lp);
    return;
  }
  TailIn t;
  t.nc = nc;
  t.overflow = false;
  t.ent_all = 0.0;
  t.min_all = kPosInf;
  t.kept_all = 0;
  t.u_draw = u_draw;
  t.probe = probe;
  t.probe_x_set = false;
  t.probe_x = 0.0f;
  t.n_list = 0;
  t.reset = false;
  t.done = 1;
  uint64_t rch[kChunksPerLane];
#pragma unroll
  for (int i = 0; i < kChunksPerLane; ++i) rch[i] = 0ull;
  finalize_tail<DT>(ws, P, row, c, prm, info, L, rowp, mrow, t, rch, lp);
}

// ==================================================== raw log-probabilities
// In-pass raw log-probabilities of the fused arrangement (lsamp_step asking
// for them): the reference takes raw - logSumExp(raw) before any transform
// and gathers the chosen token and the k best by the raw order, value
// descending, lower id on ties, +0 and -0 tied (LogitsPipelineV2.process
// :307-314, CBv2Logprobs.gather :534-549).  Pass 1 of each slice's own pass
// takes the raw logits' statistics before any exclusion (raw_add); the slice
// then lists its k best raw keys (raw_slice) and publishes a record before
// its first exchange; the row's finalizer merges the records: wave 1 the
// lists (raw_lists) while wave 0 draws, wave 0 the chosen token's value
// once it is drawn (raw_chosen).  A row whose log-sum-exp is not finite (a NaN or
// +inf logit, or every logit -inf) fails closed: ids -1 and NaN values
// (CBv2NonFiniteLogits.swift:30-38).
constexpr uint32_t kRawNan = 1u, kRawPosInf = 2u;
constexpr int kRawList = kThreads;       // candidates ranked by counting
constexpr int kRawOut = kRawList;        // the sorted best k follow them
static_assert(kRawOut + kTopkMaxLp <= kCandCap, "the raw lists fit the finalize keys");

static_assert(sizeof(ShortLds::squad) >= kMaxSlices * kTopkMaxLp * sizeof(uint64_t),
              "the raw lists fit the staging area");

struct RawAcc {
  float m;         // largest non-NaN raw logit
  float z;         // sum of exp2(x * log2e + nb) over the thread's raw logits
  float nb;        // its anchor: an integer, re-set by an exact power of two
  uint32_t flags;  // kRawNan, kRawPosInf
};

// One quad of raw logits into the thread's statistics (lanes past the slice
// end excluded by `tail`; `probe` flags a NaN or infinity in the quad).
template <int DT>
__device__ __forceinline__ void raw_add(RawAcc& a, uint4 v, uint32_t tail, uint32_t probe) {
  constexpr int N = Vec<DT>::N;
  constexpr float kLog2e = 1.4426950408889634f;
  exclude_elems<DT>(v, tail);
  float q = vec_max_nn<DT>(v);
  if (nonfinite_seen<DT>(probe)) {
    // (rare) NaN and +inf flags; the maximum of the others
    q = kNegInf;
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float x = vec_elem<DT>(v, e);
      if (x != x) a.flags |= kRawNan;
      if (x == kPosInf) a.flags |= kRawPosInf;
      q = __builtin_fmaxf(q, x);
    }
  }
  a.m = __builtin_fmaxf(a.m, q);
  if (__builtin_fmaf(q, kLog2e, a.nb) > 64.0f) {
    const float nn = -__builtin_ceilf(__builtin_amdgcn_fmed3f(q * kLog2e, -0x1p20f, 0x1p20f));
    a.z = __builtin_ldexpf(a.z, (int)__builtin_fmaxf(nn - a.nb, -512.0f));
    a.nb = nn;
  }
  float t[N];
#pragma unroll
  for (int e = 0; e < N; ++e)
    t[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(vec_elem<DT>(v, e), kLog2e, a.nb));
#pragma unroll
  for (int w = 1; w < N; w *= 2)
#pragma unroll
    for (int e = 0; e < N; e += 2 * w) t[e] += t[e + w];
  a.z += t[0];
}

// The exact K-th largest raw key of the slice (a radix select over the
// slice read again, eight bits a round), then every key at or above it
// listed in `dst`: min(K, slice length) keys.  For slices whose threshold
// leaves too many candidates (many equal logits, or -inf ones).  Whole
// work-group; its counts use the thread-maximum histogram's words.
template <int DT>
__device__ __forceinline__ int raw_select_exact(const char* rowp, int32_t base32, int32_t end32,
                                                int K, uint64_t* dst, TaskLds& L) {
  const int tid = fresh_tid();
  const int len = end32 - base32;
  if (K > len) K = len;
  uint32_t* const cnt = L.sh.tcnt;
  uint64_t prefix = 0ull;
  int need = K;
#pragma unroll 1
  for (int shift = 56; shift >= 0; shift -= 8) {
    const uint64_t hmask = shift == 56 ? 0ull : ~0ull << (shift + 8);
    for (int i = tid; i < 256; i += kThreads) cnt[i] = 0u;
    __syncthreads();
#pragma unroll 1
    for (int32_t i = base32 + tid; i < end32; i += kThreads) {
      const uint64_t key = cand_key(load_scalar<DT>(rowp, i), i);
      if ((key & hmask) == prefix) atomicAdd(&cnt[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // digits from the top: lane l holds digits 255 - 4l .. 252 - 4l
      uint32_t cb[4];
      uint32_t cs = 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        cb[i] = cnt[255 - (4 * tid + i)];
        cs += cb[i];
      }
      const uint32_t ic = wave_incl_scan(cs);
      const uint64_t hit = __ballot(ic >= (uint32_t)need);
      const int f = hit ? __builtin_ctzll(hit) : 63;
      uint32_t acc = read_lane(ic - cs, f);
      int digit = 0, above = 0;
      if (tid == f) {
        for (int i = 0; i < 4; ++i) {
          if (acc + cb[i] >= (uint32_t)need) {
            digit = 255 - (4 * tid + i);
            above = (int)acc;
            break;
          }
          acc += cb[i];
        }
      }
      digit = read_lane(digit, f);
      above = read_lane(above, f);
      if (tid == 0) {
        L.misc[0] = digit;
        L.misc[1] = above;
      }
    }
    __syncthreads();
    prefix |= (uint64_t)(uint32_t)L.misc[0] << shift;
    need -= L.misc[1];
  }
  if (tid == 0) L.nraw = 0;
  __syncthreads();
#pragma unroll 1
  for (int32_t i0 = base32; i0 < end32; i0 += kThreads) {
    const int32_t i = i0 + tid;
    const float x = i < end32 ? load_scalar<DT>(rowp, i) : 0.0f;
    const bool hit = i < end32 && cand_key(x, i) >= prefix;
    const int slot = wave_append(hit, &L.nraw);
    if (hit && slot < K) dst[slot] = cand_key(x, i);
  }
  __syncthreads();
  return K;
}

// The slice's raw record (whole work-group, after pass 1): its maximum, its
// sum relative to the maximum and its flags; with k > 0 and finite logits,
// its k best raw keys.  Threshold: each wave's c-th largest thread maximum
// (c = ceil(k / 8)), the smallest over the waves, so at least k tokens reach
// it; the threads whose maximum reaches it read their logits again (from
// L2) and list the keys at or above it, which are ranked by counting.  A
// slice whose threshold leaves more than kRawList candidates takes the
// exact select.  Leaves the short-list and histogram words zeroed.
template <int DT>
__device__ __forceinline__ void raw_slice(const SamplePlan& P, const FusedLp& lp, int row,
                                          int slice, const char* rowp, int32_t base32,
                                          int32_t end32, int nq, const RawAcc& a, TaskLds& L) {
  constexpr int N = Vec<DT>::N;
  constexpr float kLog2e = 1.4426950408889634f;
  const int tid = fresh_tid(), l = tid & 63, wv = tid >> 6;
  const int K = lp.k;
  // 1. the slice's flags, maximum, and sum relative to the maximum
  const uint32_t fw = (__ballot((a.flags & kRawNan) != 0u) ? kRawNan : 0u) |
                      (__ballot((a.flags & kRawPosInf) != 0u) ? kRawPosInf : 0u);
  const float mw = wave_max(a.m);
  __syncthreads();
  if (l == 0) {
    L.redf[wv] = mw;
    L.redi[wv] = (int32_t)fw;
  }
  __syncthreads();
  float M = L.redf[0];
  uint32_t F = (uint32_t)L.redi[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) {
    M = __builtin_fmaxf(M, L.redf[i]);
    F |= (uint32_t)L.redi[i];
  }
  double zt = 0.0;
  if (a.z > 0.0f && M > kNegInf && M < kPosInf) {
    // the thread's terms rescaled from 2^-nb to e^M (M * log2e split into a
    // rounded part and its exact residual)
    const float bh = M * kLog2e;
    const float bl = __builtin_fmaf(M, kLog2e, -bh);
    zt = (double)(a.z * __builtin_amdgcn_exp2f((-a.nb - bh) - bl));
  }
  zt = wave_sum(zt);
  __syncthreads();
  if (l == 0) L.redd[wv] = zt;
  __syncthreads();
  double zsum = 0.0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) zsum += L.redd[i];

  // 2. the k best raw keys
  int listed = 0;
  uint64_t* const cand = L.u.f.keys;
  if (K > 0 && F == 0u) {
    const int c = (K + kWaves - 1) / kWaves;
    bool taken = false;
    float wc = kNegInf;
    for (int i = 0; i < c; ++i) {
      const float mx = wave_max(taken ? kNegInf : a.m);
      const uint64_t hit = __ballot(!taken && a.m == mx);
      if (hit != 0ull && l == __builtin_ctzll(hit)) taken = true;
      wc = mx;
    }
    if (l == 0) L.redf2[wv] = wc;
    if (tid == 0) L.nraw = 0;
    __syncthreads();
    float tau = L.redf2[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) tau = __builtin_fminf(tau, L.redf2[i]);
    int n = kRawList + 1;
    if (tau > kNegInf) {
      // 3. candidates: the logits of the threads whose maximum reaches tau,
      // read again by the whole work-group at once: the reading threads'
      // (thread, quad) pairs are dealt to every thread, kRePer 16-byte loads
      // a thread in flight together (through one buffer descriptor over the
      // slice, as pass 1 loads them), so up to kThreads * kRePer pairs take
      // one round trip.  The last partial quad and unaligned rows are read
      // element by element.
      constexpr int ES = Vec<DT>::ESIZE;
      constexpr int kRePer = N == 4 ? 4 : 2;  // (fp32 slices: more quads a thread)
      const bool aligned = P.aligned != 0;
      const bool reads = a.m >= tau;
      const uint64_t mm = __ballot(reads);
      if (l == 0) L.redu[wv] = mm;
      __syncthreads();
      int before = 0, M = 0;  // reading threads in lower waves, in all
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const int cw = (int)__popcll(L.redu[w]);
        before += w < wv ? cw : 0;
        M += cw;
      }
      // the reading threads in order (in the sorted keys' area, idle until
      // the rank)
      uint32_t* const who = reinterpret_cast<uint32_t*>(cand + kRawOut);
      static_assert(kRawOut + kThreads / 2 <= kCandCap, "a reader id per thread fits");
      if (reads) who[before + (int)__popcll(mm & ((1ull << l) - 1ull))] = (uint32_t)tid;
      __syncthreads();
      const int pairs = M * nq;  // (uniform)
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<char*>(rowp) + (size_t)base32 * ES, 0, aligned ? (end32 - base32) * ES : 0,
          kBufferWord3);
#pragma unroll 1
      for (int p0 = 0; p0 < pairs; p0 += kThreads * kRePer) {
        // pair pr: quad pr % nq of the (pr / nq)-th reading thread, at
        // quad place qd of the slice (recomputed after the loads, so only
        // the loaded words stay live across them)
        auto place = [&](int pr) -> int {
          const int q = pr / nq;
          return (int)who[q] + (pr - q * nq) * kThreads;
        };
        uint4 w[kRePer];
#pragma unroll
        for (int j = 0; j < kRePer; ++j) {
          const int pr = p0 + j * kThreads + tid;
          const auto r = __builtin_amdgcn_raw_buffer_load_b128(
              rs, pr < pairs ? place(pr) * 16 : 0x40000000, 0, 0);
          w[j] = make_uint4(r[0], r[1], r[2], r[3]);
        }
#pragma unroll
        for (int j = 0; j < kRePer; ++j) {
          const int pr = p0 + j * kThreads + tid;
          const int32_t i0 = pr < pairs ? base32 + place(pr) * N : end32;  // (past the end: nothing listed)
          if (i0 < end32 && (!aligned || i0 + N > end32)) {
            uint32_t b[N];
#pragma unroll
            for (int e = 0; e < N; ++e) b[e] = i0 + e < end32 ? load_raw_bits<DT>(rowp, i0 + e) : 0u;
            if constexpr (N == 4) {
              w[j] = make_uint4(b[0], b[1], b[2], b[3]);
            } else {
              w[j] = make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16),
                                b[6] | (b[7] << 16));
            }
          }
#pragma unroll
          for (int e = 0; e < N; ++e) {
            const float x = vec_elem<DT>(w[j], e);
            const bool hit = i0 + e < end32 && x >= tau;
            const int slot = wave_append(hit, &L.nraw);
            if (hit && slot < kRawList) cand[slot] = cand_key(x, i0 + e);
          }
        }
      }
      __syncthreads();
      n = L.nraw;
    }
    if (n > kRawList) {
      n = raw_select_exact<DT>(rowp, base32, end32, K, cand, L);
      // (its counts used the words the rank counts in)
      for (int i = tid; i < kRawList; i += kThreads) L.sh.tcnt[i] = 0u;
      __syncthreads();
    }
    // 4. rank by counting, spread over the work-group: key i's count of
    // the keys above it is summed over C chunks of the list (C = kThreads
    // over n rounded up to a power of two), one (key, chunk) pair a thread;
    // a wave's pairs share their chunk, so its reads are broadcasts.  The
    // counts gather in the thread-maximum histogram's words (zero here).
    uint32_t* const above = L.sh.tcnt;
    static_assert(kTauBins >= kRawList, "a count per candidate");
    if (n > 0) {
      const int np = n <= 64 ? 64 : n <= 128 ? 128 : n <= 256 ? 256 : 512;
      const int C = kThreads / np;
      const int span = (n + C - 1) / C;
      const int i = tid & (np - 1), ch = tid / np;
      if (i < n) {
        const uint64_t key = cand[i];
        const int j0 = ch * span, j1 = j0 + span < n ? j0 + span : n;
        int r = 0, jj = j0;
        for (; jj + 4 <= j1; jj += 4) {  // (four reads in flight)
          const uint64_t c0 = cand[jj], c1 = cand[jj + 1], c2 = cand[jj + 2], c3 = cand[jj + 3];
          r = add_gt_u64(add_gt_u64(add_gt_u64(add_gt_u64(r, c0, key), c1, key), c2, key), c3, key);
        }
        for (; jj < j1; ++jj) r = add_gt_u64(r, cand[jj], key);
        if (r != 0) atomicAdd(&above[i], (uint32_t)r);
      }
      __syncthreads();
      if (tid < n) {
        const uint32_t r = above[tid];
        if (r < (uint32_t)K) cand[kRawOut + r] = cand[tid];
      }
    }
    __syncthreads();
    listed = n < K ? n : K;
  }
  // 5. the record
  RawRecord* rec = lp.rec + (size_t)row * kMaxSlices + slice;
  if (tid < listed) st_coherent(&rec->keys[tid], cand[kRawOut + tid]);
  if (tid == 0) {
    st_coherent_f32(&rec->max, M);
    st_coherent(&rec->flags, F);
    st_coherent(&rec->n, listed);
    st_coherent_f64(&rec->z, zsum);
  }
  // the words the slice's short list and histogram count on
  if (K > 0) {
    for (int i = tid; i < kHist + 64; i += kThreads) L.u.hist[i] = 0ull;
    for (int i = tid; i < kTauBins; i += kThreads) L.sh.tcnt[i] = 0u;
  }
  __syncthreads();
}

// The row's log-sum-exp of the raw logits from the slices' records (one
// wave; every wave that calls it computes the same value): lane l < G
// returns record l's key count.  A row with a NaN or +inf logit, or with
// every logit -inf, is closed.
struct RawHead {
  float lse;
  bool closed;
  int32_t n;  // (lane l < G) record l's listed keys
};
__device__ __forceinline__ RawHead raw_head(const SamplePlan& P, const FusedLp& lp, int row) {
  const int l = fresh_tid() & 63;
  const int G = P.slices;
  const RawRecord* rec = lp.rec + (size_t)row * kMaxSlices;
  float ms = kNegInf;
  double zs = 0.0;
  uint32_t fs = 0u;
  int32_t ns = 0;
  if (l < G) {
    ms = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&rec[l].max)));
    fs = ld_coherent(&rec[l].flags);
    ns = ld_coherent(&rec[l].n);
    zs = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&rec[l].z)));
  }
  const float M = wave_max(ms);
  RawHead h;
  h.closed = __ballot(fs != 0u) != 0ull || !(M > kNegInf);
  const double z = wave_sum((l < G && ms > kNegInf) ? zs * fexp((double)ms - (double)M) : 0.0);
  h.lse = h.closed ? 0.0f : M + __builtin_logf((float)z);
  h.n = ns;
  return h;
}

// The chosen token's raw log-probability (wave 0 of the finalizing work-
// group, once the token is drawn; NaN for a closed row or no token).
template <int DT>
__device__ __forceinline__ void raw_chosen(const SamplePlan& P, const FusedLp& lp, int row,
                                           int32_t tok, const char* rowp) {
  const int l = fresh_tid() & 63;
  const bool tok_in = tok >= 0 && tok < P.vocab;
  const float xc = (l == 0 && tok_in) ? load_scalar<DT>(rowp, tok) : 0.0f;
  const RawHead h = raw_head(P, lp, row);
  if (l == 0) lp.chosen[row] = (!h.closed && tok_in) ? xc - h.lse : __builtin_nanf("");
}

// The row's k best raw log-probabilities (one wave of the finalizing work-
// group, beside wave 0's draw: they do not depend on the token; `lists`
// holds kMaxSlices * kTopkMaxLp words of LDS the draw does not use).  Every
// load is issued at once: the records' heads and each key slot a record can
// list (slots past its count are dropped once the counts are in).
template <int DT>
__device__ __forceinline__ void raw_lists(const SamplePlan& P, const FusedLp& lp, int row,
                                          uint64_t* lists) {
  constexpr int kPer = kMaxSlices * kTopkMaxLp / 64;  // key slots a lane loads
  static_assert(kPer * 64 == kMaxSlices * kTopkMaxLp, "whole lanes");
  const int l = fresh_tid() & 63;
  const int G = P.slices, K = lp.k;
  if (K <= 0) return;
  const RawRecord* rec = lp.rec + (size_t)row * kMaxSlices;
  uint64_t kv[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = l + 64 * j, s = i / kTopkMaxLp, p = i % kTopkMaxLp;
    kv[j] = (s < G && p < K) ? ld_coherent(&rec[s].keys[p]) : 0ull;
  }
  const RawHead h = raw_head(P, lp, row);
  // the keys into LDS, the slots past their record's count as zeros
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = l + 64 * j, s = i / kTopkMaxLp, p = i % kTopkMaxLp;
    const int n_s = __shfl(h.n, s, 64);
    lists[i] = (s < G && p < n_s) ? kv[j] : 0ull;
  }
  // ranks 0 .. listed - 1 each take one key (keys are distinct); the slots
  // past them, and a closed row's, read (-1, NaN)
  const int listed = h.closed ? 0 : wave_sum(l < G ? h.n : 0);
  if (l < K && l >= listed) {
    lp.ids[(size_t)row * K + l] = -1;
    lp.values[(size_t)row * K + l] = __builtin_nanf("");
  }
  if (h.closed) return;
  __builtin_amdgcn_wave_barrier();
  // a key's rank: its place in its own list plus, in every other list,
  // the keys above it (lists are sorted descending and padded with zeros,
  // below every key): fixed-step searches, two lists at a time
  static_assert(kTopkMaxLp == 32, "five halving steps and a last check");
#pragma unroll 1
  for (int j = 0; j < kPer; ++j) {
    const int i = l + 64 * j, s = i / kTopkMaxLp;
    const uint64_t key = lists[i];
    if (s >= G || key == 0ull) continue;
    int r = i % kTopkMaxLp;
    constexpr int kAtOnce = 2;  // lists searched together
#pragma unroll 1
    for (int s0 = 0; s0 < G; s0 += kAtOnce) {
      int lo[kAtOnce];
#pragma unroll
      for (int u = 0; u < kAtOnce; ++u) lo[u] = 0;
#pragma unroll
      for (int step = kTopkMaxLp / 2; step >= 1; step >>= 1)
#pragma unroll
        for (int u = 0; u < kAtOnce; ++u)
          if (s0 + u < G && lists[(s0 + u) * kTopkMaxLp + lo[u] + step - 1] > key) lo[u] += step;
#pragma unroll
      for (int u = 0; u < kAtOnce; ++u)
        if (s0 + u < G && s0 + u != s)
          r += lo[u] + (lists[(s0 + u) * kTopkMaxLp + lo[u]] > key ? 1 : 0);
    }
    if (r < K) {
      lp.ids[(size_t)row * K + r] = key_id(key);
      lp.values[(size_t)row * K + r] = key_y(key) - h.lse;
    }
  }
}

// ================================================================ one task
// Does any slice of a short-list row need the histogram path (+inf logits,
// an entry-table or short-list overflow)?  Called by the whole work-group.
__device__ __forceinline__ bool short_fallback(const Workspace& ws, int row, int G, TaskLds& L) {
  const int tid = fresh_tid();
  if (tid < 64) {
    const uint32_t f = tid < G ? ld_coherent(&ws.summaries[(size_t)row * kMaxSlices + tid].flags) : 0u;
    const bool fb = __ballot((f & kSliceNoShort) != 0u) != 0ull;
    if (tid == 0) L.misc[5] = fb ? 1 : 0;
  }
  __syncthreads();
  return L.misc[5] != 0;
}

// What a fused work-group does next on its row (slice_job's result): leave
// it, or a job for another slice: its fallback histogram (kBehalfStats) or
// its select (kSelectOnly), from a re-read of that slice.
constexpr int kJobLeave = -1;
constexpr int kBehalfStats = 3;
__device__ __forceinline__ int next_job(int kind, int slice) { return (kind << 8) | slice; }

// One pass of a work-group over one slice of a row.  Split mode: MODE is the
// kernel's phase (and JM == MODE).  Fused arrangement (MODE == kFused): JM is
// the job: the work-group's own slice (kFused), or work it claimed for slice
// `slice` of a slice that left (kBehalfStats, kSelectOnly); `own` is its own
// slice.  (Each job is its own instantiation, so the own pass compiles as
// if the others did not exist.)
template <int DT, int MODE, int JM, bool LP>
__device__ __forceinline__ int slice_job(const Workspace& ws, const SamplePlan& P, int row, int slice,
                                         TaskLds& L, int own, const FusedLp& Lk) {
  constexpr int jm = JM;
  // (LP: raw log-probabilities in this pass; the finalizer writes them)
  const FusedLp* const lpp = LP ? &Lk : nullptr;
  // split mode: rows the stats kernel already drew (short lists) are done
  if (MODE == kSelectOnly && ws.rows[row].done) return kJobLeave;
  constexpr int N = Vec<DT>::N;
  constexpr int Q = Slab<DT>::Q;
  static_assert(Q <= 32, "staged quad numbers take 5 bits");
  static_assert(kSliceEntryCap <= 32 * kThreads, "entry candidates take one bit each");
  constexpr uint32_t FULL = (1u << N) - 1u;
  constexpr int ES = Vec<DT>::ESIZE;
  const int tid = fresh_tid();
  const int G = P.slices;
  const int64_t V = P.vocab;
  const int64_t base = (int64_t)slice * P.slice_len;
  const int64_t end = (base + P.slice_len < V) ? base + P.slice_len : V;
  const char* rowp = row_base(P, row);
  const bool aligned = P.aligned != 0;
  // Token positions within a row fit in 32 bits (vocab <= kMaxVocab).
  const int32_t base32 = (int32_t)base, end32 = (int32_t)end;
  const int nq = (P.slice_len + kThreads * N - 1) / (kThreads * N);  // quads per thread

  // ---------------------------------------------------- A: loads + entries
  // The row's parameters and the CSR bounds of its penalty entries come
  // through scalar loads; the first entries are requested ahead of the
  // slice's logits (vector loads complete in order), so the entry bitmap is
  // built while the slice streams in and the pass over the slice starts on
  // each quad as it lands.
  const lsamp_row_params prm = load_params(P, row);
  EntryPrefetch<> ep;
  entry_bounds(P, row, ep);
  const RowCtx c = make_ctx(P.semantics, prm);
  const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * (size_t)P.mask_words : nullptr;
  prefetch_entries(P, tid, ep);
  // the slice's grammar-mask words, staged in LDS (the short-list area,
  // idle until after pass 1) before the pass
  MaskStage ms;
  if (mrow) load_mask_stage(mrow, P.mask_words, base32, end32, tid, ms);
  uint32_t* const mw = reinterpret_cast<uint32_t*>(L.sh.squad);
  static_assert(sizeof(L.sh.squad) >= kSliceWords * sizeof(uint32_t), "staged mask words fit");
  // The slice's logits: 16-byte vectors all in flight at once, through one
  // buffer descriptor over the slice (the lane's byte offset is fixed and
  // the quad's is a scalar; lanes past the slice end read as zero, by the
  // range check, until the exclusion pass).
  Slab<DT> S;
  {
    // (an unaligned row gets an empty range, so every load reads zero and
    // the element-by-element path fills the slab in; the loads are issued
    // either way, which keeps later waits exact)
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(rowp) + (size_t)base32 * ES, 0, aligned ? (end32 - base32) * ES : 0,
        kBufferWord3);
    const int lane_off = tid * 16;
    // (every quad of the slab, without a branch: quads past the slice read
    // zero, and straight-line loads let each later wait name its own quad)
#pragma unroll
    for (int g = 0; g < Q; ++g) {
      const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs, lane_off, g * kThreads * 16, 0);
      quad_set(S.bank[g / kQuadsPerBank], g % kQuadsPerBank, make_uint4(w[0], w[1], w[2], w[3]));
    }
  }
  // (fused, own slice) the row's start ticket, issued after the slice's
  // loads so that their waits do not include it; its result is consumed at
  // the first exchange, before the arrival
  uint32_t tick = 0u;
  if (MODE == kFused && jm == kFused && tid == 0)
    tick = __hip_atomic_fetch_add(row_sync(ws, row) + kSyncArrive, kStartOne, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
  if (jm != kSelectOnly) {
    for (int i = tid; i < kHist; i += kThreads) L.u.hist[i] = 0ull;
    for (int i = tid; i < kTauBins; i += kThreads) L.sh.tcnt[i] = 0u;
  }
  if (tid == 0) {
    L.flags = 0u;
    L.ncand = 0;
  }
  SliceEntries se{L.pen, L.etok, L.ex, &L.ecount};
  EntryMarks<> em;
  float emax = kNegInf;  // this thread's patched entry values
  if (mrow) store_mask_stage(ms, P.mask_words, P.mask_bits, P.mask_tail, base32, end32, tid, mw);
  mark_slice_entries<DT>(P, c, prm, mrow, rowp, base, end, se, ep, tid, em, emax);
  if (!aligned || (end32 & (N - 1)) != 0) {
    // unaligned rows, or the row's last partial quad: element by element
    // (after the entry bitmap, whose wait these loads would otherwise delay)
    for_quads(S, nq, [&](int g, uint4& v) -> bool {
      const int32_t i0 = base32 + (tid + g * kThreads) * N;
      if (i0 >= end32 || (aligned && i0 + N <= end32)) return false;
      uint32_t b[N];
#pragma unroll
      for (int e = 0; e < N; ++e) b[e] = i0 + e < end32 ? load_raw_bits<DT>(rowp, i0 + e) : 0u;
      if constexpr (N == 4) {
        v = make_uint4(b[0], b[1], b[2], b[3]);
      } else {
        v = make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16),
                       b[6] | (b[7] << 16));
      }
      return true;
    });
  }

  // Masked tokens, tokens of the entry table (their patched values live in
  // L.ex) and lanes past the slice end become -inf in the register copy, and
  // so do NaNs.  From here on "excluded" is simply "not > -inf".  The same
  // pass takes the thread's maximum and, for short-list rows, the thread's
  // sum of exp((x - m) / T_f): each term is exp2(x * lgz + nbz) with nbz an
  // integer anchored at a quad maximum (re-anchored by an exact power of two
  // only if the running maximum climbs 64 binary orders above it), so the
  // largest terms are computed at full precision.
  // (a claimed fallback histogram skips the short list: K = 0; Krow is the
  // row's own, which sets the exchange's arrival count)
  const int Krow = jm != kSelectOnly ? short_k(c, prm, V) : 0;
  const int K = jm == kBehalfStats ? 0 : Krow;
  const bool zon = K > 0 && c.kind != LSAMP_KIND_ARGMAX;
  const float lgz = (float)(1.4426950408889634 / c.tf);  // log2(e) / T_f
  // penalty-bitmap word of quad g (the bitmap is zeroed over the largest
  // slice, so every quad's word is in bounds); fetched one quad ahead so the
  // LDS read overlaps the current quad
  // the quad maxima, kept for the screening pass (16-bit types: they fill
  // the short list's LDS area, which is idle until the publish)
  constexpr bool kKeepQm = Q * kThreads * sizeof(float) <= sizeof(L.ssrc);
  float* qmc = reinterpret_cast<float*>(L.ssrc);
  const uint32_t* penw = L.pen + ((tid * N) >> 5);
  constexpr int kQuadWords = kThreads * N / 32;  // bitmap words per quad row
  const uint32_t pen_shift = (uint32_t)((tid * N) & 31);
  // tokens of the slice from this thread's first position on: quad g holds
  // lim - g * kThreads * N of them (lanes past the end are excluded)
  const int32_t lim = end32 - base32 - tid * N;
  uint32_t pw = penw[0];
  uint32_t nf_acc = 0u;
  float xmax = kNegInf;
  // exp-sum anchor: nbz starts above every quad, so the first finite quad
  // anchors, and the shift of that first anchor clears what came before
  float zt = 0.0f, nbz = __FLT_MAX__;
  // (LP, own pass) the raw logits' statistics, before any exclusion
  RawAcc ra{kNegInf, 0.0f, __FLT_MAX__, 0u};
  for_quads_static(S, nq, [&](int g, uint4& v) -> bool {
    const int32_t i0 = base32 + (tid + g * kThreads) * N;
    const uint32_t pcur = pw;
    if (g + 1 < Q) pw = penw[(g + 1) * kQuadWords];
    const uint32_t probe = nonfinite_probe<DT>(v);
    nf_acc |= probe;
    const int32_t rem = lim - g * (kThreads * N);
    const uint32_t tail = ~0u << (uint32_t)(rem < 0 ? 0 : (rem > N ? N : rem));
    if constexpr (LP && JM == kFused) raw_add<DT>(ra, v, tail & FULL, probe);
    uint32_t ex = ((pcur >> pen_shift) | tail) & FULL;
    if (mrow) ex |= ~staged_allow_bits(mw, i0 - base32, N) & FULL;
    // (NaNs are rare, behind a branch; entry tokens are in most quads of a
    // wave, so the exclusion runs unconditionally, a no-op without bits)
    if (nonfinite_seen<DT>(probe)) {
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float x = vec_elem<DT>(v, e);
        if (x != x) ex |= 1u << e;
      }
    }
    exclude_elems<DT>(v, ex);
    if (jm != kSelectOnly) {
      const float qm = vec_max_nn<DT>(v);  // NaNs are excluded by now
      if constexpr (kKeepQm) qmc[g * kThreads + tid] = qm;
      xmax = __builtin_elementwise_maximum(xmax, qm);
      if (zon) {
        // re-anchor when the quad's terms could pass 2^64 (an exact power-of-
        // two rescale; the anchor is an integer, clamped to +-2^20)
        if (__builtin_fmaf(qm, lgz, nbz) > 64.0f) {
          const float nn = -__builtin_ceilf(__builtin_amdgcn_fmed3f(qm * lgz, -0x1p20f, 0x1p20f));
          zt = __builtin_ldexpf(zt, (int)__builtin_fmaxf(nn - nbz, -512.0f));
          nbz = nn;
        }
#pragma unroll
        for (int e = 0; e < N; ++e)
          zt += __builtin_amdgcn_exp2f(__builtin_fmaf(vec_elem<DT>(v, e), lgz, nbz));
      }
    }
    return true;
  });
  const bool zref = nbz < __FLT_MAX__;
  finish_slice_entries<DT>(P, c, prm, mrow, se, ep, em, emax);
  xmax = __builtin_fmaxf(xmax, emax);
  lds_barrier();  // the entry table is complete
  const int n_all = L.ecount;
  const bool ent_overflow = n_all > kSliceEntryCap;
  const int n_ent = n_all < kSliceEntryCap ? n_all : kSliceEntryCap;
  const bool nonfinite = nonfinite_seen<DT>(nf_acc);
  // (LP, own pass) the slice's raw record, out before any exchange
  if constexpr (LP && JM == kFused) raw_slice<DT>(P, Lk, row, slice, rowp, base32, end32, nq, ra, L);

  RowInfo info;
  if (jm != kSelectOnly) {
    // ------------------------------------------------ B: max
    if (nonfinite) atomicOr(&L.flags, LSAMP_ROW_NONFINITE);
    const float tmax = xmax;  // this thread's largest (transformed) logit
    float tlo = kPosInf;      // smallest finite thread maximum (short lists, k > 1)
    if (K > 1) {
      float hi = wave_max(tmax);
      float lo = wave_min(tmax > kNegInf ? tmax : kPosInf);
      const int wv = tid >> 6;
      __syncthreads();
      if ((tid & 63) == 0) {
        L.redf[wv] = hi;
        L.redf2[wv] = lo;
      }
      __syncthreads();
      hi = L.redf[0];
      lo = L.redf2[0];
#pragma unroll
      for (int i = 1; i < kWaves; ++i) {
        hi = __builtin_fmaxf(hi, L.redf[i]);
        lo = __builtin_fminf(lo, L.redf2[i]);
      }
      __syncthreads();
      xmax = hi;
      tlo = lo;
    } else {
      xmax = block_max(xmax, L.redf);
    }
    const bool posinf = xmax == kPosInf;
    const bool has_finite = xmax > kNegInf && !posinf;
    uint32_t sflags = L.flags | (ent_overflow ? kSliceEntryOverflow : 0u) |
                      (posinf ? kSlicePosInf : 0u);
    const int32_t top = has_finite ? bin_of(xmax, c.c32) : 0;
    SliceSummary* Ssum = ws.summaries + ((size_t)row * kMaxSlices + slice);
    if (P.processed) {
      float* out = P.processed + (size_t)row * (size_t)V;
      for_quads(S, nq, [&](int g, uint4& v) -> bool {
        const int32_t i0 = base32 + (tid + g * kThreads) * N;
        if (i0 >= end32) return false;
        const int32_t li0 = i0 - base32;
        const uint32_t pen = (L.pen[li0 >> 5] >> (uint32_t)(li0 & 31)) & FULL;
#pragma unroll
        for (int e = 0; e < N; ++e) {
          if (i0 + e >= end32 || ((pen >> e) & 1u)) continue;
          out[i0 + e] = to_filter(c, vec_elem<DT>(v, e));
        }
        return false;
      });
      for (int j = tid; j < n_ent; j += kThreads) out[L.etok[j]] = to_filter(c, L.ex[j]);
    }

    if (K > 0) {
      // -------------------------------------------- B': the short list
      // A threshold no higher than the k-th largest thread maximum leaves at
      // least k tokens at or above it; those few are sorted, and the slice's
      // top-k plus ties is published.
      int32_t npub = 0;
      float ylo = kNegInf;
      double zsum = 0.0;
      if (has_finite && !ent_overflow) {
        float tau = xmax;  // k = 1: the maximum itself
        if (K > 1) {
          // thread maxima binned below the slice maximum over a range of at
          // most 32 filter-space nats; the bin where the count reaches k
          // bounds the k-th largest from below (half a bin of slack covers
          // the rounding of the bin index)
          const float D = __builtin_fminf(xmax - tlo, (float)(32.0 * c.tf));
          const float sc = D > 0.0f ? (float)(kTauBins - 1) / D : 0.0f;
          if (tmax > kNegInf) {
            const float fb = (xmax - tmax) * sc;
            const int b = fb < (float)(kTauBins - 1) ? (int)fb : kTauBins - 1;
            atomicAdd(&L.sh.tcnt[b], 1u);
          }
          __syncthreads();
          if (tid < 64) {
            constexpr int kPer = kTauBins / 64;
            uint32_t cb[kPer];
            uint32_t cs = 0u;
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
              cb[i] = L.sh.tcnt[kPer * tid + i];
              cs += cb[i];
            }
            const uint32_t ic = wave_incl_scan(cs);
            const uint64_t hit = __ballot(ic >= (uint32_t)K);
            int bs = kTauBins;  // fewer than k threads hold a finite logit
            if (hit) {
              // first bin of each lane's run where the running count reaches
              // k; lane f's is the answer
              uint32_t acc = ic - cs;
              int pos = kPer - 1;
              bool found = false;
#pragma unroll
              for (int i = 0; i < kPer; ++i) {
                acc += cb[i];
                const bool h = !found && acc >= (uint32_t)K;
                pos = h ? i : pos;
                found = found || h;
              }
              const int f = __builtin_ctzll(hit);
              bs = kPer * f + read_lane(pos, f);
            }
            if (tid == 0) L.misc[6] = bs;
          }
          __syncthreads();
          const int bs = L.misc[6];
          // no bin reaches k: every finite token is a candidate
          tau = bs >= kTauBins ? kNegInf
                               : ((bs == kTauBins - 1 || sc == 0.0f) ? tlo
                                                                    : xmax - ((float)bs + 1.5f) / sc);
        }
        // tempered rows compare fl(x / T): a margin of 2^-20 keeps every
        // token whose filter-space value could tie with the k-th
        const float tc = c.tempered ? tau - (__builtin_fabsf(tau) * 0x1p-20f + 1e-30f) : tau;
        // entry-table terms exp((x - xmax) / T_f) = exp2(fma(x, lgz, nb)); nb's
        // rounding error (exact through an fma) is common to them all
        const float nb = -xmax * lgz;
        const float nb_err = __builtin_fmaf(-xmax, lgz, -nb);
        if (zon && !(xmax * lgz < 0x1p20f)) sflags |= kSliceShortOverflow;  // out of range
        // candidates are the tokens x >= tcp (tcp >= -FLT_MAX also rules out
        // -inf).  A quad holding one is staged whole in the thread's next LDS
        // slot (past kQStage into a discard slot) and its candidates counted,
        // all without branching per token; entry-table candidates are marked
        // by their table position.  A scan of the counts lays the slice's
        // list out, and the quads are expanded as it is published.
        const float tcp = __builtin_fmaxf(tc, -__FLT_MAX__);
        uint4* sq = L.sh.squad + tid;
        int qn = 0, cnt = 0;
        uint32_t qids = 0u;  // staged quad numbers, 5 bits per slot
        // (the kept quad maxima are read into registers at once: the
        // staging stores below would otherwise hold each read back)
        float qv[Q];
        if constexpr (kKeepQm) {
#pragma unroll
          for (int g = 0; g < Q; ++g) qv[g] = qmc[g * kThreads + tid];
        }
        for_quads_static(S, nq, [&](int g, uint4& v) -> bool {
          if ((kKeepQm ? qv[g] : vec_max_nn<DT>(v)) >= tcp) {
#pragma unroll
            for (int e = 0; e < N; ++e) cnt += vec_elem<DT>(v, e) >= tcp ? 1 : 0;
            const int slot = qn < kQStage ? qn : kQStage;
            sq[slot * kThreads] = v;
            qids |= (uint32_t)g << (5 * slot);
            ++qn;
          }
          return false;
        });
        // The slice's sum is kept in 2^40 fixed point (exact in any order):
        // the entry table's order depends on atomics, and the sum must be
        // the same in every run and in both kernel arrangements.  The entry
        // terms carry nb's rounding error back as a factor.
        const float enb = __builtin_amdgcn_exp2f(nb_err);
        uint64_t ze = 0ull;
        uint32_t ebits = 0u;  // bit k: entry tid + k * kThreads is a candidate
        for (int j = tid, k = 0; j < n_ent; j += kThreads, ++k) {
          const float x = L.ex[j];
          if (!(x > kNegInf)) continue;
          if (zon) ze += (uint64_t)(__builtin_amdgcn_exp2f(__builtin_fmaf(x, lgz, nb)) * enb * 0x1p40f);
          if (x >= tcp) {
            ebits |= 1u << k;
            ++cnt;
          }
        }
        // a thread past its slots makes the slice's count exceed any list
        const int cw = qn > kQStage ? kShortPub + 1 : cnt;
        const int ci = wave_incl_scan(cw);
        // this thread's register terms, rescaled from 2^-nbz to e^(xmax / T_f)
        // (xmax * lgz split into a rounded part and its exact residual)
        const float bh = xmax * lgz;
        const float bl = __builtin_fmaf(xmax, lgz, -bh);
        const float zr = (zon && zref) ? zt * __builtin_amdgcn_exp2f((-nbz - bh) - bl) : 0.0f;
        // (each term is at most 1, so zr <= 128; out-of-range rows fall back)
        ze += zr < 0x1p20f ? (uint64_t)(zr * 0x1p40f) : 0ull;
        ze = wave_sum(ze);
        const int wv = tid >> 6;
        __syncthreads();
        if ((tid & 63) == 0) L.redu[wv] = ze;
        if ((tid & 63) == 63) L.redi[wv] = ci;
        __syncthreads();
        ze = 0ull;
        int n = 0, off = ci - cw;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) {
          ze += L.redu[i];
          off += i < wv ? L.redi[i] : 0;
          n += L.redi[i];
        }
        zsum = (double)ze * 0x1p-40;
        if (n > kShortPub) {
          sflags |= kSliceShortOverflow;
        } else {
          // every candidate is published (unsorted; the finalize ranks them):
          // each thread lists its raw (value, id) pairs in LDS, then thread j
          // forms key j (one division per thread, not a wave's worth of
          // serial ones) and stores it
          npub = n;
          uint64_t* pub = reinterpret_cast<uint64_t*>(ws.cands + (size_t)row * kCandCap) +
                          (size_t)slice * kShortPub;
          uint64_t* lst = L.ssrc;  // [n] raw pairs: value bits << 32 | id
          auto raw = [](float x, int32_t id) {
            return ((uint64_t)__float_as_uint(x) << 32) | (uint64_t)(uint32_t)id;
          };
          // (the staged quads are read at once; a token that is not a
          // candidate writes to this thread's own slot past the list, so
          // the expansion does not branch per token)
          int w = off;
          uint4 sv[kQStage];
#pragma unroll
          for (int k = 0; k < kQStage; ++k) sv[k] = sq[k * kThreads];
          const int dump = kExpandDump + tid;
#pragma unroll
          for (int k = 0; k < kQStage; ++k) {
            if (k < qn) {
              const int32_t i0 = base32 + (tid + (int)((qids >> (5 * k)) & 31u) * kThreads) * N;
#pragma unroll
              for (int e = 0; e < N; ++e) {
                const float x = vec_elem<DT>(sv[k], e);
                const bool hit = x >= tcp;
                lst[hit ? w : dump] = raw(x, i0 + e);
                w += hit ? 1 : 0;
              }
            }
          }
          for (; ebits != 0u; ebits &= ebits - 1u) {
            const int j = tid + __builtin_ctz(ebits) * kThreads;
            lst[w++] = raw(L.ex[j], L.etok[j]);
          }
          lds_barrier();
          for (int j = tid; j < n; j += kThreads) {
            const uint64_t r = lst[j];
            st_coherent(&pub[j], cand_key(to_filter(c, __uint_as_float((uint32_t)(r >> 32))),
                                          (int32_t)(uint32_t)r));
          }
          // a lower bound on the values of the published keys
          ylo = to_filter(c, tcp);
        }
      }
      if (tid == 0) {
        st_coherent_f32(&Ssum->x_max, xmax);
        st_coherent(&Ssum->top_bin, top);
        st_coherent(&Ssum->flags, sflags);
        st_coherent(&Ssum->n_finite, (has_finite || posinf) ? 1 : 0);
        st_coherent_f64(&Ssum->zs, zsum);
        st_coherent(&Ssum->npub, npub);
        st_coherent_f32(&Ssum->ylo, ylo);
      }
      if (MODE == kFused) {
        // First exchange of a short-list row: the last slice to publish
        // draws the token.  The others wait, only when every slice of the
        // row has started, to learn whether a slice needs the histogram path
        // instead; a slice that cannot wait or gives up leaves, and if the
        // row does fall back, the last arriver builds its histogram.
        drain_memory();
        __syncthreads();
        if (tid == 0) {
          asm volatile("" ::"v"(tick));
          uint32_t* sync = row_sync(ws, row);
          // (the arrival's atomic returns the start count too; a slice that
          // has started since only makes this one leave)
          const uint32_t word = __hip_atomic_fetch_add(sync + kSyncArrive, 1u, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
          const uint32_t prev = word & kArriveMask, started = word >> 16;
          const bool last = prev + 1u == (uint32_t)G;
          int w = 1;
          if (!last)
            w = started >= (uint32_t)G
                    ? wait_exchange(ws, sync, (uint32_t)G, kClaimStats + (uint32_t)slice)
                    : 0;
          L.wait = w;
          L.last = last ? 1 : 0;
        }
        __syncthreads();
        if (L.last) {
          if (short_gather<DT>(ws, P, row, c, prm, L)) {
            short_finish<DT>(ws, P, row, c, prm, L, rowp, mrow, K, lpp);
            return kJobLeave;
          }
          // the row falls back: this slice's histogram, then those of the
          // slices that left
          if (tid == 0) L.x1 = 1;
        } else if (L.wait != 1 || !short_fallback(ws, row, G, L)) {
          return kJobLeave;
        } else {
          // the row falls back: this slice's histogram, unless the first
          // exchange's last arriver has claimed it
          if (tid == 0) L.won = claim_bit(row_sync(ws, row), kClaimStats + (uint32_t)slice) ? 1 : 0;
          __syncthreads();
          if (!L.won) return kJobLeave;
        }
      }
    }

    // ------------------------------------------------ B: histogram
    const bool want_hist = has_finite && c.kind != LSAMP_KIND_ARGMAX;
    if (want_hist) {
      const float tail_edge = (float)(top - kBins + 1);
      // Branch-free per token (excluded tokens add zero to a discard word of
      // their lane), so the tokens of a quad interleave.
      const int discard = kHist + (tid & 63);
      // Masses are relative to the top edge of the token's bin (in-window,
      // j < kBins, i.e. floor(s) >= tail_edge) or to tail_edge (the tail):
      // both are s - max(floor(s) + 1, tail_edge) <= 0, so every token adds
      // at most 2^kMassFracBits.  A -inf token's mass is 0.
      auto add = [&](float x) {
        const bool ok = x > kNegInf;
        const float s = bin_pos(x, c.c32);
        const float fb = __builtin_floorf(s);
        const int j = top - (int)fb;
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(
            s - __builtin_amdgcn_fmed3f(fb + 1.0f, tail_edge, 3.0e9f), c.lg, (float)kMassFracBits));
        const int idx = ok ? (j < kTail ? j : kTail) : discard;
        // (an excluded token's count lands in its lane's discard word, which
        // nothing reads)
        constexpr uint32_t hi = 1u << (kCountShift - 32);
        atomicAdd(reinterpret_cast<unsigned long long*>(&L.u.hist[idx]),
                  (unsigned long long)(((uint64_t)hi << 32) | (uint64_t)(uint32_t)e));
      };
      auto bin_quad = [&](int g, uint4& v) -> bool {
#pragma unroll
        for (int e = 0; e < N; ++e) add(vec_elem<DT>(v, e));
        return false;
      };
      // 16-bit slabs over static register positions (no register-relative
      // moves: C3 and C5 0.2-1.4 us faster over three runs); the fp32 slab's
      // 32 quads stay a rolled loop, which measured 1.4 us faster at C4
      if constexpr (N == 8)
        for_quads_static(S, nq, bin_quad);
      else
        for_quads(S, nq, bin_quad);
      for (int j2 = tid; j2 < n_ent; j2 += kThreads) {
        const float x = L.ex[j2];
        if (x > kNegInf && x != kPosInf) add(x);
      }
    }
    __syncthreads();
    // publish the slice summary; n_finite is the histogram's token count
    // (rows that build one) or whether the slice holds a finite logit
    int32_t nfin = 0;
    double zs = 0.0;  // total mass relative to the top edge of the slice's top bin
    if (want_hist) {
      const double inv_frac = 1.0 / (double)(1ull << kMassFracBits);
      for (int i = tid; i < kHist; i += kThreads) {
        const uint64_t w = L.u.hist[i];
        st_coherent(&Ssum->hist[i], w);
        if (w == 0ull) continue;
        nfin += (int32_t)(w >> kCountShift);
        // bin i's top edge lies i bins below the slice's; the tail's mass is
        // relative to the window's lowest edge, kBins below
        zs += (double)(w & kMassMask) * inv_frac * fexp(-(double)i / (32.0 * c.tf));
      }
      nfin = wave_sum(nfin);
      zs = wave_sum(zs);
      const int wv = tid >> 6;
      if ((tid & 63) == 0) {
        L.redi[wv] = nfin;
        L.redd[wv] = zs;
      }
      __syncthreads();
      nfin = 0;
      zs = 0.0;
#pragma unroll
      for (int i = 0; i < kWaves; ++i) {
        nfin += L.redi[i];
        zs += L.redd[i];
      }
    } else {
      nfin = (has_finite || posinf) ? 1 : 0;
    }
    if (tid == 0) {
      st_coherent_f32(&Ssum->x_max, xmax);
      st_coherent(&Ssum->top_bin, top);
      st_coherent(&Ssum->flags, sflags);
      st_coherent(&Ssum->n_finite, nfin);
      st_coherent_f64(&Ssum->z, zs);
    }
    if (MODE == kFused) {
      // The exchange (a short-list row that fell back counts its second
      // arrival).  The last arrival merges at once.  Another slice waits for
      // the rest only when every slice of the row has started, then claims
      // its own select; a slice that cannot wait, gives up, or finds its
      // select claimed leaves it to the last arriver.  Every slice that
      // merges computes the same cut (the merge is deterministic).
      const uint32_t target = (uint32_t)(Krow > 0 ? 2 * G : G);
      drain_memory();
      __syncthreads();
      // Thread 0 arrives (the atomic returns the start count too); unless
      // this is the last arrival (or the hand-off of a row that fell back,
      // below), it waits and sends the claim of its own select, whose
      // result is checked after the merge (the round trip overlaps the
      // merge's loads).  Same barriers as a plain wait.
      uint32_t claimed = 0u;
      if (tid == 0) {
        asm volatile("" ::"v"(tick));
        uint32_t* sync = row_sync(ws, row);
        const uint32_t word = __hip_atomic_fetch_add(sync + kSyncArrive, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t prev = word & kArriveMask, started = word >> 16;
        const bool last = prev + 1u == target;
        if (last) L.xlast = 1;
        int w = 1;
        if (!last && !L.x1) {
          w = started >= (uint32_t)G ? wait_exchange(ws, sync, target, (uint32_t)own) : 0;
          if (w == 1)
            claimed = __hip_atomic_fetch_or(sync + kSyncClaims, 1u << own, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
        }
        L.wait = w;
      }
      __syncthreads();
      if (L.x1) {
        // the first exchange's last arriver of a row that fell back builds
        // the histograms of the slices that left that exchange, then waits
        // (unless its arrival was the last) as any slice does
        if (tid == 0) L.job = claim_next(row_sync(ws, row), G, own, kClaimStats, L.from_stats);
        __syncthreads();
        if (L.job >= 0) return next_job(kBehalfStats, L.job);
        if (tid == 0 && !L.xlast) {
          uint32_t* sync = row_sync(ws, row);
          // (claimed histograms took a while: the start count is read again)
          const int w = (ld_coherent(sync + kSyncArrive) >> 16) >= (uint32_t)G
                            ? wait_exchange(ws, sync, target, (uint32_t)own)
                            : 0;
          if (w == 1)
            claimed = __hip_atomic_fetch_or(sync + kSyncClaims, 1u << own, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
          L.wait = w;
        }
        __syncthreads();
      }
      if (!L.xlast && L.wait != 1) return kJobLeave;
      merge_stage(ws, P, row, c, L);
      if (tid < 64) merge_wave<true>(ws, P, row, c, prm, L);
      if (tid == 0) L.won = (L.xlast || ((claimed >> own) & 1u) == 0u) ? 1 : 0;
      __syncthreads();
      if (!L.won) return kJobLeave;  // (the last arriver does this select)
      // (after a claimed histogram the registers hold another slice: the
      // own select re-reads the own slice)
      if (jm == kBehalfStats) return next_job(kSelectOnly, own);
      info = L.info;
    } else {
      uint32_t* const arrive = row_sync(ws, row) + kSyncArrive;
      if (!arrive_last(arrive, (uint32_t)G, &L.last)) return kJobLeave;
      if (K > 0 && short_gather<DT>(ws, P, row, c, prm, L)) {
        short_finish<DT>(ws, P, row, c, prm, L, rowp, mrow, K, lpp);
        if (tid == 0) *arrive = 0u;
        return kJobLeave;
      }
      merge_row(ws, P, row, c, prm, L);
      if (tid == 0) {
        ws.rows[row] = L.info;
        *arrive = 0u;
      }
      return kJobLeave;
    }
  } else if (MODE == kFused) {
    // a claimed select: the cut this work-group merged
    info = L.info;
  } else {
    if (tid == 0) L.info = ws.rows[row];
    __syncthreads();
    info = L.info;
  }

  // ------------------------------------------- C: classify against the cut
  const float y_max = info.mode == kModePosInf ? kPosInf : to_filter(c, info.x_max);
  const bool active = info.mode != kModeEmpty;
  if (tid < kSliceChunks) L.u.s.chunk[tid] = 0ull;
  if (tid == 0) {
    L.ncand = 0;
    L.nlist = 0;
  }
  __syncthreads();
  double ent = 0.0;
  float min_kept = kPosInf;
  int32_t n_kept = 0;
  uint8_t* kout = P.keep ? P.keep + (size_t)row * (size_t)V : nullptr;
  if (!active && kout)
    for (int64_t i = base + tid; i < end; i += kThreads) kout[i] = 0;
  // Kept tokens are listed (fast draw path) only when the whole row keeps at
  // most kKeptCap tokens above the cut bin; otherwise the draw scans a chunk.
  const bool list_on = info.count_above <= kKeptCap;
  // the kept count, smallest kept value and entropy feed only the statistics
  const bool want_stats = P.stats_full != 0;
  auto keep_token = [&](float x, int32_t id, uint64_t& part) {
    const float y = to_filter(c, x);
    const uint64_t wq = weight(y, y_max, c.scale);
    part += wq;
    if (want_stats) {
      ent += (double)wq * (1.0 / 1099511627776.0) * (double)weight_arg(y, y_max, c.scale);
      min_kept = __builtin_fminf(min_kept, y);
      ++n_kept;
    }
    if (list_on) {
      const int ks = atomicAdd(&L.nlist, 1);
      if (ks < kKeptCap) {
        L.u.s.klist[ks].w = wq;
        L.u.s.klist[ks].id = id;
      }
    }
  };
  auto cand_token = [&](float x, int32_t id) {
    const int cs = atomicAdd(&L.ncand, 1);
    if (cs < kWgCandCap) {
      L.u.s.cand[cs].y = to_filter(c, x);
      L.u.s.cand[cs].id = id;
    }
  };
  const ClassRule rule = make_rule(info, c);
  if (active) {
    // The bin screen passes the kept and cut-bin tokens only (a few percent
    // of a top-p row, spread over every wave): they are queued per wave in
    // LDS, in id order, as (offset in the slice, value bits), and classified
    // and weighed with every lane busy, so a wave does not pay the per-token
    // work once for each lane that holds such a token.
    uint2* q = reinterpret_cast<uint2*>(L.ssrc) + (tid >> 6) * kSelQueue;
    const int lane = tid & 63;
    int qn = 0;  // wave-uniform
    auto flush = [&]() {
      for (int i0 = 0; i0 < qn; i0 += 64) {
        const int i = i0 + lane;
        uint64_t w = 0ull;
        int ch = -1;
        if (i < qn) {
          const uint2 en = q[i];
          const float x = __uint_as_float(en.y);
          const int32_t id = base32 + (int32_t)en.x;
          const int cls = classify(rule, x);
          if (cls == kKept) {
            keep_token(x, id, w);
            ch = (int)(en.x / kChunk);
          } else if (cls == kCand) {
            cand_token(x, id);
          }
        }
        // chunk sums: one atomic per round when its kept tokens share a chunk
        const int chm = wave_min(ch < 0 ? 0x7fffffff : ch);
        const bool one = __ballot(ch >= 0 && ch != chm) == 0ull;
        if (one) {
          const uint64_t sum = wave_sum(w);
          if (lane == 0 && sum)
            atomicAdd(reinterpret_cast<unsigned long long*>(&L.u.s.chunk[chm]),
                      (unsigned long long)sum);
        } else if (w) {
          atomicAdd(reinterpret_cast<unsigned long long*>(&L.u.s.chunk[ch]), (unsigned long long)w);
        }
      }
      qn = 0;
    };
    for_quads(S, nq, [&](int g, uint4& v) -> bool {
      const int32_t li0 = (tid + g * kThreads) * N;
      uint32_t m = 0u;
#pragma unroll
      for (int e = 0; e < N; ++e)
        m |= (vec_elem<DT>(v, e) * rule.c32 >= rule.screen ? 1u : 0u) << e;
      if (__ballot(m != 0u) == 0ull) return false;
      // the lanes' offsets in the queue: an exclusive prefix of their counts
      // (at most N <= 8: four ballots)
      const int cnt = __builtin_popcount(m);
      int off = 0, tot = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint64_t bl = __ballot((cnt >> b) & 1);
        off += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bl >> 32),
                                              __builtin_amdgcn_mbcnt_lo((uint32_t)bl, 0u))
               << b;
        tot += __builtin_popcountll(bl) << b;
      }
      if (qn + tot > kSelQueue) flush();
      int o = qn + off;
#pragma unroll
      for (int e = 0; e < N; ++e)
        if ((m >> e) & 1u)
          q[o++] = make_uint2((uint32_t)(li0 + e), __float_as_uint(vec_elem<DT>(v, e)));
      qn += tot;
      return false;
    });
    flush();
    if (kout) {
      // keep bytes of tokens outside the entry table (re-read; an output for
      // parity checks only); candidates' bytes are written by the finalize
#pragma nounroll
      for (int g = 0; g < nq; ++g) {
        const int32_t i0 = base32 + (tid + g * kThreads) * N;
        if (i0 >= end32) continue;
        const int32_t li0 = i0 - base32;
        const uint32_t pen = (L.pen[li0 >> 5] >> (uint32_t)(li0 & 31)) & FULL;
        const uint32_t allow = mask_allow_bits(mrow, P.mask_words, P.mask_bits, P.mask_tail, i0, N);
#pragma nounroll
        for (int q = 0; q < N && i0 + q < end32; ++q) {
          if ((pen >> q) & 1u) continue;
          const float x = load_scalar<DT>(rowp, i0 + q);
          const int cls = ((allow >> q) & 1u) ? classify(rule, x) : kDrop;
          if (cls != kCand) kout[i0 + q] = cls == kKept ? 1 : 0;
        }
      }
    }
    for (int j2 = tid; j2 < n_ent; j2 += kThreads) {
      const float x = L.ex[j2];
      const int cls = classify(rule, x);
      const int32_t t = L.etok[j2];
      if (kout && cls != kCand) kout[t] = cls == kKept ? 1 : 0;
      if (cls == kKept) {
        uint64_t w = 0ull;
        keep_token(x, t, w);
        atomicAdd(reinterpret_cast<unsigned long long*>(&L.u.s.chunk[(t - base32) / kChunk]),
                  (unsigned long long)w);
      } else if (cls == kCand) {
        cand_token(x, t);
      }
    }
  }
  if (want_stats) {
    // one exchange for the three work-group reductions
    ent = wave_sum(ent);
    min_kept = wave_min(min_kept);
    n_kept = wave_sum(n_kept);
    const int wv = tid >> 6;
    __syncthreads();
    if ((tid & 63) == 0) {
      L.redd[wv] = ent;
      L.redf[wv] = min_kept;
      L.redi[wv] = n_kept;
    }
    __syncthreads();
    ent = 0.0;
    min_kept = kPosInf;
    n_kept = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      ent += L.redd[i];
      min_kept = __builtin_fminf(min_kept, L.redf[i]);
      n_kept += L.redi[i];
    }
  } else {
    // the chunk sums, candidates and kept list are complete past here
    __syncthreads();
  }

  // publish chunk sums, candidates, kept list, partials
  const int64_t chunk0 = base / kChunk;
  const int nch = (int)((end - base + kChunk - 1) / kChunk);
  uint64_t* rowchunks = ws.chunk_w + (size_t)row * (size_t)ws.max_chunks;
  if (tid < nch) st_coherent(&rowchunks[chunk0 + tid], L.u.s.chunk[tid]);
  const int ncand = L.ncand;
  const int nlist = list_on ? L.nlist : kKeptCap + 1;
  if (tid == 0)
    L.misc[0] = ncand > 0 ? (int)__hip_atomic_fetch_add(&ws.cand_count[row], (uint32_t)ncand,
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : 0;
  __syncthreads();
  const int gbase = L.misc[0];
  Candidate* rc = ws.cands + (size_t)row * kCandCap;
  const int ncopy = ncand < kWgCandCap ? ncand : kWgCandCap;
  for (int i = tid; i < ncopy; i += kThreads)
    if (gbase + i < kCandCap) {
      st_coherent_f32(&rc[gbase + i].y, L.u.s.cand[i].y);
      st_coherent(&rc[gbase + i].id, L.u.s.cand[i].id);
    }
  KeptItem* kl = ws.klist + ((size_t)row * kMaxSlices + slice) * kKeptCap;
  if (tid < nlist && tid < kKeptCap) {
    st_coherent(&kl[tid].w, L.u.s.klist[tid].w);
    st_coherent(&kl[tid].id, L.u.s.klist[tid].id);
  }
  if (tid == 0) {
    SelectPartial* sp = ws.partials + (size_t)row * kMaxSlices + slice;
    st_coherent_f64(&sp->ent, ent);
    st_coherent_f32(&sp->min_kept, min_kept);
    st_coherent(&sp->n_kept, n_kept);
    st_coherent(&sp->n_cand, ncand);
    st_coherent(&sp->n_list, nlist);
    st_coherent(&sp->overflow, ent_overflow ? 1 : 0);
  }
  if (arrive_last(&ws.arrive_select[row], (uint32_t)G, &L.last))
    finalize_row<DT>(ws, P, row, c, prm, info, L, rowp, mrow, lpp);
  if (MODE != kFused) return kJobLeave;
  // the exchange's last arriver does the selects of the slices that left
  if (L.xlast) {
    if (tid == 0) L.job = claim_next(row_sync(ws, row), G, own, 0u, L.from_select);
    __syncthreads();
    if (L.job >= 0) return next_job(kSelectOnly, L.job);
  }
  return kJobLeave;
}

// A task (row, slice).  Split mode: one pass.  Fused arrangement: the
// work-group's own slice (with its start ticket), then whatever it claimed
// for slices that left, and the departure; returns (thread 0) the row's
// departure count before this one, for clear_if_last.
template <int DT, int MODE, bool LP = false>
__device__ __forceinline__ uint32_t run_task(const Workspace& ws, const SamplePlan& P, int row,
                                             int slice, TaskLds& L, const FusedLp& Lk) {
  if constexpr (MODE != kFused) {
    (void)slice_job<DT, MODE, MODE, false>(ws, P, row, slice, L, slice, Lk);
    return 0u;
  } else {
    if (threadIdx.x == 0) {
      L.x1 = 0;
      L.xlast = 0;
      L.from_stats = 0;
      L.from_select = 0;
    }
    // (no barrier: the job's first barriers come after its loads are issued,
    // before anything reads these)
    int next = slice_job<DT, kFused, kFused, LP>(ws, P, row, slice, L, slice, Lk);
    // (after the own pass: at most G - 1 claimed histograms and G claimed
    // selects; every thread returns the same job, read from LDS)
    for (int n = 0; n < 2 * kMaxSlices && next >= 0; ++n) {
      next = __builtin_amdgcn_readfirstlane(next);
      const int s = next & 0xff;
      __syncthreads();
      next = (next >> 8) == kBehalfStats
                 ? slice_job<DT, kFused, kBehalfStats, LP>(ws, P, row, s, L, slice, Lk)
                 : slice_job<DT, kFused, kSelectOnly, LP>(ws, P, row, s, L, slice, Lk);
    }
    // (thread 0 has consumed its start ticket's result at the exchange)
    return threadIdx.x == 0 ? leave_row(ws, row) : 0u;
  }
}

// ================================================================ kernels
// ONE: every row fits one round of the grid (no loop over rounds, so nothing
// is hoisted out of one and spilled before the first load).
// LP: raw log-probabilities in the same pass (lsamp_step); `Lk` is read
// where it is used (the raw record and the finalize), not held throughout.
template <int DT, bool ONE, bool LP>
__global__ __launch_bounds__(kThreads) void k_fused(Workspace wsk, SamplePlan Pk, FusedLp Lk) {
  __shared__ TaskLds L;
  // The kernel arguments are read in one round of scalar loads and held as
  // opaque values (otherwise they are fetched lazily, over several dependent
  // rounds, before the first global load can be issued).
  const Workspace ws = in_sgprs(wsk);
  const SamplePlan P = in_sgprs(Pk);
  const int G = P.slices;
  const int rowslot = (int)blockIdx.x / G;
  const int slice = (int)blockIdx.x % G;
  if (ONE) {
    if (rowslot < P.rows) {
      const uint32_t out = run_task<DT, kFused, LP>(ws, P, rowslot, slice, L, Lk);
      if (threadIdx.x == 0) clear_if_last(ws, rowslot, G, out);
    }
    return;
  }
  // More tasks than work-groups: each work-group takes the next task (row-
  // major, slice-minor) from a counter when it has finished the last one, so
  // fast rows (short lists) and slow ones (wide nuclei) balance over the
  // grid.  The tasks taken always form a prefix, and a work-group finishes a
  // task before it takes another, so the slices a row waits for are held by
  // running work-groups or are next in line for the first one free.
  const uint32_t total = (uint32_t)(P.rows * G);
  // Rows in the order their tasks are taken: rows bound for the histogram
  // path (the slow ones) first, short-list rows after, so the grid's last
  // tasks are short.  Every work-group derives the same order from the
  // rows' parameters (one load per thread, two block scans).
  constexpr int kOrderCap = 1024;
  __shared__ uint16_t order[kOrderCap];
  const bool ordered = P.rows <= kOrderCap;
  if (ordered) {
    int placed_slow = 0, placed_short = 0;
    for (int r0 = 0; r0 < P.rows; r0 += kThreads) {
      const int r = r0 + (int)threadIdx.x;
      int slow = 0;
      if (r < P.rows) {
        const lsamp_row_params prm = P.params[params_index(P, r)];
        slow = short_k(make_ctx(P.semantics, prm), prm, P.vocab) == 0 ? 1 : 0;
      }
      const int fast = r < P.rows ? 1 - slow : 0;
      int n_slow = 0, n_fast = 0;
      const int es = block_excl_scan(slow, L.redi, &n_slow);
      const int ef = block_excl_scan(fast, L.redi, &n_fast);
      // (short-list rows fill the order from its end)
      if (r < P.rows)
        order[slow ? placed_slow + es : P.rows - 1 - (placed_short + ef)] = (uint16_t)r;
      placed_slow += n_slow;
      placed_short += n_fast;
    }
    __syncthreads();
  }
  // The first task of work-group b is task b (the first takes of the grid
  // would return 0 .. grid - 1 in some order, all at once on one counter);
  // later takes count from the grid's size.
  uint32_t t = blockIdx.x;
  // (thread 0) the last task's row and its departure count, checked once the
  // next take has come back: the two round trips overlap
  int pend_row = -1;
  uint32_t pend_out = 0u;
  for (bool first = true;; first = false) {
    if (!first) {
      if (threadIdx.x == 0) {
        L.task = gridDim.x + __hip_atomic_fetch_add(ws.tasks, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        if (pend_row >= 0) clear_if_last(ws, pend_row, G, pend_out);
      }
      __syncthreads();
      t = L.task;
      __syncthreads();
    }
    if (t >= total) break;
    // (through empty asm: nothing derived from the arguments is hoisted out
    // of the loop and held across tasks)
    const Workspace wsr = in_sgprs(ws);
    const SamplePlan Pr = in_sgprs(P);
    const int q = (int)(t / (uint32_t)G);
    // (row and slice through readfirstlane: the divergence analysis cannot
    // see that a value read from LDS at a uniform address is uniform once
    // the task holds a loop of its own)
    const int row = __builtin_amdgcn_readfirstlane(ordered ? (int)order[q] : q);
    const int slice_t = __builtin_amdgcn_readfirstlane((int)(t % (uint32_t)G));
    pend_out = run_task<DT, kFused, LP>(wsr, Pr, row, slice_t, L, Lk);
    pend_row = row;
    __syncthreads();
  }
  // every work-group ends with one failed take (the counter then holds
  // total - grid + grid): the last of those returns it to zero for the next
  // step
  if (threadIdx.x == 0 && t == total + gridDim.x - 1u) st_coherent(ws.tasks, 0u);
}

template <int DT>
__global__ __launch_bounds__(kThreads) void k_stats(Workspace ws, SamplePlan P) {
  __shared__ TaskLds L;
  const FusedLp none{-1, nullptr, nullptr, nullptr, nullptr};
  run_task<DT, kStatsOnly>(ws, P, (int)blockIdx.y, (int)blockIdx.x, L, none);
}

template <int DT>
__global__ __launch_bounds__(kThreads) void k_select(Workspace ws, SamplePlan P) {
  __shared__ TaskLds L;
  const FusedLp none{-1, nullptr, nullptr, nullptr, nullptr};
  run_task<DT, kSelectOnly>(ws, P, (int)blockIdx.y, (int)blockIdx.x, L, none);
}

template <int DT>
int launch_dt(const Workspace& ws, const SamplePlan& P, const FusedLp* lp, hipStream_t st,
              void* const* events) {
  auto mark = [&](int i) {
    if (events) (void)hipEventRecord(reinterpret_cast<hipEvent_t>(events[i]), st);
  };
  mark(0);
  if (P.fused) {
    const int rounds_rows = P.rows < P.rows_per_round ? P.rows : P.rows_per_round;
    const dim3 grid((unsigned)(rounds_rows * P.slices));
    const FusedLp none{-1, nullptr, nullptr, nullptr, nullptr};
    const FusedLp& lk = lp ? *lp : none;
    // (fp32 steps run fused only when every row fits one round: the
    // several-rounds instantiation with the fp32 slab does not fit the
    // registers, so it is not built, and the planner gives such steps the
    // split kernels)
    if constexpr (DT == LSAMP_DTYPE_F32) {
      if (lp)
        hipLaunchKernelGGL((k_fused<DT, true, true>), grid, dim3(kThreads), 0, st, ws, P, lk);
      else
        hipLaunchKernelGGL((k_fused<DT, true, false>), grid, dim3(kThreads), 0, st, ws, P, lk);
    } else {
      const bool one = P.rows <= P.rows_per_round;
      auto kf = lp ? (one ? k_fused<DT, true, true> : k_fused<DT, false, true>)
                   : (one ? k_fused<DT, true, false> : k_fused<DT, false, false>);
      hipLaunchKernelGGL(kf, grid, dim3(kThreads), 0, st, ws, P, lk);
    }
    mark(1);
  } else {
    const dim3 grid((unsigned)P.slices, (unsigned)P.rows);
    hipLaunchKernelGGL(k_stats<DT>, grid, dim3(kThreads), 0, st, ws, P);
    mark(1);
    hipLaunchKernelGGL(k_select<DT>, grid, dim3(kThreads), 0, st, ws, P);
  }
  mark(2);
  return (int)hipGetLastError();
}

// ============================================================ MTP verify
// Is (y, id) among the n kept candidates of a row (sorted by cand_key,
// descending)?  Binary search (in LDS when the row's candidates were staged
// there); called for cut-bin tokens only.
__device__ __forceinline__ bool in_kept_list(const Candidate* rc, int n, uint64_t key) {
  int lo = 0, hi = n - 1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    const uint64_t k = cand_key(rc[mid].y, rc[mid].id);
    if (k == key) return true;
    if (k > key) lo = mid + 1; else hi = mid - 1;
  }
  return false;
}

// Kept weight of token i (transformed logit x) in a sampled row, from the
// row's decision (its ClassRule and filter-space maximum) and its kept
// candidates.
__device__ __forceinline__ uint64_t kept_weight_of(const RowCtx& c, const ClassRule& rule,
                                                   const Candidate* kl, int nk, float y_max,
                                                   float x, int32_t i) {
  if (x != x) x = kNegInf;
  const int cls = classify(rule, x);
  if (cls == kDrop) return 0ull;
  const float y = to_filter(c, x);
  if (cls == kCand && !in_kept_list(kl, nk, cand_key(y, i))) return 0ull;
  return weight(y, y_max, c.scale);
}

__device__ __forceinline__ bool aligned16(const void* p) {
  return ((uintptr_t)p & 15u) == 0u;
}

// The two rows of a residual draw (target and draft at the rejected
// position), resolved once per work-group.
struct ResidualRows {
  RowCtx c;
  ClassRule qt, qd;
  const Candidate* ct;  // kept cut-bin candidates (in LDS when they fit)
  const Candidate* cd;
  int32_t nct, ncd;
  float ymt, ymd;       // filter-space maxima
  uint64_t Wt, Wd;      // kept weights
  const char* trow;
  const char* drow;
  int32_t V;
  bool vec;             // the target row is 16-byte aligned
};

// Token i's kept target weight, and (with_draft) its residual weight
// max(0, p_t - p_d) with both probabilities quantized to 2^-52.
__device__ __forceinline__ void residual_weights(const ResidualRows& r, float xt, float xd,
                                                 int32_t i, bool with_draft, uint64_t& wt,
                                                 uint64_t& wr) {
  wt = kept_weight_of(r.c, r.qt, r.ct, r.nct, r.ymt, xt, i);
  wr = 0ull;
  if (!with_draft || wt == 0ull) return;
  const uint64_t wd = kept_weight_of(r.c, r.qd, r.cd, r.ncd, r.ymd, xd, i);
  const uint64_t a = (uint64_t)((double)wt / (double)r.Wt * 4503599627370496.0);
  const uint64_t b = r.Wd ? (uint64_t)((double)wd / (double)r.Wd * 4503599627370496.0) : 0ull;
  wr = a > b ? a - b : 0ull;
}

constexpr int kVerifyCandLds = 1024;  // kept candidates of a row staged in LDS
constexpr int kVerifyBatch = 4;       // queue entries a lane evaluates per round trip

// Screen a wave's span of the target row (kVerifySpan tokens from q0, 64
// lanes x N-token vectors per step, coalesced): every token the target's bin
// screen does not drop (kept and cut-bin tokens; every token when the row has
// no finite screen) goes to the wave's LDS queue as its offset from q0, in id
// order.  Returns the count.  Most tokens cost a multiply and a compare.
template <int DT>
__device__ __forceinline__ int residual_screen(const ResidualRows& r, int32_t q0,
                                               uint16_t* queue, int lane) {
  constexpr int N = Vec<DT>::N;
  constexpr int kSteps = kVerifySpan / (64 * N);
  uint4 tv[kSteps];
#pragma unroll
  for (int k = 0; k < kSteps; ++k)
    tv[k] = load_vec<DT>(r.trow, (int64_t)q0 + (k * 64 + lane) * N, r.V, r.vec);
  int n = 0;
#pragma unroll
  for (int k = 0; k < kSteps; ++k) {
    const int off0 = (k * 64 + lane) * N;
    uint32_t m = 0u;
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float x = vec_elem<DT>(tv[k], e);
      const bool drop = x * r.qt.c32 < r.qt.screen || q0 + off0 + e >= r.V;
      m |= drop ? 0u : 1u << e;
    }
    // exclusive prefix of the lanes' counts (at most 8: four ballots)
    const int cnt = __builtin_popcount(m);
    int off = 0, tot = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint64_t bl = __ballot((cnt >> b) & 1);
      off += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bl >> 32),
                                            __builtin_amdgcn_mbcnt_lo((uint32_t)bl, 0u))
             << b;
      tot += __builtin_popcountll(bl) << b;
    }
    int o = n + off;
#pragma unroll
    for (int e = 0; e < N; ++e)
      if ((m >> e) & 1u) queue[o++] = (uint16_t)(off0 + e);
    n += tot;
  }
  return n;
}

// The ids and logits of queue entries g0 + b*64 + lane (b < kVerifyBatch):
// all loads of a batch go out together.
template <int DT>
__device__ __forceinline__ void residual_batch(const ResidualRows& r, int32_t q0,
                                               const uint16_t* queue, int n, int g0, int lane,
                                               bool with_draft, int32_t (&id)[kVerifyBatch],
                                               float (&xt)[kVerifyBatch],
                                               float (&xd)[kVerifyBatch]) {
#pragma unroll
  for (int b = 0; b < kVerifyBatch; ++b) {
    const int idx = g0 + b * 64 + lane;
    id[b] = idx < n ? q0 + (int32_t)queue[idx] : -1;
  }
#pragma unroll
  for (int b = 0; b < kVerifyBatch; ++b) {
    xt[b] = id[b] >= 0 ? load_scalar<DT>(r.trow, id[b]) : kNegInf;
    xd[b] = with_draft && id[b] >= 0 ? load_scalar<DT>(r.drow, id[b]) : kNegInf;
  }
}

// This lane's sums over the queued tokens of the target's kept weight and of
// the residual weight (with_draft).
template <int DT>
__device__ __forceinline__ void residual_sums(const ResidualRows& r, int32_t q0,
                                              const uint16_t* queue, int n, int lane,
                                              bool with_draft, uint64_t& st, uint64_t& sr) {
  st = 0ull;
  sr = 0ull;
  for (int g0 = 0; g0 < n; g0 += 64 * kVerifyBatch) {
    int32_t id[kVerifyBatch];
    float xt[kVerifyBatch], xd[kVerifyBatch];
    residual_batch<DT>(r, q0, queue, n, g0, lane, with_draft, id, xt, xd);
#pragma unroll
    for (int b = 0; b < kVerifyBatch; ++b) {
      uint64_t wt = 0ull, wr = 0ull;
      if (id[b] >= 0) residual_weights(r, xt[b], xd[b], id[b], with_draft, wt, wr);
      st += wt;
      sr += wr;
    }
  }
}

// The queued token whose run of the draw weight (residual, or the target's
// own) holds t, counted from the wave's first token, in id order; -1 if none.
template <int DT>
__device__ __forceinline__ int32_t residual_find(const ResidualRows& r, int32_t q0,
                                                 const uint16_t* queue, int n, int lane,
                                                 bool use_res, uint64_t t) {
  uint64_t cum = 0ull;
  int32_t found = -1;
  for (int g0 = 0; g0 < n; g0 += 64 * kVerifyBatch) {
    int32_t id[kVerifyBatch];
    float xt[kVerifyBatch], xd[kVerifyBatch];
    residual_batch<DT>(r, q0, queue, n, g0, lane, use_res, id, xt, xd);
#pragma unroll
    for (int b = 0; b < kVerifyBatch; ++b) {
      uint64_t wt = 0ull, wr = 0ull;
      if (id[b] >= 0) residual_weights(r, xt[b], xd[b], id[b], use_res, wt, wr);
      const uint64_t w = use_res ? wr : wt;
      const uint64_t incl = wave_incl_scan(w);
      const uint64_t before = cum + incl - w;
      if (w && before <= t && t < before + w) found = id[b];
      cum += read_lane(incl, 63);
    }
  }
  const uint64_t hm = __ballot(found >= 0);
  return hm ? read_lane(found, __builtin_ctzll(hm)) : -1;
}

// Rows were sampled into ws.v* by launch_sample: target (s, j) at row s*W + j,
// draft (s, j) at row S*W + s*(W-1) + j; each row's draw used uniform [s, j]
// and probed draft token [s, j].  Grid: (parts, sequences).  Part 0 of a
// sequence writes its outcome; in RESIDUAL mode, a sequence with a rejected
// position draws from the residual there with all its parts: each part sums
// both weights over each wave's kVerifySpan tokens and publishes the eight
// spans' sums, and the last part to arrive picks the span whose run holds the
// draw, walks that span again with one wave and writes the token.
template <int DT>
__global__ __launch_bounds__(kThreads) void k_verify_finish(Workspace ws, VerifyPlan Q) {
  __shared__ Candidate s_ct[kVerifyCandLds];
  __shared__ Candidate s_cd[kVerifyCandLds];
  __shared__ uint16_t s_queue[kWaves][kVerifySpan];
  __shared__ uint64_t s_wt[kWaves], s_wr[kWaves];
  __shared__ int32_t s_rej, s_last;
  const int part = blockIdx.x, s = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int W = Q.window, D = W - 1, S = Q.sequences;
  const int32_t V = Q.vocab;
  int32_t* tok = Q.tokens + (size_t)s * W;
  const int32_t* drafts = Q.draft_tokens + (size_t)s * D;
  const float* u = Q.uniforms + (size_t)s * W;
  uint8_t* am = Q.accept_mask ? Q.accept_mask + (size_t)s * D : nullptr;
  constexpr uint32_t kBad = LSAMP_ROW_OVERFLOW | LSAMP_ROW_TIMEOUT;
  if (Q.mode == LSAMP_VERIFY_RESIDUAL) {
    // wave 0, a position per lane: accept j iff u_j * p_d < p_t (p_d = 0:
    // iff p_t > 0); a row whose keep set could not be resolved fails the
    // whole window
    if (tid < 64) {
      bool failed = false;
      int jr = D;  // the first rejected position (D: every draft accepted)
      for (int j0 = 0; j0 < W; j0 += 64) {
        const int jj = j0 + lane;
        bool bad = false, rej = false;
        if (jj < W) bad = (ws.vflags[s * W + jj] & kBad) != 0u;
        if (jj < D) {
          bad = bad || (ws.vflags[S * W + s * D + jj] & kBad) != 0u;
          const lsamp_row_stats& st = ws.vstats[s * W + jj];
          const lsamp_row_stats& sd = ws.vstats[S * W + s * D + jj];
          const double pt = st.kept_weight ? (double)st.probe_weight / (double)st.kept_weight : 0.0;
          const double pd = sd.kept_weight ? (double)sd.probe_weight / (double)sd.kept_weight : 0.0;
          rej = !(pd > 0.0 ? ((double)u[jj] < pt / pd) : (pt > 0.0));
        }
        failed = failed || __ballot(bad) != 0ull;
        const uint64_t rm = __ballot(rej);
        if (rm && jr == D) jr = j0 + __builtin_ctzll(rm);
      }
      if (part == 0) {
        for (int j0 = 0; j0 < W; j0 += 64) {
          const int jj = j0 + lane;
          // (the rejected position's token is the residual draw's)
          if (jj < W && (failed || jj != jr || jr == D))
            tok[jj] = failed     ? -1
                      : jj < jr  ? drafts[jj]
                      : jj == jr ? ws.vtokens[s * W + D]  // (jr == D here: the bonus)
                                 : -1;
          if (am && jj < D) am[jj] = !failed && jj < jr ? 1 : 0;
        }
        if (lane == 0) Q.accepted[s] = failed ? 0 : jr;
      }
      if (lane == 0) s_rej = failed || jr == D ? -1 : jr;
    }
  } else if (tid == 0) {
    s_rej = -1;
    if (part == 0) {
      const lsamp_row_params prm = Q.params[s];
      const bool greedy = make_ctx(Q.semantics, prm).kind == LSAMP_KIND_ARGMAX;
      // greedy rows, and rows with a presence or frequency penalty when the
      // penalties are applied, accept exactly (DefaultSamplerV2.swift:496-502,
      // CBv2MTPVerifyPenalties.applies, EngineLoopV2.swift:241-243)
      const bool exact_row = greedy || (Q.penalized && (prm.presence_penalty != 0.0f ||
                                                        prm.frequency_penalty != 0.0f));
      bool failed = false;  // a row whose keep set could not be resolved
      for (int j = 0; j < W; ++j) {
        tok[j] = -1;
        if (ws.vflags[s * W + j] & kBad) failed = true;
      }
      if (am)
        for (int j = 0; j < D; ++j) am[j] = 0;
      if (failed) {
        Q.accepted[s] = 0;
      } else {
        int prefix = 0;
        bool still = true;
        for (int j = 0; j < W; ++j) {
          tok[j] = ws.vtokens[s * W + j];
          if (j >= D) continue;
          bool accept;
          if (Q.mode == LSAMP_VERIFY_EXACT || exact_row) {
            accept = tok[j] == drafts[j];
          } else {
            // p(draft) > min(1, delta * e^-H) on the filtered, tempered row
            const lsamp_row_stats& st = ws.vstats[s * W + j];
            const double p =
                st.kept_weight ? (double)st.probe_weight / (double)st.kept_weight : 0.0;
            const double fl = fmin(1.0, (double)Q.typical_delta * exp(-(double)st.kept_entropy));
            accept = p > fl;
          }
          if (am) am[j] = accept ? 1 : 0;
          if (still && accept)
            ++prefix;
          else
            still = false;
        }
        Q.accepted[s] = prefix;
      }
    }
  }
  __syncthreads();
  const int j = s_rej;
  if (j < 0) return;

  // residual draw at the first rejected position: normalize(max(0, p_t - p_d))
  // with both distributions quantized to 2^-52, by inverse CDF in id order
  // with uniform [s, W-1]; an empty residual draws from the target row itself
  const lsamp_row_params prm = Q.params[s];
  ResidualRows r;
  r.c = make_ctx(Q.semantics, prm);
  const int rt = s * W + j, rd = S * W + s * D + j;
  const RowInfo it = ws.rows[rt], id = ws.rows[rd];
  r.qt = make_rule(it, r.c);
  r.qd = make_rule(id, r.c);
  r.nct = it.kept_cands;
  r.ncd = id.kept_cands;
  {
    const Candidate* ct = ws.cands + (size_t)rt * kCandCap;
    const Candidate* cd = ws.cands + (size_t)rd * kCandCap;
    r.ct = ct;
    r.cd = cd;
    if (r.nct <= kVerifyCandLds) {
      for (int i = tid; i < r.nct; i += kThreads) s_ct[i] = ct[i];
      r.ct = s_ct;
    }
    if (r.ncd <= kVerifyCandLds) {
      for (int i = tid; i < r.ncd; i += kThreads) s_cd[i] = cd[i];
      r.cd = s_cd;
    }
  }
  r.ymt = it.mode == kModePosInf ? kPosInf : to_filter(r.c, it.x_max);
  r.ymd = id.mode == kModePosInf ? kPosInf : to_filter(r.c, id.x_max);
  r.Wt = ws.vstats[rt].kept_weight;
  r.Wd = ws.vstats[rd].kept_weight;
  const size_t es = DT == LSAMP_DTYPE_F32 ? 4 : 2;
  r.trow = reinterpret_cast<const char*>(Q.target) + (size_t)rt * V * es;
  r.drow = reinterpret_cast<const char*>(Q.draft) + (size_t)(s * D + j) * V * es;
  r.V = V;
  r.vec = aligned16(r.trow);
  __syncthreads();
  uint16_t* queue = s_queue[wv];
  const int P = Q.parts;
  {
    const int32_t q0 = part * kVerifyPart + wv * kVerifySpan;
    const int n = residual_screen<DT>(r, q0, queue, lane);
    uint64_t st, sr;
    residual_sums<DT>(r, q0, queue, n, lane, true, st, sr);
    st = wave_sum(st);
    sr = wave_sum(sr);
    if (lane == 0) {
      s_wt[wv] = st;
      s_wr[wv] = sr;
    }
  }
  __syncthreads();
  // publish the wave spans' sums (wave 0 stores them all, so that its own
  // wait covers every store), then take the sequence's ticket
  if (tid < 64) {
    VerifySpan* vs = ws.vspan + ((size_t)s * ws.max_parts + part) * kWaves;
    if (lane < kWaves) {
      st_coherent(&vs[lane].res, s_wr[lane]);
      st_coherent(&vs[lane].tgt, s_wt[lane]);
    }
    drain_memory();
    if (lane == 0) {
      const uint32_t t =
          __hip_atomic_fetch_add(&ws.vticket[s], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = t + 1u == (uint32_t)P;
      if (last) st_coherent(&ws.vticket[s], 0u);
      s_last = last ? 1 : 0;
    }
  }
  __syncthreads();
  if (!s_last || wv != 0) return;

  // the last part, wave 0: the draw's kind and target from every span's sums
  // (span e covers tokens from e * kVerifySpan, so the spans run in id
  // order), then the token inside the span whose run holds the target
  constexpr int kE = (kMaxVerifySpans + 63) / 64;
  const VerifySpan* vs = ws.vspan + (size_t)s * ws.max_parts * kWaves;
  const int E = P * kWaves;
  uint64_t vr[kE], vt[kE];
#pragma unroll
  for (int k = 0; k < kE; ++k) {
    const int e = k * 64 + lane;
    vr[k] = e < E ? ld_coherent(&vs[e].res) : 0ull;
    vt[k] = e < E ? ld_coherent(&vs[e].tgt) : 0ull;
  }
  uint64_t R = 0ull, T = 0ull;
#pragma unroll
  for (int k = 0; k < kE; ++k) {
    R += vr[k];
    T += vt[k];
  }
  R = wave_sum(R);
  T = wave_sum(T);
  const bool use_res = R != 0ull;
  const uint64_t tot = use_res ? R : T;
  int32_t f = -1;
  if (tot) {
    const uint64_t target = scaled_target(uniform_u32(u[D]), tot);
    uint64_t cum = 0ull, rel = 0ull;
    int es = -1;
#pragma unroll
    for (int k = 0; k < kE; ++k) {
      if (k * 64 >= E) break;
      const uint64_t v = use_res ? vr[k] : vt[k];
      const uint64_t incl = wave_incl_scan(v);
      const uint64_t before = cum + incl - v;
      const uint64_t hm = __ballot(v && before <= target && target < before + v);
      if (hm && es < 0) {
        const int hl = __builtin_ctzll(hm);
        es = k * 64 + hl;
        rel = target - read_lane(before, hl);
      }
      cum += read_lane(incl, 63);
    }
    if (es >= 0) {
      const int32_t q0 = es * kVerifySpan;
      const int n = residual_screen<DT>(r, q0, s_queue[0], lane);
      f = residual_find<DT>(r, q0, s_queue[0], n, lane, use_res, rel);
    }
  }
  if (lane == 0) tok[j] = f;
}

template <int DT>
int launch_verify_dt(const Workspace& ws, const VerifyPlan& Q, hipStream_t st) {
  hipLaunchKernelGGL(k_verify_finish<DT>, dim3((unsigned)Q.parts, (unsigned)Q.sequences),
                     dim3(kThreads), 0, st, ws, Q);
  return (int)hipGetLastError();
}

}  // namespace

int launch_verify_finish(const Workspace& ws, const VerifyPlan& Q, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (Q.dtype) {
    case LSAMP_DTYPE_F32: return launch_verify_dt<LSAMP_DTYPE_F32>(ws, Q, st);
    case LSAMP_DTYPE_BF16: return launch_verify_dt<LSAMP_DTYPE_BF16>(ws, Q, st);
    default: return launch_verify_dt<LSAMP_DTYPE_F16>(ws, Q, st);
  }
}

int launch_sample(const Workspace& ws, const SamplePlan& P, const FusedLp* lp, void* stream,
                  void* const* events) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (P.dtype) {
    case LSAMP_DTYPE_F32: return launch_dt<LSAMP_DTYPE_F32>(ws, P, lp, st, events);
    case LSAMP_DTYPE_BF16: return launch_dt<LSAMP_DTYPE_BF16>(ws, P, lp, st, events);
    default: return launch_dt<LSAMP_DTYPE_F16>(ws, P, lp, st, events);
  }
}

int set_spin_test(int32_t polls) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_spin_test), &polls, sizeof polls, 0,
                                hipMemcpyHostToDevice);
}

// Work-groups per CU of the fused kernel: the smaller occupancy of its two
// instantiations (one round / several rounds), since a launch may use either
// and the grid is sized from this value.
template <int DT>
int fused_blocks_dt() {
  int a = 0, b = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, k_fused<DT, true, false>, kThreads, 0) != hipSuccess)
    return 0;
  if constexpr (DT == LSAMP_DTYPE_F32) {
    return a;  // (one round only)
  } else {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k_fused<DT, false, false>, kThreads, 0) !=
        hipSuccess)
      return 0;
    return a < b ? a : b;
  }
}

int fused_blocks_per_cu(int dtype) {
  switch (dtype) {
    case LSAMP_DTYPE_F32: return fused_blocks_dt<LSAMP_DTYPE_F32>();
    case LSAMP_DTYPE_BF16: return fused_blocks_dt<LSAMP_DTYPE_BF16>();
    default: return fused_blocks_dt<LSAMP_DTYPE_F16>();
  }
}

}  // namespace lsamp
