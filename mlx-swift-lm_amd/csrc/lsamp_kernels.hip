// lsamp_kernels.hip — gfx950 kernels of the logits-to-token stage.
//
// A sampling step runs over tasks (row, slice): one 512-thread work-group
// owns one slice (<= 40960 tokens) of one row and keeps the slice's logits in
// registers from the moment they arrive from HBM until the token is drawn.
//
//  stats phase   16-byte vector loads of the slice, the grammar mask and the
//                sparse penalties applied exactly as the reference orders
//                them, then a histogram of the filter-space logit in 1/32-nat
//                bins (count + fixed-point mass, one packed 64-bit LDS atomic
//                per token).  The last work-group of the row merges the
//                slices' histograms and locates the bin holding the
//                top-k / top-p / min-p cut.
//  select phase  every work-group keeps the tokens above the cut bin (fixed-
//                point draw weight per 1024-token chunk, and a short list of
//                them) and lists the tokens inside it.  The last work-group of
//                the row sorts those candidates, applies the exact keep rule of
//                the row's semantics and draws the token by inverse CDF in
//                token-id order.
//
// Fused mode runs both phases in one kernel whose grid fits on the device at
// once: the slices of a row wait for the merge on a bounded spin (a wait that
// runs out sets a status bit and the work-group carries on, so the grid always
// drains).  Split mode runs the phases as two kernels, the second re-reading
// its slice from L2; it needs no co-residency.  Neither mode uses MFMA: the
// stage is a bandwidth- and reduction-bound pass, not a contraction.
#include <hip/hip_runtime.h>

#include "lsamp_device.h"
#include "lsamp_internal.h"

namespace lsamp {
namespace {

using namespace dev;

constexpr int kSliceWords = kMaxSliceLen / 32;       // penalty bitmap words
constexpr int kFinalPerThread = kCandCap / kThreads;  // sorted candidates per thread
constexpr uint32_t kReady = 1u << 16;                 // merge-done bias on arrive_stats
constexpr int kSpinLimit = 1 << 20;                   // ~0.2 s of polling

enum TaskMode { kFused = 0, kStatsOnly = 1, kSelectOnly = 2 };

// ------------------------------------------------------------ row context
struct RowCtx {
  int32_t sem;
  int32_t kind;
  float T;        // temperature dividing the filter space (CBv2 sampled rows)
  bool tempered;  // filter space is x / T
  float c32;      // histogram scale: bin = floor(x * c32)
  float scale;    // draw scale (mlx-lm: fl(1 / T))
};

__device__ __forceinline__ RowCtx make_ctx(int32_t sem, const lsamp_row_params& p) {
  RowCtx c;
  c.sem = sem;
  c.kind = p.kind;
  // Rows whose temperature cannot define a distribution fall back to argmax.
  if (c.kind != LSAMP_KIND_ARGMAX && !(p.temperature > 0.0f && p.temperature < kPosInf))
    c.kind = LSAMP_KIND_ARGMAX;
  c.T = 1.0f;
  c.tempered = false;
  c.scale = 1.0f;
  if (c.kind != LSAMP_KIND_ARGMAX) {
    if (sem == LSAMP_SEM_CBV2) {
      c.T = p.temperature;
      c.tempered = p.temperature != 1.0f;
    } else {
      c.scale = 1.0f / p.temperature;
    }
  }
  c.c32 = c.tempered ? 32.0f / c.T : 32.0f;
  return c;
}

// Filter-space value of a transformed logit (LogitsPipelineV2.swift:333-335).
__device__ __forceinline__ float to_filter(const RowCtx& c, float x) {
  return c.tempered ? x / c.T : x;
}

// Transformed value of a penalized / biased token, in the reference's order.
__device__ __forceinline__ float patch_value(const RowCtx& c, const lsamp_row_params& p,
                                             float x, const lsamp_penalty_entry& e, int dt) {
  if (c.sem == LSAMP_SEM_CBV2) {
    // LogitsPipelineV2.process (1) bias, (2) repetition, frequency, presence
    // (LogitsPipelineV2.swift:317-330), each a separately rounded fp32 op.
    if (e.bias != 0.0f) x = x + e.bias;
    if (p.repetition_penalty != 1.0f && (e.flags & LSAMP_PEN_REPETITION)) {
      const float rp = p.repetition_penalty;
      x = x > 0.0f ? x / rp : x * rp;
    }
    if ((p.frequency_penalty != 0.0f || p.presence_penalty != 0.0f) && e.count > 0) {
      const float fc = p.frequency_penalty * (float)e.count;
      x = x - fc;
      const float pm = p.presence_penalty * 1.0f;
      x = x - pm;
    }
  } else {
    // RepetitionContext / PresencePenaltyContext in the logits dtype,
    // FrequencyPenaltyContext promoting to float32 (Evaluate.swift:586-658).
    if (p.repetition_penalty != 1.0f && (e.flags & LSAMP_PEN_REPETITION)) {
      const float rp = round_dtype(p.repetition_penalty, dt);
      x = round_dtype(x < 0.0f ? x * rp : x / rp, dt);
    }
    if (p.presence_penalty != 0.0f && (e.flags & LSAMP_PEN_PRESENCE)) {
      x = round_dtype(x - round_dtype(p.presence_penalty, dt), dt);
    }
    if (p.frequency_penalty != 0.0f && e.count > 0) {
      const float h = (float)e.count * p.frequency_penalty;
      x = x - h;
    }
  }
  return x;
}

// Allowed bits (1 = allowed) of the N tokens starting at i0, N <= 32 and i0 a
// multiple of N with N a power of two, so the N bits lie in one mask word.
// Tokens at or past mask_bits, or in words past mask_words, follow `tail`.
__device__ __forceinline__ uint32_t mask_allow_bits(const uint32_t* mrow, int32_t mask_words,
                                                    int32_t mask_bits, int32_t tail, int32_t i0,
                                                    int N) {
  const uint32_t full = (N == 32) ? 0xffffffffu : ((1u << N) - 1u);
  if (!mrow) return full;
  const int32_t wi = i0 >> 5;
  const bool word_in = wi < mask_words;
  const uint32_t word = word_in ? mrow[wi] : 0u;
  int32_t nin = word_in ? mask_bits - i0 : 0;  // leading positions the mask covers
  nin = nin < 0 ? 0 : (nin > N ? N : nin);
  const uint32_t in_mask = nin >= 32 ? 0xffffffffu : ((1u << nin) - 1u);
  const uint32_t bits = (word >> (uint32_t)(i0 & 31)) & in_mask;
  return (bits | (tail == LSAMP_MASK_TAIL_KEEP ? (full & ~in_mask) : 0u)) & full;
}

__device__ __forceinline__ bool mask_allows(const uint32_t* mrow, int32_t mask_words,
                                            int32_t mask_bits, int32_t tail, int32_t i) {
  return mask_allow_bits(mrow, mask_words, mask_bits, tail, i, 1) != 0u;
}

__device__ __forceinline__ const char* row_base(const SamplePlan& P, int row) {
  const size_t es = P.dtype == LSAMP_DTYPE_F32 ? 4 : 2;
  if (row < P.rows_split)
    return reinterpret_cast<const char*>(P.logits) + (size_t)row * (size_t)P.row_stride * es;
  return reinterpret_cast<const char*>(P.logits2) +
         (size_t)(row - P.rows_split) * (size_t)P.row_stride * es;
}

__device__ __forceinline__ float load_logit(int dt, const char* rowp, int64_t i) {
  if (dt == LSAMP_DTYPE_F32) return load_scalar<LSAMP_DTYPE_F32>(rowp, i);
  if (dt == LSAMP_DTYPE_BF16) return load_scalar<LSAMP_DTYPE_BF16>(rowp, i);
  return load_scalar<LSAMP_DTYPE_F16>(rowp, i);
}

// The thread index through an empty asm statement: values derived from it
// cannot be hoisted out of the fused kernel's loop over rounds (where they
// would stay live, and spill, across the whole task).
__device__ __forceinline__ int fresh_tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

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
};

__device__ __forceinline__ ClassRule make_rule(const RowInfo& info, const RowCtx& c) {
  ClassRule r;
  r.top = info.top_bin;
  r.c32 = c.c32;
  r.posinf = info.mode == kModePosInf;
  if (info.mode != kModeNormal) {
    r.kc = r.kd = -1;
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
  if (r.posinf) return x == kPosInf ? kKept : kDrop;
  if (!__builtin_isfinite(x)) return kDrop;
  int j = r.top - bin_of(x, r.c32);
  j = j < 0 ? 0 : j;
  return j < r.kc ? kKept : (j < r.kd ? kCand : kDrop);
}

// Penalty bitmap of the slice + the slice's entries, patched.  Shared by both
// kernels (they must classify identically).
struct SliceEntries {
  uint32_t* pen;   // [kSliceWords]
  int32_t* tok;    // [kSliceEntryCap]
  float* x;        // [kSliceEntryCap] transformed, -inf when masked / NaN
  int32_t* count;  // LDS counter
};

template <int DT>
__device__ __forceinline__ int build_slice_entries(const SamplePlan& P, const RowCtx& c,
                                                   const lsamp_row_params& prm, int row,
                                                   const char* rowp, int64_t base, int64_t end,
                                                   SliceEntries& se, bool* overflow) {
  const int tid = threadIdx.x;
  for (int i = tid; i < kSliceWords; i += kThreads) se.pen[i] = 0u;
  if (tid == 0) *se.count = 0;
  __syncthreads();
  int32_t e0 = 0, e1 = 0;
  if (P.row_ptr && P.entries) {
    e0 = P.row_ptr[row];
    e1 = P.row_ptr[row + 1];
  }
  for (int32_t e = e0 + tid; e < e1; e += kThreads) {
    const int32_t t = P.entries[e].token;
    if (t >= base && t < end) {
      const int32_t li = (int32_t)(t - base);
      atomicOr(&se.pen[li >> 5], 1u << (li & 31));
      const int idx = atomicAdd(se.count, 1);
      if (idx < kSliceEntryCap) se.tok[idx] = e;
    }
  }
  __syncthreads();
  const int n_all = *se.count;
  const int n = n_all < kSliceEntryCap ? n_all : kSliceEntryCap;
  *overflow = n_all > kSliceEntryCap;
  const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * (size_t)P.mask_words : nullptr;
  for (int j = tid; j < n; j += kThreads) {
    const lsamp_penalty_entry ent = P.entries[se.tok[j]];
    float x = load_scalar<DT>(rowp, ent.token);
    x = patch_value(c, prm, x, ent, DT);
    if (!mask_allows(mrow, P.mask_words, P.mask_bits, P.mask_tail, ent.token)) x = kNegInf;
    if (x != x) x = kNegInf;
    se.x[j] = x;
    se.tok[j] = ent.token;
  }
  __syncthreads();
  return n;
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
  uint64_t dw[kChunk];
  int32_t did[kChunk];
  float cx[kChunk];
  uint8_t cent[kChunk];
  uint8_t cflag[kChunk];
};
union PhaseLds {
  uint64_t hist[kHist];
  MergeLds m;
  SelectLds s;
  FinalLds f;
};
struct TaskLds {
  PhaseLds u;
  uint32_t pen[kSliceWords];
  int32_t etok[kSliceEntryCap];
  float ex[kSliceEntryCap];
  RowInfo info;
  SelectPartial part[kMaxSlices];
  float hx[kMaxSlices];
  int32_t htop[kMaxSlices];
  uint32_t hfl[kMaxSlices];
  int32_t hn[kMaxSlices];
  float redf[kWaves];
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
  uint32_t flags;
};

// Wave-aggregated append to an LDS list: returns this lane's slot or -1.
__device__ __forceinline__ int wave_append(bool pred, int32_t* counter) {
  const uint64_t m = __ballot(pred);
  if (m == 0ull) return -1;
  const int lane = threadIdx.x & 63;
  const int leader = __ffsll((unsigned long long)m) - 1;
  int b = 0;
  if (lane == leader) b = atomicAdd(counter, (int)__popcll(m));
  b = __shfl(b, leader, 64);
  return pred ? b + (int)__popcll(m & ((1ull << lane) - 1ull)) : -1;
}

__device__ __forceinline__ int32_t key_id(uint64_t key) {
  return (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
}
__device__ __forceinline__ float key_y(uint64_t key) { return key_to_float((uint32_t)(key >> 32)); }

// Transformed value of one token read on its own (chunk scan, probe).
template <int DT>
__device__ __forceinline__ float token_value(const SamplePlan& P, const RowCtx& c, const lsamp_row_params& prm,
                             int row, const char* rowp, const uint32_t* mrow, int64_t i,
                             const float* patched, const uint8_t* has_patch) {
  float x;
  if (has_patch && has_patch[0]) {
    x = patched[0];
  } else {
    x = load_scalar<DT>(rowp, i);
    if (!mask_allows(mrow, P.mask_words, P.mask_bits, P.mask_tail, i)) x = kNegInf;
  }
  if (x != x) x = kNegInf;
  return x;
}

// ============================================================ merge (stats)
// Last stats work-group of a row: merges the G slice histograms (integer
// sums on the absolute bin grid) and locates the cut bin.  Result in L.info.
__device__ __forceinline__ void merge_row(const Workspace& ws, const SamplePlan& P, int row, const RowCtx& c,
                          const lsamp_row_params& prm, TaskLds& L) {
  const int tid = threadIdx.x;
  const int G = P.slices;
  const int64_t V = P.vocab;
  const SliceSummary* summ = ws.summaries + (size_t)row * kMaxSlices;
  if (tid < G) {
    L.hx[tid] = ld_coherent(&summ[tid].x_max);
    L.htop[tid] = ld_coherent(&summ[tid].top_bin);
    L.hfl[tid] = ld_coherent(&summ[tid].flags);
    L.hn[tid] = ld_coherent(&summ[tid].n_finite);
  }
  const uint64_t wtail = tid < G ? ld_coherent(&summ[tid].hist[kTail]) : 0ull;
  L.u.m.mass[2 * tid] = 0ull;
  L.u.m.mass[2 * tid + 1] = 0ull;
  L.u.m.cnt[2 * tid] = 0u;
  L.u.m.cnt[2 * tid + 1] = 0u;
  __syncthreads();
  float row_max = kNegInf;
  int32_t row_top = 0, n_total = 0;
  uint32_t rflags = 0u;
  bool first = true;
  for (int s = 0; s < G; ++s) {
    rflags |= L.hfl[s];
    n_total += L.hn[s];
    if (L.hn[s] > 0) {
      if (first || L.hx[s] > row_max) row_max = L.hx[s];
      if (first || L.htop[s] > row_top) row_top = L.htop[s];
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
  info.pad = 0;
  const float s_top = bin_pos(row_max, c.c32);
  info.q_top = s_top * (1.0f / 32.0f);

  if (info.mode == kModeNormal && c.kind == LSAMP_KIND_ARGMAX) {
    info.cut = 0;
    info.count_above = 0;
  } else if (info.mode == kModeNormal) {
    const double inv_frac = 1.0 / (double)(1ull << kMassFracBits);
    int32_t tcnt = 0;
    double tmass = 0.0;
    // slice-local bin i of slice s is row bin i + (row_top - top_s); the
    // slices are read four at a time (eight independent loads per thread)
    for (int s0 = 0; s0 < G; s0 += 4) {
      uint64_t w[4][2];
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int u = 0; u < 2; ++u)
          w[d][u] = (s0 + d < G && L.hn[s0 + d] > 0) ? ld_coherent(&summ[s0 + d].hist[2 * tid + u])
                                                     : 0ull;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          if (w[d][u] == 0ull) continue;
          const int s = s0 + d;
          const int i = 2 * tid + u;
          const int j = i + (row_top - L.htop[s]);
          const uint32_t wc = (uint32_t)(w[d][u] >> kCountShift);
          const uint64_t wm = w[d][u] & kMassMask;
          if (j < kBins) {
            atomicAdd(&L.u.m.cnt[j], wc);
            atomicAdd(reinterpret_cast<unsigned long long*>(&L.u.m.mass[j]), (unsigned long long)wm);
          } else {
            const int b = L.htop[s] - i;  // absolute bin
            tcnt += (int32_t)wc;
            tmass += (double)wm * inv_frac * exp(((double)b - (double)s_top) / 32.0);
          }
        }
      }
    }
    if (tid < G && L.hn[tid] > 0 && wtail) {
      const double edge = (double)(L.htop[tid] - kBins + 1);
      tcnt += (int32_t)(wtail >> kCountShift);
      tmass += (double)(wtail & kMassMask) * inv_frac * exp((edge - (double)s_top) / 32.0);
    }
    __syncthreads();
    int32_t cnt[2];
    double mass[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = 2 * tid + u;
      cnt[u] = (int32_t)L.u.m.cnt[j];
      mass[u] = cnt[u] ? (double)L.u.m.mass[j] * inv_frac *
                             exp(((double)(row_top - j) - (double)s_top) / 32.0)
                       : 0.0;
    }
    tcnt = block_sum(tcnt, L.redi);
    tmass = block_sum(tmass, L.redd);
    int32_t tot_cnt = 0;
    double tot_mass = 0.0;
    const int32_t excl_cnt = block_excl_scan(cnt[0] + cnt[1], L.redi, &tot_cnt);
    const double excl_mass = block_excl_scan(mass[0] + mass[1], L.redd, &tot_mass);
    const double z = tot_mass + tmass;
    info.z = z;

    const int32_t k_lim = (prm.top_k > 0 && (int64_t)prm.top_k < V) ? prm.top_k : 0;
    bool p_on;
    double P_lim;
    bool strict;  // CBv2 keeps exclusive mass <= P; mlx-lm keeps mass-before < P
    if (P.semantics == LSAMP_SEM_CBV2) {
      p_on = prm.top_p < 1.0f;
      P_lim = (double)(prm.top_p > 0.0f ? prm.top_p : 0.0f) * z;
      strict = false;
    } else {
      p_on = prm.top_p > 0.0f && prm.top_p < 1.0f;
      P_lim = (double)prm.top_p * z;
      strict = true;
    }
    if (c.kind != LSAMP_KIND_FILTERED) p_on = false;
    const bool k_on = c.kind == LSAMP_KIND_FILTERED && k_lim > 0;
    const float mp = prm.min_p > 1.0f ? 1.0f : prm.min_p;
    const bool m_on = c.kind == LSAMP_KIND_FILTERED && mp > 0.0f;
    int32_t j_t = kBins + 1;
    if (m_on) {
      const float st = s_top + 32.0f * __builtin_logf(mp);
      j_t = row_top - (int32_t)__builtin_floorf(__builtin_fmaxf(st, -1.0e9f));
      if (j_t < 0) j_t = 0;
      if (j_t > kBins) j_t = kBins;
    }
    info.p_limit = p_on ? P_lim : -1.0;
    int my_cut = 0x7fffffff;
    int32_t C = excl_cnt;
    double M = excl_mass;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = 2 * tid + u;
      if (cnt[u] > 0 || (m_on && j == j_t)) {
        const bool tk = k_on && C + cnt[u] >= k_lim;
        const bool tp = p_on && cnt[u] > 0 &&
                        (strict ? (M + mass[u] >= P_lim) : (M + mass[u] > P_lim));
        const bool tm = m_on && j >= j_t;
        if ((tk || tp || tm) && j < my_cut) my_cut = j;
      }
      C += cnt[u];
      M += mass[u];
    }
    const int cut = block_min(my_cut, L.redi);
    if (cut != 0x7fffffff) {
      if (cut / 2 == tid) {
        L.misc[0] = excl_cnt + ((cut & 1) ? cnt[0] : 0);
        L.misc64[0] = __builtin_bit_cast(uint64_t, excl_mass + ((cut & 1) ? mass[0] : 0.0));
      }
      __syncthreads();
      info.cut = cut;
      info.count_above = L.misc[0];
      info.mass_above = __builtin_bit_cast(double, L.misc64[0]);
    } else {
      const bool tk = k_on && tot_cnt + tcnt >= k_lim;
      const bool tp = p_on && tcnt > 0 && (strict ? (z >= P_lim) : (z > P_lim));
      const bool tm = m_on && j_t >= kBins;
      if (tk || tp || tm) {
        info.cut = kCutTail;
        info.count_above = tot_cnt;
        info.mass_above = tot_mass;
      } else {
        info.cut = kCutNone;
        info.count_above = n_total;
        info.mass_above = z;
      }
    }
  }
  __syncthreads();
  if (tid == 0) L.info = info;
  __syncthreads();
}

__device__ __forceinline__ void publish_rowinfo(RowInfo* dst, const RowInfo& v) {
  st_coherent_f32(&dst->x_max, v.x_max);
  st_coherent_f32(&dst->q_top, v.q_top);
  st_coherent(&dst->top_bin, v.top_bin);
  st_coherent(&dst->cut, v.cut);
  st_coherent(&dst->mode, v.mode);
  st_coherent(&dst->flags, v.flags);
  st_coherent(&dst->count_above, v.count_above);
  st_coherent(&dst->n_finite, v.n_finite);
  st_coherent_f64(&dst->mass_above, v.mass_above);
  st_coherent_f64(&dst->z, v.z);
  st_coherent_f64(&dst->p_limit, v.p_limit);
  st_coherent(&dst->kept_cands, v.kept_cands);
}

__device__ __forceinline__ RowInfo read_rowinfo(const RowInfo* src) {
  RowInfo v;
  v.x_max = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&src->x_max)));
  v.q_top = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&src->q_top)));
  v.top_bin = ld_coherent(&src->top_bin);
  v.cut = ld_coherent(&src->cut);
  v.mode = ld_coherent(&src->mode);
  v.flags = ld_coherent(&src->flags);
  v.count_above = ld_coherent(&src->count_above);
  v.n_finite = ld_coherent(&src->n_finite);
  v.mass_above = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&src->mass_above)));
  v.z = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&src->z)));
  v.p_limit = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&src->p_limit)));
  v.kept_cands = ld_coherent(&src->kept_cands);
  v.pad = 0;
  return v;
}

// ========================================================= finalize (select)
// Last select work-group of a row: exact cut among the candidates, kept
// weights per chunk, and the inverse-CDF draw.
template <int DT>
__device__ __forceinline__ void finalize_row(const Workspace& ws, const SamplePlan& P, int row, const RowCtx& c,
                             const lsamp_row_params& prm, const RowInfo& info, TaskLds& L,
                             const char* rowp, const uint32_t* mrow, bool fused) {
  const int tid = threadIdx.x;
  const int G = P.slices;
  const int64_t V = P.vocab;
  const int nch_row = P.nchunks;
  const float y_max = info.mode == kModePosInf ? kPosInf : to_filter(c, info.x_max);
  const bool active = info.mode != kModeEmpty;
  uint64_t* rowchunks = ws.chunk_w + (size_t)row * (size_t)ws.max_chunks;
  Candidate* rc = ws.cands + (size_t)row * kCandCap;
  FinalLds& F = L.u.f;

  // ---- every independent load first
  if (tid < G) {
    const SelectPartial* sp = ws.partials + (size_t)row * kMaxSlices + tid;
    SelectPartial v;
    v.ent = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&sp->ent)));
    v.min_kept = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&sp->min_kept)));
    v.n_kept = ld_coherent(&sp->n_kept);
    v.n_cand = ld_coherent(&sp->n_cand);
    v.n_list = ld_coherent(&sp->n_list);
    v.overflow = ld_coherent(&sp->overflow);
    v.pad = 0;
    L.part[tid] = v;
  }
  F.rowchunk[tid] = tid < nch_row ? ld_coherent(&rowchunks[tid]) : 0ull;
  if (tid == 0) {
    L.misc[0] = (int32_t)ld_coherent(&ws.cand_count[row]);
    float u = 0.0f;
    if (P.uniforms)
      u = P.uniforms[row];
    else if (P.philox_keys)
      u = philox_uniform(P.philox_keys[row], 0u);
    L.misc64[1] = (uint64_t)__float_as_uint(u);
    L.misc[1] = P.probe_tokens ? P.probe_tokens[row] : -1;
  }
  __syncthreads();
  double ent_all = 0.0;
  float min_all = kPosInf;
  int32_t kept_all = 0;
  bool overflow = (info.flags & LSAMP_ROW_OVERFLOW) != 0;
  for (int s = 0; s < G; ++s) {
    ent_all += L.part[s].ent;
    min_all = __builtin_fminf(min_all, L.part[s].min_kept);
    kept_all += L.part[s].n_kept;
    if (L.part[s].n_cand > kWgCandCap || L.part[s].overflow) overflow = true;
  }
  const int total_cand = L.misc[0];
  if (total_cand > kCandCap) overflow = true;
  const float u_draw = __uint_as_float((uint32_t)L.misc64[1]);
  const int32_t probe = L.misc[1];
  const int nc = (overflow || !active) ? 0 : total_cand;

  // ---- sort candidates: value descending, id ascending (-0 == +0)
  int n2 = 1;
  while (n2 < nc) n2 <<= 1;
  for (int i = tid; i < n2; i += kThreads) {
    uint64_t key = 0ull;
    if (i < nc) {
      const float y = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&rc[i].y)));
      const int32_t id = ld_coherent(&rc[i].id);
      key = ((uint64_t)ordered_key(y == 0.0f ? 0.0f : y) << 32) |
            (uint64_t)(0xffffffffu - (uint32_t)id);
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

  // ---- keep rule over the sorted candidates (thread t owns a contiguous run)
  const int per = (n2 + kThreads - 1) / kThreads;  // <= kFinalPerThread
  const int r0 = tid * per;
  const double P_lim = info.p_limit;
  const bool p_on = P_lim >= 0.0;
  const int32_t k_lim = (c.kind == LSAMP_KIND_FILTERED && prm.top_k > 0 && (int64_t)prm.top_k < V)
                            ? prm.top_k
                            : (c.kind == LSAMP_KIND_ARGMAX ? 1 : 0);
  const float mp = prm.min_p > 1.0f ? 1.0f : prm.min_p;
  const bool m_on = c.kind == LSAMP_KIND_FILTERED && mp > 0.0f;
  const float ln_mp = m_on ? __builtin_logf(mp) : 0.0f;
  const bool mlx = P.semantics == LSAMP_SEM_MLXLM;
  // the per-thread arrays are indexed by unrolled constants only (registers)
  double e_loc[kFinalPerThread];
  double e_sum = 0.0;
#pragma unroll
  for (int u = 0; u < kFinalPerThread; ++u) {
    const int r = r0 + u;
    double e = 0.0;
    if (u < per && r < nc) e = (double)__builtin_expf(key_y(F.keys[r]) - info.q_top);
    e_loc[u] = e;
    e_sum += e;
  }
  double e_tot = 0.0;
  double e_excl = block_excl_scan(e_sum, L.redd, &e_tot);
  int32_t surv_loc = 0;
  uint8_t surv[kFinalPerThread];
#pragma unroll
  for (int u = 0; u < kFinalPerThread; ++u) {
    const int r = r0 + u;
    surv[u] = 0;
    if (u >= per || r >= nc) continue;
    const uint32_t kr = (uint32_t)(F.keys[r] >> 32);
    const float y = key_to_float(kr);
    bool keep_p = true, keep_m = true;
    if (mlx) {
      // tie group [g0, g1) of equal values (sorted by id ascending)
      int lo = 0, hi = r;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((uint32_t)(F.keys[mid] >> 32) == kr) hi = mid; else lo = mid + 1;
      }
      const int g0 = lo;
      lo = r;
      hi = nc - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((uint32_t)(F.keys[mid] >> 32) == kr) lo = mid; else hi = mid - 1;
      }
      const int g1 = lo + 1;
      // mass ranked strictly before r when equal values put higher ids first
      // (ascending stable argsort, Evaluate.swift:463-469)
      const double sp = info.mass_above + e_excl - (double)(r - g0) * e_loc[u] +
                        (double)(g1 - 1 - r) * e_loc[u];
      if (p_on) keep_p = sp < P_lim;
      if (m_on) keep_m = (y - y_max) >= ln_mp;
    } else {
      const double sr = info.mass_above + e_excl;
      if (p_on) keep_p = sr <= P_lim;
      if (m_on) keep_m = __builtin_expf(y - y_max) >= mp;
      const int64_t rank = (int64_t)info.count_above + r;
      if (k_lim > 0 && rank >= k_lim) keep_p = false;
    }
    surv[u] = (keep_p && keep_m) ? 1 : 0;
    surv_loc += surv[u];
    e_excl += e_loc[u];
  }
  int32_t surv_tot = 0;
  int32_t surv_excl = block_excl_scan(surv_loc, L.redi, &surv_tot);
  int32_t kc_loc = 0;
  double cent = 0.0;
  float cmin = kPosInf;
#pragma unroll
  for (int u = 0; u < kFinalPerThread; ++u) {
    const int r = r0 + u;
    if (u >= per || r >= n2) continue;
    uint8_t keep = surv[u];
    if (keep && mlx && k_lim > 0) {
      keep = ((int64_t)info.count_above + surv_excl) < k_lim ? 1 : 0;
      ++surv_excl;
    }
    F.keep[r] = keep;
    if (keep) {
      const float y = key_y(F.keys[r]);
      const uint64_t wgt = weight(y, y_max, c.scale);
      atomicAdd(reinterpret_cast<unsigned long long*>(&F.rowchunk[key_id(F.keys[r]) / kChunk]),
                (unsigned long long)wgt);
      cent += (double)wgt * (1.0 / 1099511627776.0) * (double)weight_arg(y, y_max, c.scale);
      cmin = __builtin_fminf(cmin, y);
      ++kc_loc;
    }
  }
  cent = block_sum(cent, L.redd);
  cmin = block_min(cmin, L.redf);
  int32_t kept_c = 0;
  int32_t kexcl = block_excl_scan(kc_loc, L.redi, &kept_c);
  // persist kept candidates (MTP residual pass) and the keep bytes of every
  // candidate (parity output; the select phase leaves candidates' bytes alone)
  for (int u = 0; u < per; ++u) {
    const int r = r0 + u;
    if (r >= nc) break;
    if (F.keep[r]) {
      rc[kexcl].y = key_y(F.keys[r]);
      rc[kexcl].id = key_id(F.keys[r]);
      ++kexcl;
    }
    if (P.keep) P.keep[(size_t)row * (size_t)V + key_id(F.keys[r])] = F.keep[r];
  }

  // ---- total weight and the chunk holding the target
  const uint64_t wt = F.rowchunk[tid];
  uint64_t W = 0ull;
  const uint64_t wexcl = block_excl_scan(wt, L.redu, &W);
  const uint64_t target = W ? scaled_target(uniform_u32(u_draw), W) : 0ull;
  if (tid == 0) {
    L.misc[2] = -1;
    L.misc[3] = -1;
  }
  __syncthreads();
  if (W && wt && wexcl <= target && target < wexcl + wt) {
    L.misc[2] = tid;
    L.misc64[0] = target - wexcl;
  }
  __syncthreads();
  const int cstar = (overflow || !active) ? -1 : L.misc[2];
  const uint64_t ltarget = L.misc64[0];

  if (cstar >= 0) {
    const int64_t cb = (int64_t)cstar * kChunk;
    const int64_t ce = cb + kChunk < V ? cb + kChunk : V;
    const int cps = P.slice_len / kChunk;
    const int sc = cstar / cps;
    const bool list_ok = L.part[sc].n_list <= kKeptCap;
    if (tid == 0) L.nitems = 0;
    __syncthreads();
    if (list_ok) {
      // fast path: the kept tokens of this chunk are all listed
      const KeptItem* kl = ws.klist + ((size_t)row * kMaxSlices + sc) * kKeptCap;
      const int nl = L.part[sc].n_list;
      static_assert(kKeptCap <= kThreads, "one listed item per thread");
      if (tid < nl) {
        const int32_t id = ld_coherent(&kl[tid].id);
        if (id >= cb && id < ce) {
          const int slot = atomicAdd(&L.nitems, 1);
          F.did[slot] = id;
          F.dw[slot] = ld_coherent(&kl[tid].w);
        }
      }
      for (int r = tid; r < nc; r += kThreads) {
        if (!F.keep[r]) continue;
        const int32_t id = key_id(F.keys[r]);
        if (id >= cb && id < ce) {
          const int slot = atomicAdd(&L.nitems, 1);
          F.did[slot] = id;
          F.dw[slot] = weight(key_y(F.keys[r]), y_max, c.scale);
        }
      }
      __syncthreads();
      const int ni = L.nitems;
      int m2 = 1;
      while (m2 < ni) m2 <<= 1;
      for (int i = ni + tid; i < m2; i += kThreads) {
        F.did[i] = 0x7fffffff;
        F.dw[i] = 0ull;
      }
      __syncthreads();
      for (int kk = 2; kk <= m2; kk <<= 1) {
        for (int jj = kk >> 1; jj > 0; jj >>= 1) {
          for (int i = tid; i < m2; i += kThreads) {
            const int ixj = i ^ jj;
            if (ixj > i) {
              const int32_t a = F.did[i], b = F.did[ixj];
              const bool asc = (i & kk) == 0;
              if (asc ? (a > b) : (a < b)) {
                F.did[i] = b;
                F.did[ixj] = a;
                const uint64_t t = F.dw[i];
                F.dw[i] = F.dw[ixj];
                F.dw[ixj] = t;
              }
            }
          }
          __syncthreads();
        }
      }
      // items 2t, 2t+1 per thread, in id order
      const uint64_t w0 = 2 * tid < ni ? F.dw[2 * tid] : 0ull;
      const uint64_t w1 = 2 * tid + 1 < ni ? F.dw[2 * tid + 1] : 0ull;
      uint64_t tot = 0ull;
      const uint64_t ex = block_excl_scan(w0 + w1, L.redu, &tot);
      if (w0 && ex <= ltarget && ltarget < ex + w0) L.misc[3] = F.did[2 * tid];
      if (w1 && ex + w0 <= ltarget && ltarget < ex + w0 + w1) L.misc[3] = F.did[2 * tid + 1];
      __syncthreads();
    } else {
      // scan the chunk in token order (re-read from L2 / HBM)
      for (int i = tid; i < kChunk; i += kThreads) {
        F.cent[i] = 0;
        F.cflag[i] = 0;
      }
      __syncthreads();
      for (int r = tid; r < nc; r += kThreads) {
        if (!F.keep[r]) continue;
        const int32_t id = key_id(F.keys[r]);
        if (id >= cb && id < ce) F.cflag[id - cb] = 1;
      }
      int32_t e0 = 0, e1 = 0;
      if (P.row_ptr && P.entries) {
        e0 = P.row_ptr[row];
        e1 = P.row_ptr[row + 1];
      }
      for (int32_t e = e0 + tid; e < e1; e += kThreads) {
        const lsamp_penalty_entry ent = P.entries[e];
        if (ent.token < cb || ent.token >= ce) continue;
        float x = load_scalar<DT>(rowp, ent.token);
        x = patch_value(c, prm, x, ent, DT);
        if (!mask_allows(mrow, P.mask_words, P.mask_bits, P.mask_tail, ent.token)) x = kNegInf;
        if (x != x) x = kNegInf;
        F.cx[ent.token - cb] = x;
        F.cent[ent.token - cb] = 1;
      }
      __syncthreads();
      uint64_t wl[2] = {0ull, 0ull};
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int li = 2 * tid + u;
        const int64_t i = cb + li;
        if (i >= ce) continue;
        const float x = token_value<DT>(P, c, prm, row, rowp, mrow, i, &F.cx[li], &F.cent[li]);
        const int cls = classify(make_rule(info, c), x);
        if (cls == kKept || (cls == kCand && F.cflag[li]))
          wl[u] = weight(to_filter(c, x), y_max, c.scale);
      }
      uint64_t ctot = 0ull;
      const uint64_t cex = block_excl_scan(wl[0] + wl[1], L.redu, &ctot);
      if (wl[0] && cex <= ltarget && ltarget < cex + wl[0]) L.misc[3] = (int)(cb + 2 * tid);
      if (wl[1] && cex + wl[0] <= ltarget && ltarget < cex + wl[0] + wl[1])
        L.misc[3] = (int)(cb + 2 * tid + 1);
      __syncthreads();
    }
  }
  const int token = cstar >= 0 ? L.misc[3] : -1;

  // ---- probe token (MTP acceptance): its kept weight
  uint64_t probe_w = 0ull;
  if (probe >= 0 && probe < V && !overflow && active) {
    if (tid == 0) {
      L.misc[4] = 0;
      L.misc[5] = 0;
    }
    __syncthreads();
    for (int r = tid; r < nc; r += kThreads)
      if (F.keep[r] && key_id(F.keys[r]) == probe) L.misc[4] = 1;
    int32_t e0 = 0, e1 = 0;
    if (P.row_ptr && P.entries) {
      e0 = P.row_ptr[row];
      e1 = P.row_ptr[row + 1];
    }
    for (int32_t e = e0 + tid; e < e1; e += kThreads) {
      const lsamp_penalty_entry ent = P.entries[e];
      if (ent.token != probe) continue;
      const float x = patch_value(c, prm, load_scalar<DT>(rowp, probe), ent, DT);
      F.cx[0] = x;
      L.misc[5] = 1;
    }
    __syncthreads();
    if (tid == 0) {
      float x = L.misc[5] ? F.cx[0] : load_scalar<DT>(rowp, probe);
      if (!mask_allows(mrow, P.mask_words, P.mask_bits, P.mask_tail, probe) || x != x) x = kNegInf;
      const int cls = classify(make_rule(info, c), x);
      L.misc64[2] = (cls == kKept || (cls == kCand && L.misc[4]))
                        ? weight(to_filter(c, x), y_max, c.scale)
                        : 0ull;
    }
    __syncthreads();
    probe_w = L.misc64[2];
  }

  if (tid == 0) {
    uint32_t flags = info.flags;
    if (overflow) flags |= LSAMP_ROW_OVERFLOW;
    if (!overflow && (token < 0 || W == 0ull)) flags |= LSAMP_ROW_EMPTY;
    const int tok = overflow ? -1 : token;
    P.tokens[row] = tok;
    if (P.row_flags) P.row_flags[row] = flags;
    if (P.stats) {
      lsamp_row_stats st;
      st.max_value = y_max;
      st.log_normalizer =
          info.z > 0.0 ? (float)(log(info.z) + ((double)info.q_top - (double)y_max)) : 0.0f;
      st.kept = kept_all + kept_c;
      st.token = tok;
      st.kept_weight = W;
      st.probe_weight = probe_w;
      st.cut_value = __builtin_fminf(min_all, cmin);
      const double zk = (double)W * (1.0 / 1099511627776.0);
      st.kept_mass = (float)zk;
      st.kept_entropy = zk > 0.0 ? (float)(log(zk) - (ent_all + cent) / zk) : 0.0f;
      st.probe_prob = W ? (float)((double)probe_w / (double)W) : 0.0f;
      P.stats[row] = st;
    }
    ws.rows[row].kept_cands = overflow ? 0 : kept_c;
    ws.cand_count[row] = 0u;
    ws.arrive_select[row] = 0u;
    if (fused) ws.arrive_stats[row] = 0u;
  }
}

// ================================================================ one task
// Register copy of one thread's share of a slice: banks of 32 dwords (8
// quads of 16 bytes).  The loops over quads stay rolled, indexing a bank with
// the uniform loop counter (register-relative moves), so each pass over the
// slice is a short loop body instead of straight-line code per token.
typedef uint32_t bank_t __attribute__((ext_vector_type(32)));
constexpr int kQuadsPerBank = 8;

template <int DT>
struct Slab {
  static constexpr int N = Vec<DT>::N;                  // tokens per quad
  static constexpr int Q = kElemsPerThread / N;         // quads per thread
  static constexpr int NB = Q / kQuadsPerBank;          // banks
  static_assert(Q % kQuadsPerBank == 0, "whole banks");
  bank_t bank[NB];
};

__device__ __forceinline__ uint4 quad_get(const bank_t& b, int s) {
  return make_uint4(b[4 * s], b[4 * s + 1], b[4 * s + 2], b[4 * s + 3]);
}
__device__ __forceinline__ void quad_set(bank_t& b, int s, const uint4& v) {
  b[4 * s] = v.x;
  b[4 * s + 1] = v.y;
  b[4 * s + 2] = v.z;
  b[4 * s + 3] = v.w;
}

// f(g, v) for the thread's quads g < nq (g is uniform); when f returns true
// the quad is written back.
template <int DT, typename F>
__device__ __forceinline__ void for_quads(Slab<DT>& S, int nq, F&& f) {
#pragma unroll
  for (int b = 0; b < Slab<DT>::NB; ++b) {
    const int n = nq - b * kQuadsPerBank;
    if (n <= 0) break;
    const int m = n < kQuadsPerBank ? n : kQuadsPerBank;
#pragma unroll 1
    for (int s = 0; s < m; ++s) {
      uint4 v = quad_get(S.bank[b], s);
      if (f(b * kQuadsPerBank + s, v)) quad_set(S.bank[b], s, v);
    }
  }
}

// Accumulates a probe of the quad's exponent fields: bit 15 / 31 (16-bit
// types) or bit 31 (fp32) of the result is set when some element is inf/NaN.
template <int DT>
__device__ __forceinline__ uint32_t nonfinite_probe(const uint4& v) {
  constexpr uint32_t M = DT == LSAMP_DTYPE_F32 ? 0x7f800000u
                                               : (DT == LSAMP_DTYPE_BF16 ? 0x7f807f80u : 0x7c007c00u);
  constexpr uint32_t A = DT == LSAMP_DTYPE_F32 ? 0x00800000u
                                               : (DT == LSAMP_DTYPE_BF16 ? 0x00800080u : 0x04000400u);
  return ((v.x & M) + A) | ((v.y & M) + A) | ((v.z & M) + A) | ((v.w & M) + A);
}
template <int DT>
__device__ __forceinline__ bool nonfinite_seen(uint32_t acc) {
  return (acc & (DT == LSAMP_DTYPE_F32 ? 0x80000000u : 0x80008000u)) != 0u;
}

template <int DT, int MODE>
__device__ __forceinline__ void run_task(const Workspace& ws, const SamplePlan& P, int row, int slice,
                                         TaskLds& L) {
  constexpr int N = Vec<DT>::N;
  constexpr int Q = Slab<DT>::Q;
  constexpr uint32_t FULL = (1u << N) - 1u;
  constexpr int ES = Vec<DT>::ESIZE;
  const int tid = fresh_tid();
  const int G = P.slices;
  const lsamp_row_params prm = P.params[row];
  const RowCtx c = make_ctx(P.semantics, prm);
  const int64_t V = P.vocab;
  const int64_t base = (int64_t)slice * P.slice_len;
  const int64_t end = (base + P.slice_len < V) ? base + P.slice_len : V;
  const char* rowp = row_base(P, row);
  const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * (size_t)P.mask_words : nullptr;
  const bool aligned = P.aligned != 0;
  // Token positions within a row fit in 32 bits (vocab <= kMaxVocab).
  const int32_t base32 = (int32_t)base, end32 = (int32_t)end;
  const int nq = (P.slice_len + kThreads * N - 1) / (kThreads * N);  // quads per thread

  // ---------------------------------------------------- A: loads + entries
  // Aligned whole quads are read as 16-byte vectors, all in flight at once;
  // lanes past the slice end read as zero until the exclusion pass.
  // (uniform base address per quad + the lane's 32-bit byte offset)
  Slab<DT> S;
  const uint32_t lane_off = (uint32_t)tid * 16u;
#pragma unroll
  for (int g = 0; g < Q; ++g) {
    if (g < nq) {
      const int32_t i0 = base32 + (tid + g * kThreads) * N;
      const char* qbase = rowp + ((size_t)base32 + (size_t)g * kThreads * N) * ES;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (aligned && i0 + N <= end32) v = *reinterpret_cast<const uint4*>(qbase + lane_off);
      quad_set(S.bank[g / kQuadsPerBank], g % kQuadsPerBank, v);
    }
  }
  if (!aligned || (end32 & (N - 1)) != 0) {
    // unaligned rows, or the row's last partial quad: element by element
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
  if (MODE != kSelectOnly)
    for (int i = tid; i < kHist; i += kThreads) L.u.hist[i] = 0ull;
  if (tid == 0) L.flags = 0u;
  SliceEntries se{L.pen, L.etok, L.ex, &L.ecount};
  bool ent_overflow = false;
  const int n_ent = build_slice_entries<DT>(P, c, prm, row, rowp, base, end, se, &ent_overflow);

  // Masked tokens, tokens of the entry table (their patched values live in
  // L.ex) and lanes past the slice end become -inf in the register copy, and
  // so do NaNs.  From here on "excluded" is simply "not > -inf".  The same
  // pass takes the thread's maximum.
  uint32_t nf_acc = 0u;
  float xmax = kNegInf;
  for_quads(S, nq, [&](int g, uint4& v) -> bool {
    const int32_t i0 = base32 + (tid + g * kThreads) * N;
    const uint32_t probe = nonfinite_probe<DT>(v);
    nf_acc |= probe;
    uint32_t ex = FULL;
    if (i0 < end32) {
      const int32_t nvalid = end32 - i0;
      const uint32_t valid = nvalid >= N ? FULL : ((1u << nvalid) - 1u);
      const uint32_t allow = mask_allow_bits(mrow, P.mask_words, P.mask_bits, P.mask_tail, i0, N);
      const int32_t li0 = i0 - base32;
      const uint32_t pen = (L.pen[li0 >> 5] >> (uint32_t)(li0 & 31)) & FULL;
      ex = (~allow | pen | ~valid) & FULL;
    }
    if (nonfinite_seen<DT>(probe)) {
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float x = vec_elem<DT>(v, e);
        if (x != x) ex |= 1u << e;
      }
    }
    if (ex != 0u) exclude_elems<DT>(v, ex);
    if (MODE != kSelectOnly) {
#pragma unroll
      for (int e = 0; e < N; ++e) xmax = __builtin_fmaxf(xmax, vec_elem<DT>(v, e));
    }
    return ex != 0u;
  });
  const bool nonfinite = nonfinite_seen<DT>(nf_acc);

  RowInfo info;
  if (MODE != kSelectOnly) {
    // ------------------------------------------------ B: max, histogram
    for (int j = tid; j < n_ent; j += kThreads) xmax = __builtin_fmaxf(xmax, L.ex[j]);
    if (nonfinite) atomicOr(&L.flags, LSAMP_ROW_NONFINITE);
    xmax = block_max(xmax, L.redf);
    const bool posinf = xmax == kPosInf;
    const bool has_finite = xmax > kNegInf && !posinf;
    const uint32_t sflags = L.flags | (ent_overflow ? kSliceEntryOverflow : 0u) |
                            (posinf ? kSlicePosInf : 0u);
    const int32_t top = has_finite ? bin_of(xmax, c.c32) : 0;
    const bool want_hist = has_finite && c.kind != LSAMP_KIND_ARGMAX;
    if (want_hist) {
      const float Lg = 1.4426950408889634f / 32.0f;
      const float tail_edge = (float)(top - kBins + 1);
      auto add = [&](float x) {
        const float s = bin_pos(x, c.c32);
        const float fb = __builtin_floorf(s);
        const int j = top - (int)fb;
        const bool in_win = j < kBins;
        const float e =
            __builtin_amdgcn_exp2f((s - (in_win ? fb : tail_edge)) * Lg + (float)kMassFracBits);
        atomicAdd(reinterpret_cast<unsigned long long*>(&L.u.hist[in_win ? j : kTail]),
                  (unsigned long long)((1ull << kCountShift) | (uint64_t)(uint32_t)e));
      };
      for_quads(S, nq, [&](int g, uint4& v) -> bool {
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const float x = vec_elem<DT>(v, e);
          if (x > kNegInf) add(x);
        }
        return false;
      });
      for (int j2 = tid; j2 < n_ent; j2 += kThreads) {
        const float x = L.ex[j2];
        if (x > kNegInf && x != kPosInf) add(x);
      }
    }
    __syncthreads();
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
    // publish the slice summary; n_finite is the histogram's token count
    // (rows that build one) or whether the slice holds a finite logit
    SliceSummary* Ssum = ws.summaries + ((size_t)row * kMaxSlices + slice);
    int32_t nfin = 0;
    if (want_hist) {
      for (int i = tid; i < kHist; i += kThreads) {
        const uint64_t w = L.u.hist[i];
        nfin += (int32_t)(w >> kCountShift);
        st_coherent(&Ssum->hist[i], w);
      }
      nfin = block_sum(nfin, L.redi);
    } else {
      nfin = (has_finite || posinf) ? 1 : 0;
    }
    if (tid == 0) {
      st_coherent_f32(&Ssum->x_max, xmax);
      st_coherent(&Ssum->top_bin, top);
      st_coherent(&Ssum->flags, sflags);
      st_coherent(&Ssum->n_finite, nfin);
    }
    const bool is_last = arrive_last(&ws.arrive_stats[row], (uint32_t)G, &L.last);
    if (is_last) {
      merge_row(ws, P, row, c, prm, L);
      info = L.info;
      if (MODE == kFused) {
        if (tid == 0) publish_rowinfo(ws.rows + row, info);
        drain_memory();
        __syncthreads();
        if (tid == 0)
          (void)__hip_atomic_fetch_add(&ws.arrive_stats[row], kReady, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
      } else {
        if (tid == 0) {
          ws.rows[row] = info;
          ws.arrive_stats[row] = 0u;
        }
        return;
      }
    } else {
      if (MODE != kFused) return;
      // wait for the row's merge (bounded: the grid always drains)
      if (tid == 0) {
        int it = 0;
        while (ld_coherent(&ws.arrive_stats[row]) < kReady) {
          if (++it >= kSpinLimit) {
            atomicOr(ws.status, kStatusSpinTimeout);
            break;
          }
          __builtin_amdgcn_s_sleep(4);
        }
        L.info = read_rowinfo(ws.rows + row);
      }
      __syncthreads();
      info = L.info;
    }
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
  auto keep_token = [&](float x, int32_t id, uint64_t& part) {
    const float y = to_filter(c, x);
    const uint64_t wq = weight(y, y_max, c.scale);
    part += wq;
    ent += (double)wq * (1.0 / 1099511627776.0) * (double)weight_arg(y, y_max, c.scale);
    min_kept = __builtin_fminf(min_kept, y);
    ++n_kept;
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
    for_quads(S, nq, [&](int g, uint4& v) -> bool {
      const int32_t i0 = base32 + (tid + g * kThreads) * N;
      // screen the quad by its largest element; the rare quads that hold a
      // kept or candidate token are classified element by element
      float qm = vec_elem<DT>(v, 0);
#pragma unroll
      for (int e = 1; e < N; ++e) qm = __builtin_fmaxf(qm, vec_elem<DT>(v, e));
      uint64_t part = 0ull;
      if (qm * rule.c32 >= rule.screen) {
        uint32_t kb = 0u, cb = 0u;
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const int cls = classify(rule, vec_elem<DT>(v, e));
          kb |= (uint32_t)(cls == kKept) << e;
          cb |= (uint32_t)(cls == kCand) << e;
        }
        for (uint32_t bits = kb | cb; bits != 0u; bits &= bits - 1u) {
          const int e = __builtin_ctz(bits);
          const float x = vec_elem_dyn<DT>(v, e);
          if ((kb >> e) & 1u)
            keep_token(x, i0 + e, part);
          else
            cand_token(x, i0 + e);
        }
      }
      // chunk sums: a wave's quads lie in one 1024-token chunk
      if (__ballot(part != 0ull)) {
        const uint64_t sum = wave_sum(part);
        if ((tid & 63) == 0) {
          const int32_t wi0 = ((tid & ~63) + g * kThreads) * N;
          atomicAdd(reinterpret_cast<unsigned long long*>(&L.u.s.chunk[wi0 / kChunk]),
                    (unsigned long long)sum);
        }
      }
      return false;
    });
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
  ent = block_sum(ent, L.redd);
  min_kept = block_min(min_kept, L.redf);
  n_kept = block_sum(n_kept, L.redi);

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
  if (!arrive_last(&ws.arrive_select[row], (uint32_t)G, &L.last)) return;
  finalize_row<DT>(ws, P, row, c, prm, info, L, rowp, mrow, MODE == kFused);
}

// ================================================================ kernels
template <int DT>
__global__ __launch_bounds__(kThreads) void k_fused(Workspace ws, SamplePlan P) {
  __shared__ TaskLds L;
  const int G = P.slices;
  const int rowslot = (int)blockIdx.x / G;
  const int slice = (int)blockIdx.x % G;
  for (int r0 = 0; r0 < P.rows; r0 += P.rows_per_round) {
    const int row = r0 + rowslot;
    if (row < P.rows) run_task<DT, kFused>(ws, P, row, slice, L);
    __syncthreads();
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void k_stats(Workspace ws, SamplePlan P) {
  __shared__ TaskLds L;
  run_task<DT, kStatsOnly>(ws, P, (int)blockIdx.y, (int)blockIdx.x, L);
}

template <int DT>
__global__ __launch_bounds__(kThreads) void k_select(Workspace ws, SamplePlan P) {
  __shared__ TaskLds L;
  run_task<DT, kSelectOnly>(ws, P, (int)blockIdx.y, (int)blockIdx.x, L);
}

template <int DT>
int launch_dt(const Workspace& ws, const SamplePlan& P, hipStream_t st, void* const* events) {
  auto mark = [&](int i) {
    if (events) (void)hipEventRecord(reinterpret_cast<hipEvent_t>(events[i]), st);
  };
  mark(0);
  if (P.fused) {
    const int rounds_rows = P.rows < P.rows_per_round ? P.rows : P.rows_per_round;
    hipLaunchKernelGGL(k_fused<DT>, dim3((unsigned)(rounds_rows * P.slices)), dim3(kThreads), 0, st,
                       ws, P);
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

}  // namespace

int launch_sample(const Workspace& ws, const SamplePlan& P, void* stream, void* const* events) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (P.dtype) {
    case LSAMP_DTYPE_F32: return launch_dt<LSAMP_DTYPE_F32>(ws, P, st, events);
    case LSAMP_DTYPE_BF16: return launch_dt<LSAMP_DTYPE_BF16>(ws, P, st, events);
    default: return launch_dt<LSAMP_DTYPE_F16>(ws, P, st, events);
  }
}

int fused_blocks_per_cu(int dtype) {
  int n = 0;
  hipError_t e;
  switch (dtype) {
    case LSAMP_DTYPE_F32:
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_fused<LSAMP_DTYPE_F32>, kThreads, 0);
      break;
    case LSAMP_DTYPE_BF16:
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_fused<LSAMP_DTYPE_BF16>, kThreads, 0);
      break;
    default:
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_fused<LSAMP_DTYPE_F16>, kThreads, 0);
      break;
  }
  return e == hipSuccess ? n : 0;
}

}  // namespace lsamp
