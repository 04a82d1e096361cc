// lsamp_kernels.hip — gfx950 kernels of the logits-to-token stage.
//
// One sampling step is two launches over a (slices, rows) grid of 512-thread
// work-groups; each work-group owns one slice (<= 32768 tokens) of one row.
//
//  k_stats   reads its slice of logits once from HBM (16-byte vector loads),
//            applies the grammar mask and the sparse penalties exactly as the
//            reference orders them, and builds a histogram of the filter-space
//            logit in 1/32-nat bins (count + fixed-point mass, one packed
//            64-bit LDS atomic per token).  The last work-group of the row to
//            finish merges the slices' histograms and locates the bin that
//            holds the top-k / top-p / min-p cut.
//  k_select  re-reads its slice (L2-resident: same XCD as k_stats), keeps the
//            tokens above the cut bin (fixed-point draw weight per 1024-token
//            chunk) and lists the tokens inside it.  The last work-group of
//            the row sorts those candidates, applies the exact keep rule of
//            the row's semantics, and draws the token by inverse CDF in
//            token-id order: chunk prefix sums, then one 1024-token scan.
//
// Neither kernel waits on another work-group: cross-work-group results are
// published before an atomic arrival counter and only the last arriver reads
// them, so no launch shape can deadlock.  MFMA is not used: the stage is a
// bandwidth- and reduction-bound pass, not a contraction.
#include <hip/hip_runtime.h>

#include "lsamp_device.h"
#include "lsamp_internal.h"

namespace lsamp {
namespace {

using namespace dev;

constexpr int kSliceWords = kMaxSliceLen / 32;       // penalty bitmap words
constexpr int kSliceChunks = kMaxSliceLen / kChunk;  // chunks per slice
constexpr int kMaxRowChunks = kMaxSlices * kSliceChunks;
constexpr int kFinalPerThread = kCandCap / kThreads;  // sorted candidates per thread

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

// Allowed bits (1 = allowed) of the N tokens starting at i0.
__device__ __forceinline__ uint32_t mask_allow_bits(const uint32_t* mrow, int32_t mask_words,
                                                    int32_t mask_bits, int32_t tail, int64_t i0,
                                                    int N) {
  const uint32_t full = (N == 32) ? 0xffffffffu : ((1u << N) - 1u);
  if (!mrow) return full;
  if (i0 + N <= mask_bits && (i0 >> 5) < mask_words) {
    return (mrow[i0 >> 5] >> (uint32_t)(i0 & 31)) & full;
  }
  uint32_t bits = 0;
  for (int q = 0; q < N; ++q) {
    const int64_t i = i0 + q;
    uint32_t a;
    if (i >= mask_bits || (i >> 5) >= mask_words)
      a = tail == LSAMP_MASK_TAIL_KEEP ? 1u : 0u;
    else
      a = (mrow[i >> 5] >> (uint32_t)(i & 31)) & 1u;
    bits |= a << q;
  }
  return bits;
}

__device__ __forceinline__ bool mask_allows(const uint32_t* mrow, int32_t mask_words,
                                            int32_t mask_bits, int32_t tail, int64_t i) {
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

// Token classes relative to the row's cut.
constexpr int kDrop = 0, kKept = 1, kCand = 2;

__device__ __forceinline__ int classify(const RowInfo& info, const RowCtx& c, float x) {
  if (info.mode == kModePosInf) return x == kPosInf ? kKept : kDrop;
  if (!(x > kNegInf) || x == kPosInf) return kDrop;
  if (info.mode != kModeNormal) return kDrop;
  if (info.cut == kCutNone) return kKept;
  int j = info.top_bin - bin_of(x, c.c32);
  if (j > kBins || j < 0) j = j < 0 ? 0 : kBins;
  if (info.cut == kCutTail) return j < kBins ? kKept : kCand;
  return j < info.cut ? kKept : (j == info.cut ? kCand : kDrop);
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

// ================================================================ k_stats
template <int DT>
__global__ __launch_bounds__(kThreads) void k_stats(Workspace ws, SamplePlan P) {
  constexpr int N = Vec<DT>::N;
  constexpr int NV = kElemsPerThread / N;
  constexpr uint32_t FULL = (1u << N) - 1u;

  __shared__ uint64_t s_hist[kHist];
  __shared__ uint32_t s_pen[kSliceWords];
  __shared__ int32_t s_etok[kSliceEntryCap];
  __shared__ float s_ex[kSliceEntryCap];
  __shared__ int32_t s_ecount;
  __shared__ float s_redf[kWaves];
  __shared__ int32_t s_redi[kWaves];
  __shared__ double s_redd[kWaves];
  __shared__ uint32_t s_flags;
  __shared__ int32_t s_last;
  // merge-phase scratch
  __shared__ float s_hx[kMaxSlices];
  __shared__ int32_t s_htop[kMaxSlices];
  __shared__ uint32_t s_hfl[kMaxSlices];
  __shared__ int32_t s_hn[kMaxSlices];
  __shared__ int32_t s_cutinfo_cnt;
  __shared__ double s_cutinfo_mass;

  const int tid = threadIdx.x;
  const int slice = blockIdx.x;
  const int row = blockIdx.y;
  const lsamp_row_params prm = P.params[row];
  const RowCtx c = make_ctx(P.semantics, prm);
  const int64_t V = P.vocab;
  const int64_t base = (int64_t)slice * P.slice_len;
  const int64_t end = (base + P.slice_len < V) ? base + P.slice_len : V;
  const char* rowp = row_base(P, row);
  const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * (size_t)P.mask_words : nullptr;
  const bool aligned = P.aligned != 0;

  // 1. issue the slice's loads (held in registers through both sweeps)
  uint4 raw[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int64_t i0 = base + (int64_t)(tid + k * kThreads) * N;
    if (i0 < end) raw[k] = load_vec<DT>(rowp, i0, end, aligned);
  }

  // 2. penalties of the slice
  for (int i = tid; i < kHist; i += kThreads) s_hist[i] = 0ull;
  if (tid == 0) s_flags = 0u;
  SliceEntries se{s_pen, s_etok, s_ex, &s_ecount};
  bool ent_overflow = false;
  const int n_ent = build_slice_entries<DT>(P, c, prm, row, rowp, base, end, se, &ent_overflow);

  // 3. sweep 1: exclusions, non-finite flag, max
  uint32_t excl[NV];
  uint32_t fl = 0u;
  float xmax = kNegInf;
  int32_t nfin = 0;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int64_t i0 = base + (int64_t)(tid + k * kThreads) * N;
    if (i0 >= end) {
      excl[k] = FULL;
      continue;
    }
    const int64_t nvalid = end - i0 < N ? end - i0 : N;
    const uint32_t valid = nvalid >= N ? FULL : ((1u << nvalid) - 1u);
    const uint32_t allow = mask_allow_bits(mrow, P.mask_words, P.mask_bits, P.mask_tail, i0, N);
    const int32_t li0 = (int32_t)(i0 - base);
    const uint32_t pen = (s_pen[li0 >> 5] >> (uint32_t)(li0 & 31)) & FULL;
    excl[k] = (~allow | pen | ~valid) & FULL;
#pragma unroll
    for (int q = 0; q < N; ++q) {
      const float x = vec_elem<DT>(raw[k], q);
      if (((valid >> q) & 1u) && !__builtin_isfinite(x)) fl |= LSAMP_ROW_NONFINITE;
      if ((excl[k] >> q) & 1u) continue;
      if (!(x > kNegInf)) continue;
      if (x == kPosInf) {
        fl |= kSlicePosInf;
        continue;
      }
      xmax = __builtin_fmaxf(xmax, x);
      ++nfin;
    }
  }
  for (int j = tid; j < n_ent; j += kThreads) {
    const float x = s_ex[j];
    if (!(x > kNegInf)) continue;
    if (x == kPosInf) {
      fl |= kSlicePosInf;
      continue;
    }
    xmax = __builtin_fmaxf(xmax, x);
    ++nfin;
  }
  if (fl) atomicOr(&s_flags, fl);
  xmax = block_max(xmax, s_redf);
  nfin = block_sum(nfin, s_redi);
  const uint32_t sflags = s_flags | (ent_overflow ? kSliceEntryOverflow : 0u);
  const int32_t top = nfin > 0 ? bin_of(xmax, c.c32) : 0;

  // 4. sweep 2: histogram (count, mass relative to the bin's lower edge)
  const bool want_hist = nfin > 0 && c.kind != LSAMP_KIND_ARGMAX;
  if (want_hist) {
    const float L = 1.4426950408889634f / 32.0f;
    const float tail_edge = (float)(top - kBins + 1);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (excl[k] == FULL) continue;
#pragma unroll
      for (int q = 0; q < N; ++q) {
        if ((excl[k] >> q) & 1u) continue;
        const float x = vec_elem<DT>(raw[k], q);
        if (!(x > kNegInf) || x == kPosInf) continue;
        const float s = bin_pos(x, c.c32);
        const float fb = __builtin_floorf(s);
        const int j = top - (int)fb;
        float e;
        int idx;
        if (j < kBins) {
          e = __builtin_amdgcn_exp2f((s - fb) * L + 30.0f);
          idx = j;
        } else {
          e = __builtin_amdgcn_exp2f((s - tail_edge) * L + 30.0f);
          idx = kTail;
        }
        atomicAdd(reinterpret_cast<unsigned long long*>(&s_hist[idx]),
                  (unsigned long long)((1ull << kCountShift) | (uint64_t)(uint32_t)e));
      }
    }
    for (int j2 = tid; j2 < n_ent; j2 += kThreads) {
      const float x = s_ex[j2];
      if (!(x > kNegInf) || x == kPosInf) continue;
      const float s = bin_pos(x, c.c32);
      const float fb = __builtin_floorf(s);
      const int j = top - (int)fb;
      float e;
      int idx;
      if (j < kBins) {
        e = __builtin_amdgcn_exp2f((s - fb) * L + 30.0f);
        idx = j;
      } else {
        e = __builtin_amdgcn_exp2f((s - tail_edge) * L + 30.0f);
        idx = kTail;
      }
      atomicAdd(reinterpret_cast<unsigned long long*>(&s_hist[idx]),
                (unsigned long long)((1ull << kCountShift) | (uint64_t)(uint32_t)e));
    }
  }

  // 5. parity output: filter-space logits before the filters
  if (P.processed) {
    float* out = P.processed + (size_t)row * (size_t)V;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int64_t i0 = base + (int64_t)(tid + k * kThreads) * N;
      if (i0 >= end) continue;
      const int32_t li0 = (int32_t)(i0 - base);
      const uint32_t pen = (s_pen[li0 >> 5] >> (uint32_t)(li0 & 31)) & FULL;
#pragma unroll
      for (int q = 0; q < N; ++q) {
        if (i0 + q >= end || ((pen >> q) & 1u)) continue;
        const float x = vec_elem<DT>(raw[k], q);
        out[i0 + q] = ((excl[k] >> q) & 1u) || (x != x) ? kNegInf : to_filter(c, x);
      }
    }
    for (int j = tid; j < n_ent; j += kThreads) out[s_etok[j]] = to_filter(c, s_ex[j]);
  }

  // 6. publish the slice summary
  __syncthreads();
  SliceSummary* S = ws.summaries + ((size_t)row * kMaxSlices + slice);
  if (tid == 0) {
    st_coherent_f32(&S->x_max, xmax);
    st_coherent(&S->top_bin, top);
    st_coherent(&S->flags, sflags);
    st_coherent(&S->n_finite, nfin);
  }
  if (want_hist)
    for (int i = tid; i < kHist; i += kThreads) st_coherent(&S->hist[i], s_hist[i]);
  if (!arrive_last(&ws.arrive_stats[row], (uint32_t)P.slices, &s_last)) return;

  // 7. last arriver: merge the row
  const int G = P.slices;
  if (tid < G) {
    const SliceSummary* Ss = ws.summaries + ((size_t)row * kMaxSlices + tid);
    s_hx[tid] = ld_coherent(&Ss->x_max);
    s_htop[tid] = ld_coherent(&Ss->top_bin);
    s_hfl[tid] = ld_coherent(&Ss->flags);
    s_hn[tid] = ld_coherent(&Ss->n_finite);
  }
  __syncthreads();
  float row_max = kNegInf;
  int32_t row_top = 0, n_total = 0;
  uint32_t rflags = 0u;
  bool first = true;
  for (int s = 0; s < G; ++s) {
    rflags |= s_hfl[s];
    n_total += s_hn[s];
    if (s_hn[s] > 0) {
      if (first || s_hx[s] > row_max) row_max = s_hx[s];
      if (first || s_htop[s] > row_top) row_top = s_htop[s];
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
  info.t_min_p = kNegInf;
  info.kept_cands = 0;
  const float s_top = bin_pos(row_max, c.c32);
  info.q_top = s_top * (1.0f / 32.0f);

  if (info.mode == kModeNormal && c.kind == LSAMP_KIND_ARGMAX) {
    info.cut = 0;
    info.count_above = 0;
  } else if (info.mode == kModeNormal) {
    // per-bin counts and masses of the row (thread t owns bins 2t, 2t+1)
    int32_t cnt[2] = {0, 0};
    double mass[2] = {0.0, 0.0};
    int32_t tcnt = 0;
    double tmass = 0.0;
    const double inv_frac = 1.0 / (double)(1ull << kMassFracBits);
    for (int s = 0; s < G; ++s) {
      if (s_hn[s] <= 0) continue;
      const int shift = row_top - s_htop[s];
      const uint64_t* h = ws.summaries[(size_t)row * kMaxSlices + s].hist;
      for (int u = 0; u < 2; ++u) {
        const int i = 2 * tid + u;  // slice-local bin
        const uint64_t w = ld_coherent(&h[i]);
        if (w == 0ull) continue;
        const int32_t wc = (int32_t)(w >> kCountShift);
        const double wm = (double)(w & kMassMask) * inv_frac;
        const int b = s_htop[s] - i;  // absolute bin
        const double f = exp(((double)b - (double)s_top) / 32.0);
        const int j = i + shift;
        if (j >= kBins) {
          tcnt += wc;
          tmass += wm * f;
        }
      }
      if (tid == s) {
        const uint64_t w = ld_coherent(&h[kTail]);
        if (w) {
          tcnt += (int32_t)(w >> kCountShift);
          const double edge = (double)(s_htop[s] - kBins + 1);
          tmass += (double)(w & kMassMask) * inv_frac * exp((edge - (double)s_top) / 32.0);
        }
      }
    }
    // gather-by-owner: each row bin j collects its slices directly
    for (int u = 0; u < 2; ++u) {
      const int j = 2 * tid + u;
      for (int s = 0; s < G; ++s) {
        if (s_hn[s] <= 0) continue;
        const int i = j - (row_top - s_htop[s]);
        if (i < 0 || i >= kBins) continue;
        const uint64_t w = ld_coherent(&ws.summaries[(size_t)row * kMaxSlices + s].hist[i]);
        if (w == 0ull) continue;
        cnt[u] += (int32_t)(w >> kCountShift);
        mass[u] += (double)(w & kMassMask) * inv_frac;
      }
      mass[u] *= exp(((double)(row_top - j) - (double)s_top) / 32.0);
    }
    tcnt = block_sum(tcnt, s_redi);
    tmass = block_sum(tmass, s_redd);
    int32_t tot_cnt = 0;
    double tot_mass = 0.0;
    const int32_t excl_cnt = block_excl_scan(cnt[0] + cnt[1], s_redi, &tot_cnt);
    const double excl_mass = block_excl_scan(mass[0] + mass[1], s_redd, &tot_mass);
    const double z = tot_mass + tmass;
    info.z = z;

    const int32_t k_lim = (prm.top_k > 0 && (int64_t)prm.top_k < V) ? prm.top_k : 0;
    bool p_on;
    double P_lim;
    bool strict;  // CBv2: exclusive mass <= P keeps; mlx-lm: ascending cum > 1-P keeps
    if (P.semantics == LSAMP_SEM_CBV2) {
      p_on = prm.top_p < 1.0f;
      P_lim = (double)(prm.top_p > 0.0f ? prm.top_p : 0.0f) * z;
      strict = false;
    } else {
      p_on = c.kind == LSAMP_KIND_FILTERED && prm.top_p > 0.0f && prm.top_p < 1.0f;
      P_lim = (double)prm.top_p * z;
      strict = true;
    }
    if (c.kind == LSAMP_KIND_CATEGORICAL) p_on = false;
    const bool k_on = c.kind == LSAMP_KIND_FILTERED && k_lim > 0;
    float mp = prm.min_p > 1.0f ? 1.0f : prm.min_p;
    const bool m_on = c.kind == LSAMP_KIND_FILTERED && mp > 0.0f;
    int32_t j_t = kBins + 1;
    if (m_on) {
      const float st = s_top + 32.0f * __builtin_logf(mp);
      j_t = row_top - (int32_t)__builtin_floorf(__builtin_fmaxf(st, -1.0e9f));
      if (j_t < 0) j_t = 0;
      if (j_t > kBins) j_t = kBins;
      info.t_min_p = __builtin_logf(mp);
    }
    info.p_limit = p_on ? P_lim : -1.0;

    int my_cut = 0x7fffffff;
    int32_t C = excl_cnt;
    double M = excl_mass;
    for (int u = 0; u < 2; ++u) {
      const int j = 2 * tid + u;
      if (cnt[u] > 0 || (m_on && j == j_t)) {
        const bool tk = k_on && C + cnt[u] >= k_lim;
        const bool tp = p_on && cnt[u] > 0 && (strict ? (M + mass[u] >= P_lim) : (M + mass[u] > P_lim));
        const bool tm = m_on && j >= j_t;
        if ((tk || tp || tm) && j < my_cut) my_cut = j;
      }
      C += cnt[u];
      M += mass[u];
    }
    const int cut = block_min(my_cut, s_redi);
    if (cut != 0x7fffffff) {
      // owner thread publishes the prefix at the cut
      if (cut / 2 == tid) {
        s_cutinfo_cnt = excl_cnt + ((cut & 1) ? cnt[0] : 0);
        s_cutinfo_mass = excl_mass + ((cut & 1) ? mass[0] : 0.0);
      }
      __syncthreads();
      info.cut = cut;
      info.count_above = s_cutinfo_cnt;
      info.mass_above = s_cutinfo_mass;
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
  if (tid == 0) {
    ws.rows[row] = info;
    ws.arrive_stats[row] = 0u;
  }
}

// =============================================================== k_select
struct SelectShared {
  // bulk phase
  uint32_t pen[kSliceWords];
  int32_t etok[kSliceEntryCap];
  float ex[kSliceEntryCap];
  Candidate wcand[kWgCandCap];
  uint64_t chunk[kSliceChunks];
};
struct FinalShared {
  uint64_t keys[kCandCap];
  uint8_t keep[kCandCap];
  uint64_t rowchunk[kMaxRowChunks];
  float cx[kChunk];
  uint8_t cent[kChunk];
  uint8_t cflag[kChunk];
};
union SelectLds {
  SelectShared a;
  FinalShared b;
};

template <int DT>
__global__ __launch_bounds__(kThreads) void k_select(Workspace ws, SamplePlan P) {
  constexpr int N = Vec<DT>::N;
  constexpr int NV = kElemsPerThread / N;
  constexpr uint32_t FULL = (1u << N) - 1u;

  __shared__ SelectLds L;
  __shared__ int32_t s_ecount;
  __shared__ int32_t s_ncand;
  __shared__ float s_redf[kWaves];
  __shared__ int32_t s_redi[kWaves];
  __shared__ double s_redd[kWaves];
  __shared__ uint64_t s_redu[kWaves];
  __shared__ int32_t s_last;
  __shared__ int32_t s_misc[4];
  __shared__ uint64_t s_misc64[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int slice = blockIdx.x;
  const int row = blockIdx.y;
  const lsamp_row_params prm = P.params[row];
  const RowCtx c = make_ctx(P.semantics, prm);
  const RowInfo info = ws.rows[row];
  const int64_t V = P.vocab;
  const int64_t base = (int64_t)slice * P.slice_len;
  const int64_t end = (base + P.slice_len < V) ? base + P.slice_len : V;
  const char* rowp = row_base(P, row);
  const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * (size_t)P.mask_words : nullptr;
  const bool aligned = P.aligned != 0;
  const float y_max = info.mode == kModePosInf ? kPosInf : to_filter(c, info.x_max);
  const bool active = info.mode != kModeEmpty;

  for (int i = tid; i < kSliceChunks; i += kThreads) L.a.chunk[i] = 0ull;
  if (tid == 0) s_ncand = 0;
  SliceEntries se{L.a.pen, L.a.etok, L.a.ex, &s_ecount};
  bool ent_overflow = false;
  const int n_ent = build_slice_entries<DT>(P, c, prm, row, rowp, base, end, se, &ent_overflow);

  double ent = 0.0;
  float min_kept = kPosInf;
  int32_t n_kept = 0;
  if (!active && P.keep) {
    for (int64_t i = base + tid; i < end; i += kThreads) P.keep[(size_t)row * (size_t)V + i] = 0;
  }
  if (active) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int64_t i0 = base + (int64_t)(tid + k * kThreads) * N;
      const bool in = i0 < end;
      uint64_t part = 0ull;
      uint32_t cand_bits = 0u;
      float cy[N];
      if (in) {
        const uint4 raw = load_vec<DT>(rowp, i0, end, aligned);
        const int64_t nvalid = end - i0 < N ? end - i0 : N;
        const uint32_t valid = nvalid >= N ? FULL : ((1u << nvalid) - 1u);
        const uint32_t allow = mask_allow_bits(mrow, P.mask_words, P.mask_bits, P.mask_tail, i0, N);
        const int32_t li0 = (int32_t)(i0 - base);
        const uint32_t pen = (L.a.pen[li0 >> 5] >> (uint32_t)(li0 & 31)) & FULL;
        const uint32_t ex = (~allow | pen | ~valid) & FULL;
        uint8_t* kout = P.keep ? P.keep + (size_t)row * (size_t)V : nullptr;
#pragma unroll
        for (int q = 0; q < N; ++q) {
          cy[q] = 0.0f;
          // keep bytes of candidates are written by the finalize alone (one
          // writer per byte: plain stores from different XCDs have no order)
          if ((ex >> q) & 1u) {
            if (kout && ((valid & ~pen) >> q & 1u)) kout[i0 + q] = 0;
            continue;
          }
          const float x = vec_elem<DT>(raw, q);
          const int cls = classify(info, c, x);
          if (kout && cls != kCand) kout[i0 + q] = cls == kKept ? 1 : 0;
          if (cls == kKept) {
            const float y = to_filter(c, x);
            const uint64_t w = weight(y, y_max, c.scale);
            part += w;
            ent += (double)w * (1.0 / 1099511627776.0) * (double)weight_arg(y, y_max, c.scale);
            min_kept = __builtin_fminf(min_kept, y);
            ++n_kept;
          } else if (cls == kCand) {
            cy[q] = to_filter(c, x);
            cand_bits |= 1u << q;
          }
        }
      }
      // chunk sums: a wave's vectors lie in one chunk
      const uint64_t any = __ballot(part != 0ull);
      if (any) {
        const uint64_t sum = wave_sum(part);
        if (lane == 0) {
          const int64_t wi0 = (int64_t)((tid & ~63) + k * kThreads) * N;  // slice-local
          atomicAdd(reinterpret_cast<unsigned long long*>(&L.a.chunk[wi0 / kChunk]),
                    (unsigned long long)sum);
        }
      }
      // candidates: wave-aggregated append per element position
#pragma unroll
      for (int q = 0; q < N; ++q) {
        const bool is_c = (cand_bits >> q) & 1u;
        const uint64_t m = __ballot(is_c);
        if (m == 0ull) continue;
        int basei = 0;
        if (lane == __ffsll((unsigned long long)m) - 1)
          basei = atomicAdd(&s_ncand, (int)__popcll(m));
        basei = __shfl(basei, __ffsll((unsigned long long)m) - 1, 64);
        if (is_c) {
          const int off = basei + (int)__popcll(m & ((1ull << lane) - 1ull));
          if (off < kWgCandCap) {
            L.a.wcand[off].y = cy[q];
            L.a.wcand[off].id = (int32_t)(i0 + q);
          }
        }
      }
    }
    for (int j2 = tid; j2 < n_ent; j2 += kThreads) {
      const float x = L.a.ex[j2];
      const int cls = classify(info, c, x);
      const int32_t t = L.a.etok[j2];
      if (P.keep && cls != kCand) P.keep[(size_t)row * (size_t)V + t] = cls == kKept ? 1 : 0;
      if (cls == kKept) {
        const float y = to_filter(c, x);
        const uint64_t w = weight(y, y_max, c.scale);
        atomicAdd(reinterpret_cast<unsigned long long*>(&L.a.chunk[(t - base) / kChunk]),
                  (unsigned long long)w);
        ent += (double)w * (1.0 / 1099511627776.0) * (double)weight_arg(y, y_max, c.scale);
        min_kept = __builtin_fminf(min_kept, y);
        ++n_kept;
      } else if (cls == kCand) {
        const int off = atomicAdd(&s_ncand, 1);
        if (off < kWgCandCap) {
          L.a.wcand[off].y = to_filter(c, x);
          L.a.wcand[off].id = t;
        }
      }
    }
  }
  ent = block_sum(ent, s_redd);
  min_kept = block_min(min_kept, s_redf);
  n_kept = block_sum(n_kept, s_redi);

  // publish chunk sums, candidates, partials
  const int64_t chunk0 = base / kChunk;
  const int nch = (int)((end - base + kChunk - 1) / kChunk);
  uint64_t* rowchunks = ws.chunk_w + (size_t)row * (size_t)ws.max_chunks;
  for (int i = tid; i < nch; i += kThreads) st_coherent(&rowchunks[chunk0 + i], L.a.chunk[i]);
  const int ncand = s_ncand;
  if (tid == 0)
    s_misc[0] = ncand > 0 ? (int)__hip_atomic_fetch_add(&ws.cand_count[row], (uint32_t)ncand,
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : 0;
  __syncthreads();
  const int gbase = s_misc[0];
  const int ncopy = ncand < kWgCandCap ? ncand : kWgCandCap;
  Candidate* rc = ws.cands + (size_t)row * kCandCap;
  for (int i = tid; i < ncopy; i += kThreads)
    if (gbase + i < kCandCap) {
      st_coherent_f32(&rc[gbase + i].y, L.a.wcand[i].y);
      st_coherent(&rc[gbase + i].id, L.a.wcand[i].id);
    }
  if (tid == 0) {
    SelectPartial* sp = ws.partials + (size_t)row * kMaxSlices + slice;
    st_coherent_f64(&sp->ent, ent);
    st_coherent_f32(&sp->min_kept, min_kept);
    st_coherent(&sp->n_kept, n_kept);
    st_coherent(&sp->n_cand, ncand);
    st_coherent(&sp->pad, ent_overflow ? 1 : 0);
  }
  if (!arrive_last(&ws.arrive_select[row], (uint32_t)P.slices, &s_last)) return;

  // ------------------------------------------------------------ finalize
  const int G = P.slices;
  double ent_all = 0.0;
  float min_all = kPosInf;
  int32_t kept_all = 0;
  bool overflow = (info.flags & LSAMP_ROW_OVERFLOW) != 0;
  for (int s = 0; s < G; ++s) {
    const SelectPartial* sp = ws.partials + (size_t)row * kMaxSlices + s;
    const double pe = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&sp->ent)));
    ent_all += pe;
    min_all = __builtin_fminf(min_all, ld_coherent(&sp->min_kept));
    kept_all += ld_coherent(&sp->n_kept);
    if (ld_coherent(&sp->n_cand) > kWgCandCap || ld_coherent(&sp->pad)) overflow = true;
  }
  const uint32_t total_cand = ld_coherent(&ws.cand_count[row]);
  if (total_cand > (uint32_t)kCandCap) overflow = true;
  const int nc = overflow ? 0 : (int)total_cand;
  const int nch_row = P.nchunks;

  // sort candidates: value descending, id ascending
  int n2 = 1;
  while (n2 < nc) n2 <<= 1;
  for (int i = tid; i < n2; i += kThreads) {
    uint64_t key = 0ull;
    if (i < nc) {
      const float y =
          __builtin_bit_cast(float, ld_coherent(reinterpret_cast<const uint32_t*>(&rc[i].y)));
      const int32_t id = ld_coherent(&rc[i].id);
      // -0 and +0 are equal values: both order as +0, ties then go by id
      key = ((uint64_t)ordered_key(y == 0.0f ? 0.0f : y) << 32) |
            (uint64_t)(0xffffffffu - (uint32_t)id);
    }
    L.b.keys[i] = key;
  }
  __syncthreads();
  for (int kk = 2; kk <= n2; kk <<= 1) {
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      for (int i = tid; i < n2; i += kThreads) {
        const int ixj = i ^ jj;
        if (ixj > i) {
          const uint64_t a = L.b.keys[i], b = L.b.keys[ixj];
          const bool desc = (i & kk) == 0;
          if (desc ? (a < b) : (a > b)) {
            L.b.keys[i] = b;
            L.b.keys[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }

  // keep rule over the sorted candidates (thread t owns a contiguous run)
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
  double e_loc[kFinalPerThread];
  double e_sum = 0.0;
  for (int u = 0; u < per; ++u) {
    const int r = r0 + u;
    double e = 0.0;
    if (r < nc) {
      const float y = key_to_float((uint32_t)(L.b.keys[r] >> 32));
      e = (double)__builtin_expf(y - info.q_top);
    }
    e_loc[u] = e;
    e_sum += e;
  }
  double e_tot = 0.0;
  double e_excl = block_excl_scan(e_sum, s_redd, &e_tot);
  int32_t surv_loc = 0;
  uint8_t surv[kFinalPerThread];
  for (int u = 0; u < per; ++u) {
    const int r = r0 + u;
    surv[u] = 0;
    if (r >= nc) continue;
    const uint32_t kr = (uint32_t)(L.b.keys[r] >> 32);
    const float y = key_to_float(kr);
    bool keep_p = true, keep_m = true;
    if (mlx) {
      // tie group [g0, g1) of equal values (sorted by id ascending)
      int lo = 0, hi = r;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((uint32_t)(L.b.keys[mid] >> 32) == kr) hi = mid; else lo = mid + 1;
      }
      const int g0 = lo;
      lo = r;
      hi = nc - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((uint32_t)(L.b.keys[mid] >> 32) == kr) lo = mid; else hi = mid - 1;
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
  int32_t surv_excl = block_excl_scan(surv_loc, s_redi, &surv_tot);
  int32_t kc_loc = 0;
  for (int u = 0; u < per; ++u) {
    const int r = r0 + u;
    if (r >= n2) break;
    uint8_t keep = surv[u];
    if (keep && mlx && k_lim > 0) {
      keep = ((int64_t)info.count_above + surv_excl) < k_lim ? 1 : 0;
      ++surv_excl;
    }
    L.b.keep[r] = keep;
    kc_loc += keep;
  }
  // row chunk sums (published by every slice)
  for (int i = tid; i < nch_row; i += kThreads) L.b.rowchunk[i] = ld_coherent(&rowchunks[i]);
  __syncthreads();
  for (int u = 0; u < per; ++u) {
    const int r = r0 + u;
    if (r >= nc || !L.b.keep[r]) continue;
    const float y = key_to_float((uint32_t)(L.b.keys[r] >> 32));
    const int32_t id = (int32_t)(0xffffffffu - (uint32_t)(L.b.keys[r] & 0xffffffffull));
    const uint64_t w = weight(y, y_max, c.scale);
    atomicAdd(reinterpret_cast<unsigned long long*>(&L.b.rowchunk[id / kChunk]),
              (unsigned long long)w);
  }
  // entropy / min / count contributions of kept candidates
  double cent = 0.0;
  float cmin = kPosInf;
  for (int u = 0; u < per; ++u) {
    const int r = r0 + u;
    if (r >= nc || !L.b.keep[r]) continue;
    const float y = key_to_float((uint32_t)(L.b.keys[r] >> 32));
    const uint64_t w = weight(y, y_max, c.scale);
    cent += (double)w * (1.0 / 1099511627776.0) * (double)weight_arg(y, y_max, c.scale);
    cmin = __builtin_fminf(cmin, y);
  }
  cent = block_sum(cent, s_redd);
  cmin = block_min(cmin, s_redf);
  const int32_t kept_c = block_sum(kc_loc, s_redi);

  // persist kept candidates (ids) for the MTP residual pass
  if (!overflow) {
    int32_t kexcl_tot = 0;
    int32_t kexcl = block_excl_scan(kc_loc, s_redi, &kexcl_tot);
    for (int u = 0; u < per; ++u) {
      const int r = r0 + u;
      if (r >= nc || !L.b.keep[r]) continue;
      const float y = key_to_float((uint32_t)(L.b.keys[r] >> 32));
      const int32_t id = (int32_t)(0xffffffffu - (uint32_t)(L.b.keys[r] & 0xffffffffull));
      rc[kexcl].y = y;
      rc[kexcl].id = id;
      ++kexcl;
    }
    if (P.keep) {
      for (int r = tid; r < nc; r += kThreads) {
        const int32_t id = (int32_t)(0xffffffffu - (uint32_t)(L.b.keys[r] & 0xffffffffull));
        P.keep[(size_t)row * (size_t)V + id] = L.b.keep[r];
      }
    }
  }

  // total weight and the chunk that holds the target
  uint64_t wt = tid < nch_row ? L.b.rowchunk[tid] : 0ull;
  uint64_t W = 0ull;
  const uint64_t wexcl = block_excl_scan(wt, s_redu, &W);
  float u_draw = 0.0f;
  if (P.uniforms)
    u_draw = P.uniforms[row];
  else if (P.philox_keys)
    u_draw = philox_uniform(P.philox_keys[row], 0u);
  const uint64_t target = W ? scaled_target(uniform_u32(u_draw), W) : 0ull;
  if (tid == 0) {
    s_misc[1] = -1;
    s_misc[2] = -1;
  }
  __syncthreads();
  if (W && tid < nch_row && wt && wexcl <= target && target < wexcl + wt) {
    s_misc[1] = tid;
    s_misc64[0] = target - wexcl;
  }
  __syncthreads();
  const int cstar = (overflow || !active) ? -1 : s_misc[1];
  const uint64_t ltarget = s_misc64[0];

  // scan the chosen chunk in token order
  if (cstar >= 0) {
    const int64_t cb = (int64_t)cstar * kChunk;
    const int64_t ce = cb + kChunk < V ? cb + kChunk : V;
    for (int i = tid; i < kChunk; i += kThreads) {
      L.b.cent[i] = 0;
      L.b.cflag[i] = 0;
    }
    __syncthreads();
    for (int i = tid; i < nc; i += kThreads) {
      if (!L.b.keep[i]) continue;
      const int32_t id = (int32_t)(0xffffffffu - (uint32_t)(L.b.keys[i] & 0xffffffffull));
      if (id >= cb && id < ce) L.b.cflag[id - cb] = 1;
    }
    int32_t e0 = 0, e1 = 0;
    if (P.row_ptr && P.entries) {
      e0 = P.row_ptr[row];
      e1 = P.row_ptr[row + 1];
    }
    for (int32_t e = e0 + tid; e < e1; e += kThreads) {
      const lsamp_penalty_entry ent2 = P.entries[e];
      if (ent2.token < cb || ent2.token >= ce) continue;
      float x = load_logit(DT, rowp, ent2.token);
      x = patch_value(c, prm, x, ent2, DT);
      if (!mask_allows(mrow, P.mask_words, P.mask_bits, P.mask_tail, ent2.token)) x = kNegInf;
      if (x != x) x = kNegInf;
      L.b.cx[ent2.token - cb] = x;
      L.b.cent[ent2.token - cb] = 1;
    }
    __syncthreads();
    uint64_t wl[2] = {0ull, 0ull};
    for (int u = 0; u < 2; ++u) {
      const int64_t i = cb + 2 * tid + u;
      if (i >= ce) continue;
      const int li = (int)(i - cb);
      float x;
      if (L.b.cent[li]) {
        x = L.b.cx[li];
      } else {
        x = load_logit(DT, rowp, i);
        if (!mask_allows(mrow, P.mask_words, P.mask_bits, P.mask_tail, i) || x != x) x = kNegInf;
      }
      const int cls = classify(info, c, x);
      if (cls == kKept || (cls == kCand && L.b.cflag[li]))
        wl[u] = weight(to_filter(c, x), y_max, c.scale);
    }
    uint64_t ctot = 0ull;
    const uint64_t cex = block_excl_scan(wl[0] + wl[1], s_redu, &ctot);
    if (wl[0] && cex <= ltarget && ltarget < cex + wl[0]) s_misc[2] = (int)(cb + 2 * tid);
    if (wl[1] && cex + wl[0] <= ltarget && ltarget < cex + wl[0] + wl[1])
      s_misc[2] = (int)(cb + 2 * tid + 1);
    __syncthreads();
  }
  const int token = cstar >= 0 ? s_misc[2] : -1;

  // probe token (MTP acceptance): its kept weight
  uint64_t probe_w = 0ull;
  if (P.probe_tokens) {
    const int32_t pt = P.probe_tokens[row];
    if (tid == 0) s_misc[3] = 0;
    __syncthreads();
    if (pt >= 0 && pt < V && !overflow && active) {
      for (int i = tid; i < nc; i += kThreads) {
        if (!L.b.keep[i]) continue;
        const int32_t id = (int32_t)(0xffffffffu - (uint32_t)(L.b.keys[i] & 0xffffffffull));
        if (id == pt) s_misc[3] = 1;
      }
      __syncthreads();
      if (tid == 0) {
        float x = load_logit(DT, rowp, pt);
        int32_t e0 = 0, e1 = 0;
        if (P.row_ptr && P.entries) {
          e0 = P.row_ptr[row];
          e1 = P.row_ptr[row + 1];
        }
        for (int32_t e = e0; e < e1; ++e)
          if (P.entries[e].token == pt) {
            x = patch_value(c, prm, x, P.entries[e], DT);
            break;
          }
        if (!mask_allows(mrow, P.mask_words, P.mask_bits, P.mask_tail, pt) || x != x) x = kNegInf;
        const int cls = classify(info, c, x);
        if (cls == kKept || (cls == kCand && s_misc[3])) {
          s_misc64[1] = weight(to_filter(c, x), y_max, c.scale);
        } else {
          s_misc64[1] = 0ull;
        }
      }
      __syncthreads();
      probe_w = s_misc64[1];
    }
  }

  if (tid == 0) {
    uint32_t flags = info.flags;
    if (overflow) flags |= LSAMP_ROW_OVERFLOW;
    if (!overflow && (token < 0 || W == 0ull)) flags |= LSAMP_ROW_EMPTY;
    P.tokens[row] = overflow ? -1 : token;
    if (P.row_flags) P.row_flags[row] = flags;
    if (P.stats) {
      lsamp_row_stats st;
      st.max_value = y_max;
      st.log_normalizer = info.z > 0.0 ? (float)(log(info.z) + ((double)info.q_top - (double)y_max)) : 0.0f;
      st.kept = kept_all + kept_c;
      st.token = overflow ? -1 : token;
      st.kept_weight = W;
      st.probe_weight = probe_w;
      st.cut_value = __builtin_fminf(min_all, cmin);
      const double zk = (double)W * (1.0 / 1099511627776.0);
      st.kept_mass = (float)zk;
      st.kept_entropy = zk > 0.0 ? (float)(log(zk) - (ent_all + cent) / zk) : 0.0f;
      st.probe_prob = W ? (float)((double)probe_w / (double)W) : 0.0f;
      P.stats[row] = st;
    }
    RowInfo* ri = ws.rows + row;
    ri->kept_cands = overflow ? 0 : kept_c;
    ws.cand_count[row] = 0u;
    ws.arrive_select[row] = 0u;
  }
}

}  // namespace

int launch_sample(const Workspace& ws, const SamplePlan& P, void* stream, void* const* events) {
  const dim3 grid((unsigned)P.slices, (unsigned)P.rows);
  const dim3 block(kThreads);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto mark = [&](int i) {
    if (events) (void)hipEventRecord(reinterpret_cast<hipEvent_t>(events[i]), st);
  };
  mark(0);
  switch (P.dtype) {
    case LSAMP_DTYPE_F32:
      hipLaunchKernelGGL(k_stats<LSAMP_DTYPE_F32>, grid, block, 0, st, ws, P);
      mark(1);
      hipLaunchKernelGGL(k_select<LSAMP_DTYPE_F32>, grid, block, 0, st, ws, P);
      break;
    case LSAMP_DTYPE_BF16:
      hipLaunchKernelGGL(k_stats<LSAMP_DTYPE_BF16>, grid, block, 0, st, ws, P);
      mark(1);
      hipLaunchKernelGGL(k_select<LSAMP_DTYPE_BF16>, grid, block, 0, st, ws, P);
      break;
    default:
      hipLaunchKernelGGL(k_stats<LSAMP_DTYPE_F16>, grid, block, 0, st, ws, P);
      mark(1);
      hipLaunchKernelGGL(k_select<LSAMP_DTYPE_F16>, grid, block, 0, st, ws, P);
      break;
  }
  mark(2);
  return (int)hipGetLastError();
}

}  // namespace lsamp
