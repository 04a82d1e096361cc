// lsamp_row.h — per-row building blocks shared by the sampling kernels
// (lsamp_kernels.hip, lsamp_topk.hip): the row's resolved context and its
// penalty / bias / mask transforms in the reference's order, the sparse
// penalty entries of a slice, the register copy of a slice, and the sort key
// of (filter-space value, token id).
#pragma once

#include <hip/hip_runtime.h>

#include "lsamp_device.h"
#include "lsamp_internal.h"

namespace lsamp {
namespace rowops {

using namespace dev;

constexpr int kSliceWords = kMaxSliceLen / 32;  // penalty bitmap words

// A copy of a kernel argument whose every dword went through an SGPR as an
// opaque value: all of its scalar loads are issued together, and none is
// repeated later.
template <typename T>
__device__ __forceinline__ T in_sgprs(const T& v) {
  constexpr int kW = (int)((sizeof(T) + 3) / 4);
  uint32_t w[kW];
  __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
  for (int i = 0; i < kW; ++i) asm volatile("" : "+s"(w[i]));
  T out;
  __builtin_memcpy(&out, w, sizeof(T));
  return out;
}

// The thread index through an empty asm statement: values derived from it
// cannot be hoisted out of the fused kernel's loop over rounds (where they
// would stay live, and spill, across the whole task).
__device__ __forceinline__ int fresh_tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// e^a for the rescale factors of the merges (a <= ~0.1): the hardware base-2
// exponential, about 1e-7 relative.  The fused kernel evaluates no double-
// precision exp / log (their constants would stay in registers for the
// whole kernel).
__device__ __forceinline__ double fexp(double a) {
  return (double)__builtin_amdgcn_exp2f((float)(a * 1.4426950408889634));
}

// ------------------------------------------------------------ row context
struct RowCtx {
  int32_t sem;
  int32_t kind;
  float T;        // temperature dividing the filter space (CBv2 sampled rows)
  bool tempered;  // filter space is x / T
  float c32;      // histogram scale: bin = floor(x * c32), x the transformed logit
  float lg;       // log2(e) / (32 * T_f): bin units -> log2 of filter-space mass
  double tf;      // T_f, the filter space's temperature (T when tempered, else 1)
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
  // Bins are 1/32 of the transformed logit x itself (not of x / T): the
  // window of kBins bins then spans 32 logit units at every temperature, and
  // a low temperature cannot push a top-k cut out of it.  Masses carry T.
  c.c32 = 32.0f;
  c.tf = c.tempered ? (double)c.T : 1.0;
  c.lg = (float)(1.4426950408889634 / (32.0 * c.tf));
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
  const uint32_t word = word_in ? gmem(mrow)[wi] : 0u;
  int32_t nin = word_in ? mask_bits - i0 : 0;  // leading positions the mask covers
  nin = nin < 0 ? 0 : (nin > N ? N : nin);
  const uint32_t in_mask = nin >= 32 ? 0xffffffffu : ((1u << nin) - 1u);
  const uint32_t bits = (word >> (uint32_t)(i0 & 31)) & in_mask;
  return (bits | (tail == LSAMP_MASK_TAIL_KEEP ? (full & ~in_mask) : 0u)) & full;
}

// The grammar mask of one slice, staged in LDS for the pass over the slice:
// word w holds the allow bits (what mask_allow_bits gives) of the slice's
// tokens 32w .. 32w + 31, so the pass reads LDS instead of waiting on a
// global word for every quad.  Slices start on a multiple of 32 tokens.
// The raw words are requested ahead of the slice's logits (loads complete
// in order, so they land first), then converted and stored.
constexpr int kMaskStage = kMaxSliceLen / 32 / kThreads;  // words per thread
struct MaskStage {
  uint32_t w[kMaskStage];  // raw words tid, tid + kThreads, ...
};
__device__ __forceinline__ void load_mask_stage(const uint32_t* mrow, int32_t mask_words,
                                                int32_t base32, int32_t end32, int tid,
                                                MaskStage& ms) {
  const int nw = (end32 - base32 + 31) >> 5;
#pragma unroll
  for (int k = 0; k < kMaskStage; ++k) {
    const int lw = tid + k * kThreads;
    const int32_t wi = (base32 >> 5) + lw;
    ms.w[k] = (lw < nw && wi < mask_words) ? gmem(mrow)[wi] : 0u;
  }
}
__device__ __forceinline__ void store_mask_stage(const MaskStage& ms, int32_t mask_words,
                                                 int32_t mask_bits, int32_t tail, int32_t base32,
                                                 int32_t end32, int tid, uint32_t* mw) {
  const int nw = (end32 - base32 + 31) >> 5;
#pragma unroll
  for (int k = 0; k < kMaskStage; ++k) {
    const int lw = tid + k * kThreads;
    if (lw >= nw) continue;
    const int32_t wi = (base32 >> 5) + lw;
    const bool word_in = wi < mask_words;
    int32_t nin = word_in ? mask_bits - wi * 32 : 0;  // leading tokens the mask covers
    nin = nin < 0 ? 0 : (nin > 32 ? 32 : nin);
    const uint32_t in_mask = nin >= 32 ? 0xffffffffu : ((1u << nin) - 1u);
    mw[lw] = (ms.w[k] & in_mask) | (tail == LSAMP_MASK_TAIL_KEEP ? ~in_mask : 0u);
  }
}
// The staged allow bits of the N tokens from slice offset li0 (N-aligned).
__device__ __forceinline__ uint32_t staged_allow_bits(const uint32_t* mw, int32_t li0, int N) {
  const uint32_t full = (N == 32) ? 0xffffffffu : ((1u << N) - 1u);
  return (mw[li0 >> 5] >> (uint32_t)(li0 & 31)) & full;
}

__device__ __forceinline__ bool mask_allows(const uint32_t* mrow, int32_t mask_words,
                                            int32_t mask_bits, int32_t tail, int32_t i) {
  return mask_allow_bits(mrow, mask_words, mask_bits, tail, i, 1) != 0u;
}

// Per-row parameter, uniform and probe slots (plain step: the row itself).
__device__ __forceinline__ int params_index(const SamplePlan& P, int row) {
  if (P.vwin == 0) return row;
  return row < P.rows_split ? row / P.vwin : (row - P.rows_split) / (P.vwin - 1);
}
__device__ __forceinline__ int uniform_index(const SamplePlan& P, int row) {
  if (P.vwin == 0 || row < P.rows_split) return row;
  const int d = row - P.rows_split, D = P.vwin - 1;
  return (d / D) * P.vwin + d % D;
}
__device__ __forceinline__ int probe_index(const SamplePlan& P, int row) {
  if (P.vwin == 0) return row;
  const int D = P.vwin - 1;
  if (row >= P.rows_split) return row - P.rows_split;
  const int j = row % P.vwin;
  return j < D ? (row / P.vwin) * D + j : -1;
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

// The row's parameters, as one 32-byte scalar load.
__device__ __forceinline__ lsamp_row_params load_params(const SamplePlan& P, int row) {
  static_assert(sizeof(lsamp_row_params) == 32, "two 16-byte words");
  typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
  const u32x8 raw = load_uniform(reinterpret_cast<const u32x8*>(P.params + params_index(P, row)));
  return __builtin_bit_cast(lsamp_row_params, raw);
}

// Penalty bitmap of the slice + the slice's entries, patched.  Shared by both
// kernels (they must classify identically).
struct SliceEntries {
  uint32_t* pen;    // [kSliceWords]
  int32_t* tok;     // [kSliceEntryCap]
  float* x;         // [kSliceEntryCap] transformed, -inf when masked / NaN
  int32_t* count;   // LDS counter
};

// The row's first KP * kThreads penalty entries, one per thread and pass,
// requested right behind the slice's logits (the CSR bounds come through
// scalar loads, so they do not wait for the slice).  Entries past them are
// loaded after the whole slice (loads complete in order), so a kernel with
// registers to spare prefetches more.
constexpr int kEntPrefetch = 2;  // the default depth: 1,024 entries
template <int KP = kEntPrefetch>
struct EntryPrefetch {
  static constexpr int K = KP;
  int32_t e0, e1;
  lsamp_penalty_entry ent[KP];  // zero past the row's entries
  __device__ bool has(int tid, int k) const { return e0 + tid + k * kThreads < e1; }
};

// The row's CSR bounds (scalar loads; the row's parameters are requested
// just before, so that both arrive in one round).
template <int KP>
__device__ __forceinline__ void entry_bounds(const SamplePlan& P, int row, EntryPrefetch<KP>& ep) {
  ep.e0 = 0;
  ep.e1 = 0;
  if (P.row_ptr && P.entries) {
    // (laundered addresses: see load_uniform; the second word is the next
    // row's start, or the row's length in a fixed-capacity table, chosen by
    // a scalar select so both loads go out in one round)
    uint64_t a = (uint64_t)(P.row_ptr + row);
    uint64_t b = P.row_len ? (uint64_t)(P.row_len + row) : a + sizeof(int32_t);
    asm volatile("" : "+s"(a), "+s"(b));
    typedef const __attribute__((address_space(4))) int32_t* CI;
    const int32_t w0 = *(CI)a, w1 = *(CI)b;
    ep.e0 = w0;
    ep.e1 = P.row_len ? w0 + w1 : w1;
  }
}

template <int KP>
__device__ __forceinline__ void prefetch_entries(const SamplePlan& P, int tid,
                                                 EntryPrefetch<KP>& ep) {
  static_assert(sizeof(lsamp_penalty_entry) == 16, "one 16-byte load per entry");
  // one buffer descriptor over the row's entries: lanes past them read zero,
  // and no branch holds a load back
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<lsamp_penalty_entry*>(P.entries) + ep.e0, 0,
      (ep.e1 - ep.e0) * (int)sizeof(lsamp_penalty_entry), kBufferWord3);
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs, (tid + k * kThreads) * 16, 0, 0);
    ep.ent[k] = __builtin_bit_cast(lsamp_penalty_entry, make_uint4(w[0], w[1], w[2], w[3]));
  }
}

// The slice's penalty entries in two steps around the pass over the slice.
// mark_slice_entries sets the bitmap of entry tokens (which the pass
// excludes) and gives each entry its table slot; the logits of the
// prefetched entries are requested here and arrive while the pass runs.
// finish_slice_entries patches them into the table.  Both steps fold the
// patched values of the calling thread's entries into `emax`.
template <int KP = kEntPrefetch>
struct EntryMarks {
  int slot[KP];
  float xr[KP];
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

template <int DT>
__device__ __forceinline__ float patched_entry(const SamplePlan& P, const RowCtx& c,
                                               const lsamp_row_params& prm, const uint32_t* mrow,
                                               float x, const lsamp_penalty_entry& ent) {
  x = patch_value(c, prm, x, ent, DT);
  if (!mask_allows(mrow, P.mask_words, P.mask_bits, P.mask_tail, ent.token)) x = kNegInf;
  return x != x ? kNegInf : x;
}

template <int DT, int KP>
__device__ __forceinline__ void mark_slice_entries(const SamplePlan& P, const RowCtx& c,
                                                   const lsamp_row_params& prm, const uint32_t* mrow,
                                                   const char* rowp, int64_t base, int64_t end,
                                                   SliceEntries& se, const EntryPrefetch<KP>& ep,
                                                   int tid, EntryMarks<KP>& em, float& emax) {
  for (int i = tid; i < kSliceWords; i += kThreads) se.pen[i] = 0u;
  if (tid == 0) *se.count = 0;
  lds_barrier();
  auto mark = [&](int32_t t) {
    const int32_t li = t - (int32_t)base;
    atomicOr(&se.pen[li >> 5], 1u << (li & 31));
    return atomicAdd(se.count, 1);
  };
  // The prefetched entries take their slots a wave at a time (one counter
  // update per wave, not one per entry); their gather is unconditional, from
  // the slice's first token when there is no entry, so that nothing waits
  // for it before it is used.
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    const int32_t t = ep.ent[k].token;
    const bool in = ep.has(tid, k) && t >= base && t < end;
    if (in) {
      const int32_t li = t - (int32_t)base;
      atomicOr(&se.pen[li >> 5], 1u << (li & 31));
    }
    em.slot[k] = wave_append(in, se.count);
    em.xr[k] = load_scalar<DT>(rowp, in ? t : base);
  }
  // the rest of a long history
  for (int32_t e = ep.e0 + tid + KP * kThreads; e < ep.e1; e += kThreads) {
    const lsamp_penalty_entry ent = gload16(P.entries + e);
    if (ent.token >= base && ent.token < end) {
      const int idx = mark(ent.token);
      if (idx < kSliceEntryCap) {
        const float x = patched_entry<DT>(P, c, prm, mrow, load_scalar<DT>(rowp, ent.token), ent);
        se.x[idx] = x;
        se.tok[idx] = ent.token;
        emax = __builtin_fmaxf(emax, x);
      }
    }
  }
  lds_barrier();  // the bitmap is complete
}

template <int DT, int KP>
__device__ __forceinline__ void finish_slice_entries(const SamplePlan& P, const RowCtx& c,
                                                     const lsamp_row_params& prm,
                                                     const uint32_t* mrow, SliceEntries& se,
                                                     const EntryPrefetch<KP>& ep,
                                                     const EntryMarks<KP>& em, float& emax) {
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    if (em.slot[k] >= 0 && em.slot[k] < kSliceEntryCap) {
      const float x = patched_entry<DT>(P, c, prm, mrow, em.xr[k], ep.ent[k]);
      se.x[em.slot[k]] = x;
      se.tok[em.slot[k]] = ep.ent[k].token;
      emax = __builtin_fmaxf(emax, x);
    }
  }
}

__device__ __forceinline__ int32_t key_id(uint64_t key) {
  return (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
}
__device__ __forceinline__ float key_y(uint64_t key) { return key_to_float((uint32_t)(key >> 32)); }

// Top-p bound on the mass ranked before a token, z the row's total mass (both
// relative to the same e^q): CBv2 keeps exclusive mass <= top_p * z, a
// non-positive top_p keeping the top token (LogitsPipelineV2.swift:199-206,
// 440-445); mlx-lm keeps mass-before < top_p * z for 0 < top_p < 1
// (Evaluate.swift:462-471).  Negative: top-p is off.
__device__ __forceinline__ double top_p_limit(const SamplePlan& P, const RowCtx& c,
                                              const lsamp_row_params& prm, double z) {
  if (c.kind != LSAMP_KIND_FILTERED) return -1.0;
  if (P.semantics == LSAMP_SEM_CBV2)
    return prm.top_p < 1.0f ? (double)(prm.top_p > 0.0f ? prm.top_p : 0.0f) * z : -1.0;
  return (prm.top_p > 0.0f && prm.top_p < 1.0f) ? (double)prm.top_p * z : -1.0;
}

// Rows drawn through the short list: argmax rows (k = 1) and filtered rows
// whose top-k is active and at most kShortMaxK.  0: the histogram path.
__device__ __forceinline__ int short_k(const RowCtx& c, const lsamp_row_params& prm, int64_t V) {
  if (c.kind == LSAMP_KIND_ARGMAX) return 1;
  if (c.kind == LSAMP_KIND_FILTERED && prm.top_k > 0 && (int64_t)prm.top_k < V &&
      prm.top_k <= kShortMaxK)
    return prm.top_k;
  return 0;
}

__device__ __forceinline__ uint32_t key_hi(float y) { return ordered_key(y == 0.0f ? 0.0f : y); }
__device__ __forceinline__ uint64_t cand_key(float y, int32_t id) {
  return ((uint64_t)key_hi(y) << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}

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

// f(g, v) for the quads g whose bit is set in `sel` (uniform, Q <= 32): a
// rolled loop over the set bits of each bank, so a pass that touches a few
// quads costs a few iterations.  When f returns true the quad is written back.
template <int DT, typename F>
__device__ __forceinline__ void for_quads_sel(Slab<DT>& S, uint32_t sel, F&& f) {
  static_assert(Slab<DT>::Q <= 32, "one mask word");
#pragma unroll
  for (int b = 0; b < Slab<DT>::NB; ++b) {
#pragma unroll 1
    for (uint32_t m = (sel >> (b * kQuadsPerBank)) & 0xffu; m != 0u; m &= m - 1u) {
      const int s = __builtin_ctz(m);
      uint4 v = quad_get(S.bank[b], s);
      if (f(b * kQuadsPerBank + s, v)) quad_set(S.bank[b], s, v);
    }
  }
}

// The upper 16 bits of a float rounded toward +inf (an exact bf16 value keeps
// its bits): an upper bound of the value that packs two to a register.
__device__ __forceinline__ uint32_t hi16_up(float x) {
  const uint32_t b = __float_as_uint(x);
  return ((int32_t)b >= 0 ? b + 0xffffu : b) >> 16;
}

// for_quads with every quad at a static register position: fully unrolled
// (larger code, but no register-relative moves, which cost about a third of
// a pass); used by the passes over every token.
template <int DT, typename F>
__device__ __forceinline__ void for_quads_static(Slab<DT>& S, int nq, F&& f) {
#pragma unroll
  for (int g = 0; g < Slab<DT>::Q; ++g) {
    if (g < nq) {
      uint4 v = quad_get(S.bank[g / kQuadsPerBank], g % kQuadsPerBank);
      if (f(g, v)) quad_set(S.bank[g / kQuadsPerBank], g % kQuadsPerBank, v);
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

}  // namespace rowops
}  // namespace lsamp
