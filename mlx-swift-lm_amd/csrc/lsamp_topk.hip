// lsamp_topk.hip — the one-pass top-k kernel of a sampling step.
//
// Rows: argmax rows (either semantics) and CBv2 rows whose top-k is active
// and at most kTopkMaxK.  The CBv2 keep rule (LogitsPipelineV2.
// applyTopKTopPMinP, LogitsPipelineV2.swift:421-453) keeps only tokens ranked
// below k, so a row needs just its k best keys (filter-space value
// descending, token id ascending), its maximum and its total mass.
//
// One 512-thread work-group owns one slice of one row and keeps the slice in
// registers from the load to the end: penalties, the grammar bitmask and the
// temperature are applied as the reference orders them (lsamp_row.h), the
// slice's best keys are found from a threshold, sorted, and published with
// the slice's maximum and mass.  The slice that starts last finalizes the
// row: it merges the slices' sorted lists, applies the keep rule and draws by
// inverse CDF in token-id order (the fixed-point draw of lsamp.h).
//
// Placement: work-groups are dispatched round-robin over the 8 XCDs, so work-
// group b runs on XCD b % 8.  Row r's slices are given to work-groups of XCD
// r % 8, so a row's penalty entries and gathered logits are read through one
// L2.
//
// Hand-off without co-residency: each work-group takes a ticket (an atomic on
// the row's counter) as it starts.  Only the last ticket of a row waits, and
// only for slices that started before it, which finish without waiting for
// anyone.  Their payloads are 64-bit words tagged with the step's epoch, each
// stored and loaded atomically, so every word shows on its own whether it is
// this step's and no fence has to order them.
//
// Threshold: with min-p on, a token below the slice maximum + T ln(min-p)
// cannot be kept (the row maximum is at least the slice's), so that bound is
// tried first.  Otherwise (or when it leaves more than kCandCap tokens), the
// k-th largest thread maximum bounds the slice's k-th key from below; a slice
// whose candidates still overflow (many equal values) finds its exact k-th
// key by a radix select over the 64-bit keys.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "lsamp_device.h"
#include "lsamp_internal.h"
#include "lsamp_row.h"

namespace lsamp {
namespace {

using namespace dev;
using namespace rowops;

constexpr int kCandCap = 1024;   // candidate keys a slice keeps in LDS
constexpr int kRStageCap = 256;  // raw quads staged for the raw candidate scan
constexpr int kRCandCap = 256;   // raw candidates a slice keeps
constexpr int kTkTauBins = 1024;  // thread-maximum histogram
constexpr int kSpin = 1 << 20;   // polls before the finalizer gives a slice up
// lsamp_test_set_spin_limit: > 0 makes the finalizer's wait unreachable (no word
// counts as seen) and gives it up after this many polls
__device__ int32_t g_topk_spin_test = 0;
#ifndef LSAMP_TOPK_FIRST_QUADS
#define LSAMP_TOPK_FIRST_QUADS 2
#endif
constexpr int kTopkFirstQuads = LSAMP_TOPK_FIRST_QUADS;  // slab quads requested ahead of the entries
#ifndef LSAMP_TOPK_REST_AFTER_MARK
#define LSAMP_TOPK_REST_AFTER_MARK 0  // the rest of the slab: 1 after the entries are marked
#endif
static_assert(kTopkWords <= kThreads, "one payload word per thread");
static_assert(kMaxSlices * kTopkMaxK <= kThreads, "one merged key per thread");


// Header words of a slice's payload.  kHNpub holds the slice's key count and,
// in the high half, its raw key count; kHRMax / kHRZ the raw logits' largest
// finite value and their sum of exp(x - that value) (raw log-probabilities).
enum : int { kHMax = 0, kHZHi, kHZLo, kHNpub, kHFlags, kHNinf, kHRMax, kHRZ };
// Slice flags (header word kHFlags).
constexpr uint32_t kFNonfinite = 1u;   // a raw logit is NaN or +-inf
constexpr uint32_t kFLive = 2u;        // a token survived masking (finite or +inf)
constexpr uint32_t kFPosInf = 4u;      // a transformed logit is +inf
constexpr uint32_t kFEntOverflow = 8u; // more penalty entries than the slice table holds
constexpr uint32_t kFRawNaN = 16u;     // a raw logit is NaN
constexpr uint32_t kFRawPosInf = 32u;  // a raw logit is +inf
constexpr float kLog2e = 1.4426950408889634f;

struct TopkLds {
  uint32_t pen[kSliceWords];
  int32_t etok[kSliceEntryCap];
  float ex[kSliceEntryCap];
  uint64_t cand[kCandCap];
  int32_t racc[kCandCap];
  uint64_t best[kMaxSlices * kTopkMaxK];  // slice s's sorted keys at s * kTopkMaxK
  uint64_t rbest[kMaxSlices * kTopkMaxLp];  // slice s's sorted raw keys at s * kTopkMaxLp
  uint64_t merged[kTopkMaxK];             // the row's best keys, sorted
  uint32_t hist[kTkTauBins];
  // the row's slice headers (finalizer)
  float hmax[kMaxSlices];
  double hz[kMaxSlices];
  int32_t hnpub[kMaxSlices];
  uint32_t hflags[kMaxSlices];
  int32_t hninf[kMaxSlices];
  float hrmax[kMaxSlices];
  float hrz[kMaxSlices];
  // reductions
  float redf[kWaves];
  float redf2[kWaves];
  uint32_t redu[kWaves];
  int32_t redi[kWaves];
  uint64_t redz[kWaves];
  float rredf[kWaves];    // raw: the wave's largest finite logit
  float rtop[kWaves];     // raw: each wave's c-th largest finite thread maximum
  uint32_t rstage[4 * kRStageCap];  // raw: the quads that may hold candidates
  int32_t rstage_at[kRStageCap];  // their first token ids
  uint64_t rcand[kRCandCap];      // raw candidates (raw pairs, then keys)
  int32_t rracc[kRCandCap];       // their ranks (the parts sort)
  int32_t nstage;
  int32_t nrcand;
  double rredz[kWaves];   // raw: the wave's sum of exp(x - slice raw maximum)
  int32_t misc[8];
  uint64_t prefix;
  int32_t ecount;
  int32_t ncand;
  uint32_t tag;
  int32_t last;
  int32_t lost;  // the finalizer gave up waiting for a slice
};

// The larger of each 16-bit half of a and b, unsigned (one packed op).
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}

// Ordered 64-bit key of an element of the slice (filter space, id).
__device__ __forceinline__ uint64_t elem_key(const RowCtx& c, float x, int32_t id) {
  return cand_key(to_filter(c, x), id);
}
// A candidate as first listed (its transformed value and id), and its key.
__device__ __forceinline__ uint64_t raw_cand(float x, int32_t id) {
  return ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)id;
}
__device__ __forceinline__ uint64_t cand_key_of(const RowCtx& c, uint64_t r) {
  return elem_key(c, __uint_as_float((uint32_t)(r >> 32)), (int32_t)(uint32_t)r);
}
// Key of a raw logit in the raw order of log-probabilities (value
// descending, lower id on ties, +0 and -0 tied, NaN last): NaN has value
// key 0, below every other value's.
__device__ __forceinline__ uint64_t raw_key(float x, int32_t id) {
  return ((uint64_t)(x != x ? 0u : key_hi(x)) << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}
__device__ __forceinline__ uint64_t raw_key_of(uint64_t r) {
  return raw_key(__uint_as_float((uint32_t)(r >> 32)), (int32_t)(uint32_t)r);
}

// The exclusion bits of a thread's quads (N bits a quad, packed), kept when
// the registers keep the raw logits (the variant that also ranks them).
// (A vector type, not an array: read with a quad index known only at run
// time, an array would be placed in scratch memory.)
template <int DT>
struct ExBits {
  static constexpr int N = Vec<DT>::N;
  static constexpr int PER = 32 / N;  // quads per word
  static constexpr int W = (Slab<DT>::Q + PER - 1) / PER;
  static_assert(W == 4, "four words");
  typedef uint32_t words_t __attribute__((ext_vector_type(4)));
  words_t w;
  __device__ __forceinline__ void clear() { w = words_t{0u, 0u, 0u, 0u}; }
  __device__ __forceinline__ void set(int g, uint32_t ex) {  // g known at compile time
    w[g / PER] |= ex << ((g % PER) * N);
  }
  __device__ __forceinline__ uint32_t get(int g) const {  // any uniform g
    const int i = g / PER;
    const uint32_t x = i < 2 ? (i == 0 ? w.x : w.y) : (i == 2 ? w.z : w.w);
    return (x >> ((g % PER) * N)) & ((1u << N) - 1u);
  }
};

// The exact K-th largest key among a slice's tokens x >= t, for a slice
// whose candidates overflow (many equal values): a radix select over the
// 64-bit keys, eight bits a pass from the top, reading the slice again from
// memory (L2) with the same exclusions as the first pass (the entry bitmap
// and table in LDS, the grammar mask, NaN).  Called by the whole work-group.
template <int DT>
__device__ __noinline__ uint64_t kth_key_mem(const RowCtx c, const char* rowp,
                                             const uint32_t* mrow, int32_t mask_words,
                                             int32_t mask_bits, int32_t mask_tail, int32_t base32,
                                             int32_t end32, int n_ent, float t, int K,
                                             TopkLds& L) {
  const int tid = (int)threadIdx.x;
  uint64_t prefix = 0ull;
  int need = K;
#pragma unroll 1
  for (int shift = 56; shift >= 0; shift -= 8) {
    const uint64_t hmask = shift == 56 ? 0ull : ~0ull << (shift + 8);
    for (int i = tid; i < 256; i += kThreads) L.hist[i] = 0u;
    __syncthreads();
    auto count = [&](float x, int32_t id) {
      if (!(x >= t) || !(x > kNegInf)) return;
      const uint64_t key = elem_key(c, x, id);
      if ((key & hmask) == prefix) atomicAdd(&L.hist[(key >> shift) & 255u], 1u);
    };
#pragma unroll 1
    for (int32_t i = base32 + tid; i < end32; i += kThreads) {
      const int32_t li = i - base32;
      if ((L.pen[li >> 5] >> (li & 31)) & 1u) continue;  // an entry: from the table
      if (mrow && !mask_allows(mrow, mask_words, mask_bits, mask_tail, i)) continue;
      count(load_scalar<DT>(rowp, i), i);  // (a NaN fails x >= t)
    }
    for (int j = tid; j < n_ent; j += kThreads) count(L.ex[j], L.etok[j]);
    __syncthreads();
    if (tid < 64) {
      // digits from the top: lane l holds digits 255 - 4l .. 252 - 4l
      uint32_t cb[4];
      uint32_t cs = 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        cb[i] = L.hist[255 - (4 * tid + i)];
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
  return prefix;
}

// The slice's K best raw keys (every token, NaN included), for a slice whose
// threshold left too few or too many candidates (NaN, +inf or many equal
// logits): a radix select of the exact K-th key over the slice read again
// from memory (L2), then every key at or above it listed as a raw pair in
// L.cand.  Returns how many were listed (min(K, slice length)).  Called by
// the whole work-group.
template <int DT>
__device__ __noinline__ int raw_select_mem(const char* rowp, int32_t base32, int32_t end32, int K,
                                           uint64_t* dst, int32_t* cnt, TopkLds& L) {
  const int tid = (int)threadIdx.x;
  const int len = end32 - base32;
  if (K > len) K = len;
  uint64_t prefix = 0ull;
  int need = K;
#pragma unroll 1
  for (int shift = 56; shift >= 0; shift -= 8) {
    const uint64_t hmask = shift == 56 ? 0ull : ~0ull << (shift + 8);
    for (int i = tid; i < 256; i += kThreads) L.hist[i] = 0u;
    __syncthreads();
#pragma unroll 1
    for (int32_t i = base32 + tid; i < end32; i += kThreads) {
      const uint64_t key = raw_key(load_scalar<DT>(rowp, i), i);
      if ((key & hmask) == prefix) atomicAdd(&L.hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // digits from the top: lane l holds digits 255 - 4l .. 252 - 4l
      uint32_t cb[4];
      uint32_t cs = 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        cb[i] = L.hist[255 - (4 * tid + i)];
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
  // the keys >= the K-th: exactly K of them (keys are distinct)
  if (tid == 0) *cnt = 0;
  __syncthreads();
#pragma unroll 1
  for (int32_t i0 = base32; i0 < end32; i0 += kThreads) {
    const int32_t i = i0 + tid;
    const float x = i < end32 ? load_scalar<DT>(rowp, i) : 0.0f;
    const bool hit = i < end32 && raw_key(x, i) >= prefix;
    const int slot = wave_append(hit, cnt);
    if (hit && slot < K) dst[slot] = raw_cand(x, i);
  }
  __syncthreads();
  return K;
}

template <int DT, bool LP>
__device__ __forceinline__ void topk_task(const SamplePlan& P, const TopkWs& T, const TopkLp& LPo,
                                          int row, int slice, TopkLds& L) {
  constexpr int N = Vec<DT>::N;
  constexpr int Q = Slab<DT>::Q;
  constexpr uint32_t FULL = (1u << N) - 1u;
  constexpr int ES = Vec<DT>::ESIZE;
  const int tid = fresh_tid();
  const int l = tid & 63;
  const int wv = tid >> 6;
  const int G = P.slices;
  const int64_t V = P.vocab;
  const int64_t base = (int64_t)slice * P.slice_len;
  const int64_t end = (base + P.slice_len < V) ? base + P.slice_len : V;
  const char* rowp = row_base(P, row);
  const bool aligned = P.aligned != 0;
  const int32_t base32 = (int32_t)base, end32 = (int32_t)end;
  const int nq = (P.slice_len + kThreads * N - 1) / (kThreads * N);

  // ---------------------------------------------------------- A: loads
  // In dependency order, each request as early as its inputs allow: the
  // first quads of the slice (they need only the kernel arguments), the
  // row's scalar data (CSR bounds, parameters, draw inputs: one round trip),
  // the first penalty entries (they need the bounds), the rest of the slice,
  // then the epoch and the ticket.  The vector counter completes in issue
  // order, so whatever is requested later holds up no wait for the data
  // ahead of it.
  //
  // The slab is requested in two parts around the entries: the first pass
  // waits for the entries, and a request behind the whole slab would wait
  // for all of it.  (Every quad is loaded without a branch: quads past the
  // slice read zero, and straight-line loads let each later wait name its
  // own quad.)
  Slab<DT> S;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(rowp) + (size_t)base32 * ES, 0, aligned ? (end32 - base32) * ES : 0,
      kBufferWord3);
  const int lane_off = tid * 16;
  constexpr int kFirst = Q < kTopkFirstQuads ? Q : kTopkFirstQuads;
  auto load_quads = [&](auto g0, auto g1) {
#pragma unroll
    for (int g = decltype(g0)::value; g < decltype(g1)::value; ++g) {
      const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs, lane_off, g * kThreads * 16, 0);
      quad_set(S.bank[g / kQuadsPerBank], g % kQuadsPerBank, make_uint4(w[0], w[1], w[2], w[3]));
    }
  };
  load_quads(std::integral_constant<int, 0>{}, std::integral_constant<int, kFirst>{});
  // (the parameters first: the bounds are used as soon as they arrive, and
  // one wait then covers both)
  const lsamp_row_params prm = load_params(P, row);
  EntryPrefetch<> ep;
  entry_bounds(P, row, ep);
  prefetch_entries(P, tid, ep);
  // the slice's grammar-mask words, staged in LDS (the candidate area, idle
  // until the extraction) before the first pass
  const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * (size_t)P.mask_words : nullptr;
  MaskStage ms;
  if (mrow) load_mask_stage(mrow, P.mask_words, base32, end32, tid, ms);
  uint32_t* const mw = reinterpret_cast<uint32_t*>(L.cand);
  static_assert(sizeof(L.cand) >= kSliceWords * sizeof(uint32_t), "staged mask words fit");
#if LSAMP_TOPK_REST_AFTER_MARK == 0
  load_quads(std::integral_constant<int, kFirst>{}, std::integral_constant<int, Q>{});
#endif
  const RowCtx c = make_ctx(P.semantics, prm);
  // (defaults the compiler cannot see as constants: with constant ones it
  // moves the later `+ 1`s into this branch, where they would wait for the
  // atomic at once)
  uint32_t ticket, epoch;
  asm volatile("v_mov_b32 %0, 0" : "=v"(ticket));
  asm volatile("v_mov_b32 %0, 0" : "=v"(epoch));
  if (tid == 0) {
    epoch = __hip_atomic_load(gmem(T.epoch) + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // (an increment, not an add: the compiler rewrites a uniform add as a
    // wave-aggregated one whose result it waits for on the spot)
    ticket = __builtin_amdgcn_atomic_inc32(gmem(T.ticket) + row, 0xffffffffu, __ATOMIC_RELAXED,
                                           "agent");
  }
  // the row's sampler: argmax rows, and CBv2 rows with an active top-k of at
  // most kTopkMaxK; any other row (a caller whose host copy of the
  // parameters did not match) fails closed
  const int Kr = short_k(c, prm, V);
  const bool bad_row = Kr <= 0 || Kr > kTopkMaxK ||
                       (c.kind == LSAMP_KIND_FILTERED && P.semantics != LSAMP_SEM_CBV2);
  const int K = bad_row ? 1 : Kr;
  const bool zon = c.kind != LSAMP_KIND_ARGMAX;
  if (tid == 0) {
    L.ncand = 0;
    L.lost = 0;
    L.nstage = 0;
    L.nrcand = 0;
  }
  for (int i = tid; i < kCandCap; i += kThreads) L.racc[i] = 0;
  if constexpr (LP)
    for (int i = tid; i < kRCandCap; i += kThreads) L.rracc[i] = 0;

  // ---------------------------------------------------------- B: entries
  SliceEntries se{L.pen, L.etok, L.ex, &L.ecount};
  EntryMarks<decltype(ep)::K> em;
  float emax = kNegInf;
  if (mrow) store_mask_stage(ms, P.mask_words, P.mask_bits, P.mask_tail, base32, end32, tid, mw);
  mark_slice_entries<DT>(P, c, prm, mrow, rowp, base, end, se, ep, tid, em, emax);
#if LSAMP_TOPK_REST_AFTER_MARK != 0
  load_quads(std::integral_constant<int, kFirst>{}, std::integral_constant<int, Q>{});
#endif
  if (!aligned || (end32 & (N - 1)) != 0) {
    // unaligned rows, or the row's last partial quad: element by element
    for_quads(S, nq, [&](int g, uint4& v) -> bool {
      const int32_t i0 = base32 + (tid + g * kThreads) * N;
      if (i0 >= end32 || (aligned && i0 + N <= end32)) return false;
      uint32_t bb[N];
#pragma unroll
      for (int e = 0; e < N; ++e) bb[e] = i0 + e < end32 ? load_raw_bits<DT>(rowp, i0 + e) : 0u;
      if constexpr (N == 4) {
        v = make_uint4(bb[0], bb[1], bb[2], bb[3]);
      } else {
        v = make_uint4(bb[0] | (bb[1] << 16), bb[2] | (bb[3] << 16), bb[4] | (bb[5] << 16),
                       bb[6] | (bb[7] << 16));
      }
      return true;
    });
  }

  // ---------------------------------------------------------- C: pass 1
  // Masked tokens, entry tokens (patched values in L.ex), lanes past the
  // slice and NaNs become -inf in the registers.  The thread's maximum, its
  // quads' maxima and its sum of exp((x - m) / T_f) (anchored at a quad
  // maximum, re-anchored by an exact power of two) are taken as quads land.
  // (With raw log-probabilities (LP) the registers keep the raw logits, the
  // exclusions are kept as bits, and the raw logits' maximum, quad maxima
  // and sum of exp(x) are taken too, past the slice's end excluded only.)
  const float lgz = (float)(1.4426950408889634 / c.tf);
  const uint32_t* penw = L.pen + ((tid * N) >> 5);
  constexpr int kQuadWords = kThreads * N / 32;
  const uint32_t pen_shift = (uint32_t)((tid * N) & 31);
  const int32_t lim = end32 - base32 - tid * N;
  // the first quad index that is not whole for every thread of this slice
  const int nq_tail = (end32 - base32) / (kThreads * N);
  uint32_t pw = penw[0];
  uint32_t nf_acc = 0u;
  float xmax = kNegInf;
  float zt = 0.0f, nbz = __FLT_MAX__;
  int32_t ninf = 0;  // +inf tokens (counted in the rare quads that hold one)
  // each quad's maximum, rounded up to 16 bits and packed two to a register:
  // the candidate pass visits only the quads whose maximum reaches its bound
  uint32_t qmp[Q / 2];
#pragma unroll
  for (int i = 0; i < Q / 2; ++i) qmp[i] = 0xff80ff80u;  // -inf, -inf
  // (16-bit logits) the largest raw magnitude seen (sign bits cleared), as
  // an unsigned 16-bit pair: NaN and +-inf are the patterns at or above the
  // infinity's, so a packed maximum a word flags every one of them, masked,
  // penalized or not
  uint32_t rawhi = 0u;
  constexpr uint32_t kInfHalf = DT == LSAMP_DTYPE_BF16 ? 0x7f80u : 0x7c00u;
  // (LP) raw statistics and the exclusion bits
  float rmax = kNegInf, zr = 0.0f, nbr = __FLT_MAX__;
  bool rnan = false;
  uint32_t rqp[LP ? Q / 2 : 1];
#pragma unroll
  for (int i = 0; i < (LP ? Q / 2 : 1); ++i) rqp[i] = 0xff80ff80u;
  ExBits<DT> exb;
  exb.clear();
  for_quads_static(S, nq, [&](int g, uint4& vin) -> bool {
    const int32_t i0 = base32 + (tid + g * kThreads) * N;
    const uint32_t pcur = pw;
    if (g + 1 < Q) pw = penw[(g + 1) * kQuadWords];
    uint32_t ex = (pcur >> pen_shift) & FULL;
    uint32_t tl = 0u;
    if (g >= nq_tail) {
      // the quads that can reach past this slice's end: every earlier one is
      // whole for every thread (the last slice of a row is shorter)
      const int32_t rem = lim - g * (kThreads * N);
      tl = (~0u << (uint32_t)(rem < 0 ? 0 : (rem > N ? N : rem))) & FULL;
      ex |= tl;
    }
    if constexpr (LP) {
      uint4 vr = vin;
      if (g >= nq_tail) exclude_elems<DT>(vr, tl);
      float rq = vec_max_nn<DT>(vr);
      if (rq != rq) {
        // a NaN in the quad (rare): the largest of the others
        rq = kNegInf;
#pragma unroll
        for (int e = 0; e < N; ++e) rq = __builtin_fmaxf(rq, vec_elem<DT>(vr, e));
      }
      rmax = __builtin_fmaxf(rmax, rq);
      if (g & 1)
        rqp[g / 2] = (rqp[g / 2] & 0xffffu) | (hi16_up(rq) << 16);
      else
        rqp[g / 2] = (rqp[g / 2] & 0xffff0000u) | hi16_up(rq);
      if (__builtin_fmaf(rq, kLog2e, nbr) > 64.0f) {
        const float nn = -__builtin_ceilf(__builtin_amdgcn_fmed3f(rq * kLog2e, -0x1p20f, 0x1p20f));
        zr = __builtin_ldexpf(zr, (int)__builtin_fmaxf(nn - nbr, -512.0f));
        nbr = nn;
      }
      float t[N];
#pragma unroll
      for (int e = 0; e < N; ++e)
        t[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(vec_elem<DT>(vr, e), kLog2e, nbr));
#pragma unroll
      for (int w = 1; w < N; w *= 2)
#pragma unroll
        for (int e = 0; e < N; e += 2 * w) t[e] += t[e + w];
      zr += t[0];
    }
    // (the registers are masked in place, unless LP keeps them raw)
    uint4 vcopy = vin;
    uint4& v = LP ? vcopy : vin;
    if (mrow) ex |= ~staged_allow_bits(mw, i0 - base32, N) & FULL;
    if constexpr (N == 8) {
      constexpr uint32_t M = 0x7fff7fffu;
      const uint32_t hw = pk_max_u16(pk_max_u16(v.x & M, v.y & M), pk_max_u16(v.z & M, v.w & M));
      rawhi = pk_max_u16(rawhi, hw);
      // (the raw magnitudes are taken before the words are overwritten: with
      // the order left open the compiler keeps a copy of the quad)
      asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w) : "v"(rawhi));
    } else {
      const uint32_t probe = nonfinite_probe<DT>(v);
      nf_acc |= probe;
      if (nonfinite_seen<DT>(probe)) {
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const float x = vec_elem<DT>(v, e);
          if (x != x) {
            ex |= 1u << e;
            rnan = true;
          }
        }
      }
    }
    exclude_elems<DT>(v, ex);
    // the quad's elements, unpacked once for its maximum and its exp-sum
    float f[N];
#pragma unroll
    for (int e = 0; e < N; ++e) f[e] = vec_elem<DT>(v, e);
    auto fmax_of = [&]() {
      float m = f[0];
#pragma unroll
      for (int e = 1; e < N; ++e) m = __builtin_elementwise_maximum(m, f[e]);
      return m;
    };
    float qm = fmax_of();
    if constexpr (N == 8) {
      // a NaN (the maximum propagates it) or +inf in the quad: NaNs out,
      // +inf tokens counted (rare)
      if (!(qm < kPosInf)) {
        uint32_t nan = 0u;
#pragma unroll
        for (int e = 0; e < N; ++e) {
          nan |= (f[e] != f[e] ? 1u : 0u) << e;
          ninf += f[e] == kPosInf ? 1 : 0;
        }
        exclude_elems<DT>(v, nan);
        ex |= nan;
#pragma unroll
        for (int e = 0; e < N; ++e) f[e] = vec_elem<DT>(v, e);
        qm = fmax_of();
        nf_acc = 0x80008000u;
      }
    } else {
      if (qm == kPosInf) {
#pragma unroll
        for (int e = 0; e < N; ++e) ninf += vec_elem<DT>(v, e) == kPosInf ? 1 : 0;
      }
    }
    xmax = __builtin_elementwise_maximum(xmax, qm);
    if (g & 1)
      qmp[g / 2] = (qmp[g / 2] & 0xffffu) | (hi16_up(qm) << 16);
    else
      qmp[g / 2] = (qmp[g / 2] & 0xffff0000u) | hi16_up(qm);
    if (zon) {
      if (__builtin_fmaf(qm, lgz, nbz) > 64.0f) {
        const float nn = -__builtin_ceilf(__builtin_amdgcn_fmed3f(qm * lgz, -0x1p20f, 0x1p20f));
        zt = __builtin_ldexpf(zt, (int)__builtin_fmaxf(nn - nbz, -512.0f));
        nbz = nn;
      }
      // (a pairwise sum per quad: one dependent add a quad on zt)
      float t[N];
#pragma unroll
      for (int e = 0; e < N; ++e) t[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(f[e], lgz, nbz));
#pragma unroll
      for (int w = 1; w < N; w *= 2)
#pragma unroll
        for (int e = 0; e < N; e += 2 * w) t[e] += t[e + w];
      zt += t[0];
    }
    if constexpr (LP) {
      exb.set(g, ex);
      return false;  // the registers keep the raw logits
    } else {
      return true;   // (masked in place)
    }
  });
  if constexpr (N == 8) {
    if ((rawhi & 0xffffu) >= kInfHalf || (rawhi >> 16) >= kInfHalf) nf_acc = 0x80008000u;
    rnan = (rawhi & 0xffffu) > kInfHalf || (rawhi >> 16) > kInfHalf;
  }
  const bool zref = nbz < __FLT_MAX__;
  finish_slice_entries<DT>(P, c, prm, mrow, se, ep, em, emax);
  xmax = __builtin_fmaxf(xmax, emax);
  lds_barrier();  // the entry table is complete
  const int n_all = L.ecount;
  const bool ent_overflow = n_all > kSliceEntryCap;
  const int n_ent = n_all < kSliceEntryCap ? n_all : kSliceEntryCap;

  // ---------------------------------------------------------- D: slice max
  for (int j = tid; j < n_ent; j += kThreads) ninf += L.ex[j] == kPosInf ? 1 : 0;
  const float tmax = xmax;
  {
    const float hi = wave_max(tmax);
    const float lo = wave_min(tmax > kNegInf ? tmax : kPosInf);
    uint32_t nf = __ballot(nonfinite_seen<DT>(nf_acc)) != 0ull ? kFNonfinite : 0u;
    const int32_t ni = wave_sum(ninf);
    float rhi = kNegInf, rct = kNegInf;
    if constexpr (LP) {
      // raw: the largest finite logit, NaN and +inf seen, and the wave's
      // c-th largest finite thread maximum, c = ceil(LPo.k / 8): the waves'
      // 8c largest are >= the smallest of these, so that bounds the slice's
      // LPo.k-th largest thread maximum (and token) from below
      const float rf = rmax < kPosInf ? rmax : kNegInf;
      rhi = wave_max(rf);
      nf |= (__ballot(rnan) ? kFRawNaN : 0u) | (__ballot(rmax == kPosInf) ? kFRawPosInf : 0u);
      const int cth = (LPo.k + kWaves - 1) / kWaves;
      float v = rf;
      rct = rhi;
      for (int i = 1; i < cth; ++i) {
        const uint64_t at = __ballot(v == rct);  // drop one lane holding it
        if (at && l == __builtin_ctzll(at)) v = kNegInf;
        rct = wave_max(v);
      }
    }
    if (l == 0) {
      L.redf[wv] = hi;
      L.redf2[wv] = lo;
      L.redu[wv] = nf;
      L.redi[wv] = ni;
      if constexpr (LP) {
        L.rredf[wv] = rhi;
        L.rtop[wv] = rct;
      }
    }
  }
  __syncthreads();
  float smax = L.redf[0], tlo = L.redf2[0];
  uint32_t sflags = L.redu[0];
  int32_t sninf = L.redi[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) {
    smax = __builtin_fmaxf(smax, L.redf[i]);
    tlo = __builtin_fminf(tlo, L.redf2[i]);
    sflags |= L.redu[i];
    sninf += L.redi[i];
  }
  // (LP) the slice's largest finite raw logit, the raw threshold and the
  // raw sum of exp(x - rsmax) (double, fixed order over the waves).  The
  // threshold is the smallest of the waves' c-th largest finite thread
  // maxima, c = ceil(LPo.k / 8): the waves' 8c largest are at or above it,
  // so at least LPo.k tokens are.
  float rsmax = kNegInf, rtau = kPosInf;
  if constexpr (LP) {
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      rsmax = __builtin_fmaxf(rsmax, L.rredf[i]);
      rtau = __builtin_fminf(rtau, L.rtop[i]);
    }
    double rz = 0.0;
    if (rsmax > kNegInf && nbr < __FLT_MAX__) {
      const float bh = rsmax * kLog2e;
      const float bl = __builtin_fmaf(rsmax, kLog2e, -bh);
      rz = (double)zr * (double)__builtin_amdgcn_exp2f((-nbr - bh) - bl);
    }
    rz = wave_sum(rz);
    if (l == 0) L.rredz[wv] = rz;
  }
  const bool posinf = smax == kPosInf;
  const bool has_finite = smax > kNegInf && !posinf;
  if (smax > kNegInf) sflags |= kFLive;
  if (posinf) sflags |= kFPosInf;
  if (ent_overflow) sflags |= kFEntOverflow;

  // the slice's mass sum exp((x - smax) / T_f), in 2^40 fixed point (exact in
  // any order: the entry table's order depends on atomics)
  uint64_t ze = 0ull;
  if (zon && has_finite) {
    const float nb = -smax * lgz;
    const float nb_err = __builtin_fmaf(-smax, lgz, -nb);
    const float enb = __builtin_amdgcn_exp2f(nb_err);
    for (int j = tid; j < n_ent; j += kThreads) {
      const float x = L.ex[j];
      if (x > kNegInf) ze += (uint64_t)(__builtin_amdgcn_exp2f(__builtin_fmaf(x, lgz, nb)) * enb * 0x1p40f);
    }
    const float bh = smax * lgz;
    const float bl = __builtin_fmaf(smax, lgz, -bh);
    const float zr = zref ? zt * __builtin_amdgcn_exp2f((-nbz - bh) - bl) : 0.0f;
    ze += zr < 0x1p20f ? (uint64_t)(zr * 0x1p40f) : 0ull;
  }
  ze = wave_sum(ze);
  if (l == 0) L.redz[wv] = ze;

  // ---------------------------------------------------------- E: threshold
  // candidates are the tokens x >= tc (x-space); tempered rows compare
  // fl(x / T), so a margin of 2^-20 keeps every token whose filter-space
  // value could tie with the k-th
  const float mp = prm.min_p > 1.0f ? 1.0f : prm.min_p;
  const bool m_on = c.kind == LSAMP_KIND_FILTERED && mp > 0.0f && !bad_row;
  auto margin = [&](float t) {
    if (!(t < kPosInf)) return t;  // +inf: exactly the +inf tokens
    const float tc = c.tempered ? t - (__builtin_fabsf(t) * 0x1p-20f + 1e-30f) : t;
    return __builtin_fmaxf(tc, -__FLT_MAX__);
  };
  // min-p: a kept token has y >= y_max + ln(min_p) >= y_smax + ln(min_p); in
  // x-space, with a hundredth of a nat to spare for the rounding of x / T
  const float tau_m = m_on ? smax + (float)c.tf * (__builtin_logf(mp) - 0.01f) : kNegInf;
  // the K-th largest thread maximum, from a histogram of the maxima within
  // dcap below the slice maximum hmax (half a bin of slack covers the bin
  // index's rounding); lo: the smallest thread maximum above -inf
  auto tau_hist = [&](float hmax, float lo, float mine, float dcap, int K) -> float {
    for (int i = tid; i < kTkTauBins; i += kThreads) L.hist[i] = 0u;
    __syncthreads();
    const float D = __builtin_fminf(hmax - lo, dcap);
    const float sc = D > 0.0f ? (float)(kTkTauBins - 1) / D : 0.0f;
    if (mine > kNegInf) {
      const float fb = (hmax - mine) * sc;
      const int b = fb < (float)(kTkTauBins - 1) ? (int)fb : kTkTauBins - 1;
      atomicAdd(&L.hist[b], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      constexpr int kPer = kTkTauBins / 64;
      uint32_t cb[kPer];
      uint32_t cs = 0u;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        cb[i] = L.hist[kPer * tid + i];
        cs += cb[i];
      }
      const uint32_t ic = wave_incl_scan(cs);
      const uint64_t hit = __ballot(ic >= (uint32_t)K);
      int bs = kTkTauBins;
      if (hit) {
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
    return bs >= kTkTauBins
               ? kNegInf
               : ((bs == kTkTauBins - 1 || sc == 0.0f) ? lo : hmax - ((float)bs + 1.5f) / sc);
  };

  // ---------------------------------------------------------- F: candidates
  // the tokens x >= t (and, after a radix select, key >= kmin) in L.cand as
  // raw (x, id) pairs (their keys are computed by the sort, in parallel);
  // L.ncand counts them all, kept or not
  auto extract = [&](float t, bool by_key, uint64_t kmin) {
    // the quads of the wave where some lane's quad maximum reaches t, then
    // one such quad at a time: a bitmask of its hits, a slot range for the
    // lanes with hits (one LDS atomic each)
    uint32_t sel = 0u;
#pragma unroll
    for (int g = 0; g < Q; ++g) {
      const uint32_t w = qmp[g / 2];
      const float qm = __uint_as_float(g & 1 ? w & 0xffff0000u : w << 16);
      if (__ballot(qm >= t) != 0ull) sel |= 1u << g;
    }
    for_quads_sel(S, sel, [&](int g, uint4& vq) -> bool {
      const int32_t i0 = base32 + (tid + g * kThreads) * N;
      uint4 v = vq;
      if constexpr (LP) exclude_elems<DT>(v, exb.get(g));  // (raw registers)
      uint32_t hits = 0u;
#pragma unroll
      for (int e = 0; e < N; ++e) hits |= (vec_elem<DT>(v, e) >= t ? 1u : 0u) << e;
      if (by_key) {
        uint32_t h2 = 0u;
        for (uint32_t h = hits; h; h &= h - 1u) {
          const int e = __builtin_ctz(h);
          if (elem_key(c, vec_elem_dyn<DT>(v, e), i0 + e) >= kmin) h2 |= 1u << e;
        }
        hits = h2;
      }
      if (hits) {
        int slot = atomicAdd(&L.ncand, __builtin_popcount(hits));
        for (uint32_t h = hits; h; h &= h - 1u, ++slot) {
          const int e = __builtin_ctz(h);
          if (slot < kCandCap) L.cand[slot] = raw_cand(vec_elem_dyn<DT>(v, e), i0 + e);
        }
      }
      return false;
    });
    for (int k0 = 0; k0 < n_ent; k0 += kThreads) {
      const int j = k0 + tid;
      const float x = j < n_ent ? L.ex[j] : kNegInf;
      bool hit = x >= t && x > kNegInf;
      if (by_key && hit) hit = elem_key(c, x, L.etok[j]) >= kmin;
      const int slot = wave_append(hit, &L.ncand);
      if (hit && slot < kCandCap) L.cand[slot] = raw_cand(x, L.etok[j]);
    }
  };

  // First threshold: +inf tokens, the maximum (k = 1), the min-p bound, or
  // the k-th largest thread maximum.  Too many candidates: the min-p bound
  // with the thread-maximum bound, then the exact k-th key.
  float t0;
  if (posinf) {
    t0 = kPosInf;
  } else if (K == 1) {
    t0 = smax;
  } else if (m_on) {
    t0 = tau_m;
  } else {
    t0 = tau_hist(smax, tlo, tmax, (float)(32.0 * c.tf), K);
  }
  float tc = margin(t0);
  bool by_key = false, hist_tried = !(m_on && !posinf && K > 1);
  uint64_t kmin = 0ull;
  int n = 0;
#pragma unroll 1
  for (int attempt = 0; attempt < 3; ++attempt) {
    if (smax > kNegInf) extract(tc, by_key, kmin);
    __syncthreads();
    n = L.ncand;
    if (n <= kCandCap) break;
    if (!hist_tried) {
      hist_tried = true;
      tc = margin(__builtin_fmaxf(tau_hist(smax, tlo, tmax, (float)(32.0 * c.tf), K), tau_m));
    } else {
      kmin = kth_key_mem<DT>(c, rowp, mrow, P.mask_words, P.mask_bits, P.mask_tail, base32,
                             end32, n_ent, tc, K, L);
      by_key = true;
    }
    if (tid == 0) L.ncand = 0;
    __syncthreads();
  }
  if (n > kCandCap) n = kCandCap;  // (cannot happen: the select leaves K)

  // ---------------------------------------------------------- G: sort
  // rank of a key = the keys above it (keys are distinct: ids are); the
  // comparisons of a key are split over `parts` threads.  The n raw pairs in
  // L.cand become keys (keyof); the best npub go to dst in order.
  // (src: the candidates, ranks accumulated in racc, which starts at zero)
  // (wide: the comparisons split over every thread even for a wave's worth)
  auto sort_into = [&](int n, int npub, uint64_t* dst, auto keyof, uint64_t* src,
                       int32_t* racc, bool wide) {
    if (n > 0 && n <= 64 && !wide) {
      // a wave's worth: lane i turns candidate i into its key, then ranks it
      // against all of them (broadcast reads, eight at a time), no atomics
      if (tid < 64) {
        const uint64_t key = tid < n ? keyof(src[tid]) : 0ull;
        if (tid < n) src[tid] = key;
        __builtin_amdgcn_wave_barrier();
        int r = 0;
        for (int j0 = 0; j0 < n; j0 += 8) {
          uint64_t cj[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) cj[q] = src[j0 + q];
#pragma unroll
          for (int q = 0; q < 8; ++q) r += (j0 + q < n && cj[q] > key) ? 1 : 0;
        }
        if (tid < n && r < npub) dst[r] = key;
      }
    } else if (n > 0) {
      for (int i = tid; i < n; i += kThreads) src[i] = keyof(src[i]);
      __syncthreads();
      const int parts = n <= kThreads / 2 ? kThreads / n : 1;
      if (parts > 1) {
        const int i = tid % n, part = tid / n;
        if (part < parts) {
          const uint64_t key = src[i];
          const int j0 = (n * part) / parts, j1 = (n * (part + 1)) / parts;
          int r = 0;
          for (int j = j0; j < j1; ++j) r += src[j] > key ? 1 : 0;
          if (r) atomicAdd(&racc[i], r);
        }
        __syncthreads();
        for (int i2 = tid; i2 < n; i2 += kThreads) {
          const int r = racc[i2];
          if (r < npub) dst[r] = src[i2];
        }
      } else {
        for (int i = tid; i < n; i += kThreads) {
          const uint64_t key = src[i];
          int r = 0;
          for (int j = 0; j < n; ++j) r += src[j] > key ? 1 : 0;
          if (r < npub) dst[r] = key;
        }
      }
    }
  };
  const int npub = n < K ? n : K;
  uint64_t* mine = L.best + slice * kTopkMaxK;
  sort_into(n, npub, mine, [&](uint64_t r) { return cand_key_of(c, r); }, L.cand, L.racc, false);

  // ---------------------------------------------------------- payload words
  if (tid == 0) {
    L.tag = epoch + 1u;
    L.last = ticket + 1u == (uint32_t)G ? 1 : 0;
  }
  uint64_t zs = 0ull;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) zs += L.redz[i];
  const double zsum = (double)zs * 0x1p-40;
  int nraw = 0;  // (LP) the slice's raw keys, sorted in rbest
  double rzs = 0.0;
  if constexpr (LP) {
#pragma unroll
    for (int i = 0; i < kWaves; ++i) rzs += L.rredz[i];
  }
  auto word = [&](int w) -> uint32_t {
    if (LP && w >= kTopkWordsBase) {
      const int p = (w - kTopkWordsBase) >> 1;
      if (p >= nraw) return 0u;
      const uint64_t key = L.rbest[slice * kTopkMaxLp + p];
      return (w - kTopkWordsBase) & 1 ? (uint32_t)key : (uint32_t)(key >> 32);
    }
    if (w >= kTopkHead) {
      const int p = (w - kTopkHead) >> 1;
      if (p >= npub) return 0u;
      const uint64_t key = mine[p];
      return (w - kTopkHead) & 1 ? (uint32_t)key : (uint32_t)(key >> 32);
    }
    const uint64_t zb = __builtin_bit_cast(uint64_t, zsum);
    switch (w) {
      case kHMax: return __float_as_uint(smax);
      case kHZHi: return (uint32_t)(zb >> 32);
      case kHZLo: return (uint32_t)zb;
      case kHNpub: return (uint32_t)npub;
      case kHFlags: return sflags;
      case kHNinf: return (uint32_t)sninf;
      case kHRMax: return LP ? __float_as_uint(rsmax) : 0u;
      case kHRZ: return LP ? __float_as_uint((float)rzs) : 0u;
      default: return 0u;
    }
  };
  uint64_t* const pub = T.pub + ((size_t)row * kMaxSlices + slice) * kTopkWords;
  // (LP with raw keys) the slice's payload, which the draw needs, goes out
  // before its raw keys are ranked; with keep bytes requested it waits for
  // them (the finalizer marks kept tokens once every slice cleared its range)
  const bool early = LP && LPo.k > 0 && !P.keep;

  // ---------------------------------------------------------- raw top-k (LP)
  // The slice's best LPo.k raw keys: the tokens at or above the LPo.k-th
  // largest raw thread maximum (gated by the raw quad maxima); a slice with
  // +inf, or whose threshold leaves too few or too many, takes the exact
  // select over memory.
  if constexpr (LP) {
    const int Kr = LPo.k;
    if (Kr > 0) {
      const bool rfin = (sflags & kFRawPosInf) == 0u;
      const float tr = rfin ? rtau : kNegInf;
      if (tr > kNegInf) {
        // the quads whose raw maximum reaches tr are staged in LDS (the
        // thread's qualifying quads, one slot range a wave: a scan of the
        // counts and one LDS atomic), while wave 0 may still be sorting the
        // slice's keys; then all threads scan the staged elements
        uint32_t qsel = 0u;
#pragma unroll
        for (int g = 0; g < Q; ++g) {
          const uint32_t w = rqp[g / 2];
          const float rq = __uint_as_float(g & 1 ? w & 0xffff0000u : w << 16);
          qsel |= (g < nq && rq >= tr ? 1u : 0u) << g;
        }
        const uint32_t qc = (uint32_t)__builtin_popcount(qsel);
        const uint32_t qi = wave_incl_scan(qc);
        const uint32_t qt = read_lane(qi, 63);
        int qb = 0;
        if (l == 0 && qt) qb = atomicAdd(&L.nstage, (int)qt);
        int slot = read_lane(qb, 0) + (int)(qi - qc);
#pragma unroll
        for (int g = 0; g < Q; ++g) {
          if ((qsel >> g) & 1u) {
            if (slot < kRStageCap) {
              const uint4 qv = quad_get(S.bank[g / kQuadsPerBank], g % kQuadsPerBank);
              L.rstage[4 * slot] = qv.x;
              L.rstage[4 * slot + 1] = qv.y;
              L.rstage[4 * slot + 2] = qv.z;
              L.rstage[4 * slot + 3] = qv.w;
              L.rstage_at[slot] = base32 + (tid + g * kThreads) * N;
            }
            ++slot;
          }
        }
      }
      __syncthreads();  // staged (and the slice's keys are sorted)
      if (early && L.last == 0 && tid < kTopkWordsBase)
        st_coherent(&pub[tid], ((uint64_t)L.tag << 32) | word(tid));
      int nr = 0;
      if (tr > kNegInf) {
        const int ns = L.nstage;
        if (ns <= kRStageCap) {
          for (int j = tid; j < ns * N; j += kThreads) {
            const int q = j / N, e = j - q * N;
            const uint32_t w = L.rstage[4 * q + e * 4 / N];
            float x;
            if constexpr (DT == LSAMP_DTYPE_F32)
              x = __uint_as_float(w);
            else if constexpr (DT == LSAMP_DTYPE_BF16)
              x = __uint_as_float((e & 1) ? w & 0xffff0000u : w << 16);
            else
              x = half_bits_to_f32((e & 1) ? w >> 16 : w & 0xffffu);
            const int32_t id = L.rstage_at[q] + e;
            const bool hit = x >= tr && id < end32;
            const int cs = wave_append(hit, &L.nrcand);
            if (hit && cs < kRCandCap) L.rcand[cs] = raw_cand(x, id);
          }
        }
        __syncthreads();
        nr = ns <= kRStageCap ? L.nrcand : kRCandCap + 1;
      }
      if (nr < Kr || nr > kRCandCap) {
        __syncthreads();  // every thread has read the counts
        nr = raw_select_mem<DT>(rowp, base32, end32, Kr, L.rcand, &L.nrcand, L);
      }
      // the slice's best min(k, n) raw keys in order (the comparisons split
      // over every thread: a wave alone is a long dependent chain)
      nraw = nr < Kr ? nr : Kr;
      sort_into(nr, nraw, L.rbest + slice * kTopkMaxLp, [](uint64_t r) { return raw_key_of(r); },
                L.rcand, L.rracc, true);
    }
  }

  // ---------------------------------------------------------- parity outputs
  if (P.processed) {
    float* out = P.processed + (size_t)row * (size_t)V;
    for_quads(S, nq, [&](int g, uint4& vq) -> bool {
      const int32_t i0 = base32 + (tid + g * kThreads) * N;
      if (i0 >= end32) return false;
      uint4 v = vq;
      if constexpr (LP) exclude_elems<DT>(v, exb.get(g));
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
  if (P.keep) {
    // the slice's keep bytes: a sampled row whose maximum is +inf keeps
    // exactly its +inf tokens (each slice marks its own); otherwise the
    // finalizer marks the kept tokens after every slice has cleared its range
    uint8_t* kr = P.keep + (size_t)row * (size_t)V;
    const bool inf_keep = posinf && c.kind == LSAMP_KIND_FILTERED && !bad_row;
    for_quads(S, nq, [&](int g, uint4& vq) -> bool {
      const int32_t i0 = base32 + (tid + g * kThreads) * N;
      uint4 v = vq;
      if constexpr (LP) exclude_elems<DT>(v, exb.get(g));
#pragma unroll
      for (int e = 0; e < N; ++e)
        if (i0 + e < end32) kr[i0 + e] = (inf_keep && vec_elem<DT>(v, e) == kPosInf) ? 1 : 0;
      return false;
    });
    __syncthreads();
    if (inf_keep)
      for (int j = tid; j < n_ent; j += kThreads)
        if (L.ex[j] == kPosInf) kr[L.etok[j]] = 1;
    drain_memory();  // these bytes land before the payload says the slice is done
  }

  // ---------------------------------------------------------- H: publish
  __syncthreads();
  const uint32_t tag = L.tag;
  const bool last = L.last != 0;
  if (!last) {
    // the payload (unless it went out early) and the raw keys
    const int w0 = early ? kTopkWordsBase : 0;
    const int w1 = LP && LPo.k > 0 ? kTopkWordsBase + 2 * nraw : kTopkWordsBase;
    if (tid >= w0 && tid < w1) st_coherent(&pub[tid], ((uint64_t)tag << 32) | word(tid));
    return;
  }

  // ---------------------------------------------------------- I: finalize
  // the row's draw inputs, requested first: they arrive while the other
  // slices' payloads are polled for
  const float u_in = P.uniforms ? gmem(P.uniforms)[row] : 0.0f;
  const uint64_t key_in = (!P.uniforms && P.philox_keys) ? gmem(P.philox_keys)[row] : 0ull;
  const int32_t probe = P.probe_tokens ? gmem(P.probe_tokens)[row] : -1;
  const int32_t spin_test =
      __hip_atomic_load(&g_topk_spin_test, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // this slice's header; the others' words, polled until tagged with this
  // step (their slices started before this one, so each finishes)
  if (tid < kTopkHead) {
    const uint32_t w = word(tid);
    switch (tid) {
      case kHMax: L.hmax[slice] = __uint_as_float(w); break;
      case kHNpub: L.hnpub[slice] = (int32_t)w; break;
      case kHFlags: L.hflags[slice] = w; break;
      case kHNinf: L.hninf[slice] = (int32_t)w; break;
      case kHRMax: L.hrmax[slice] = __uint_as_float(w); break;
      case kHRZ: L.hrz[slice] = __uint_as_float(w); break;
      default: break;
    }
  }
  if (tid == 0) L.hz[slice] = zsum;
  if (tid < kTopkWordsBase) {
    // every slice's word in one round trip, then only the missing ones again
    const uint64_t* pub0 = T.pub + (size_t)row * kMaxSlices * kTopkWords + tid;
    uint64_t w8[kMaxSlices];
#pragma unroll
    for (int s = 0; s < kMaxSlices; ++s)
      w8[s] = (s < G && s != slice) ? ld_coherent(pub0 + s * kTopkWords) : ((uint64_t)tag << 32);
    const int lim = spin_test > 0 ? spin_test : kSpin;
    for (int it = 0;; ++it) {
      bool all = spin_test <= 0;
#pragma unroll
      for (int s = 0; s < kMaxSlices; ++s) all = all && (uint32_t)(w8[s] >> 32) == tag;
      if (all) break;
      if (it >= lim) {
        L.lost = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int s = 0; s < kMaxSlices; ++s)
        if ((uint32_t)(w8[s] >> 32) != tag) w8[s] = ld_coherent(pub0 + s * kTopkWords);
    }
    for (int s = 0; s < G; ++s) {
      if (s == slice) continue;
      const uint32_t d = (uint32_t)w8[s];
      if (tid >= kTopkHead) {
        const int p = (tid - kTopkHead) >> 1;
        uint32_t* half = reinterpret_cast<uint32_t*>(&L.best[s * kTopkMaxK + p]);
        half[(tid - kTopkHead) & 1 ? 0 : 1] = d;
      } else if (tid == kHMax) {
        L.hmax[s] = __uint_as_float(d);
      } else if (tid == kHZHi) {
        reinterpret_cast<uint32_t*>(&L.hz[s])[1] = d;
      } else if (tid == kHZLo) {
        reinterpret_cast<uint32_t*>(&L.hz[s])[0] = d;
      } else if (tid == kHNpub) {
        // (clamped: a slice given up on leaves an old word)
        L.hnpub[s] = d < (uint32_t)kTopkMaxK ? (int32_t)d : kTopkMaxK;
      } else if (tid == kHFlags) {
        L.hflags[s] = d;
      } else if (tid == kHNinf) {
        L.hninf[s] = (int32_t)d;
      } else if (LP && tid == kHRMax) {
        L.hrmax[s] = __uint_as_float(d);
      } else if (LP && tid == kHRZ) {
        L.hrz[s] = __uint_as_float(d);
      }
    }
  }
  __syncthreads();
  // The row's header totals, every lane from the slices' headers (broadcast
  // reads, no cross-lane steps).
  // (unrolled, every header read unconditionally and masked, so that the
  // reads go out together and one wait covers them)
  int total = 0;
  float row_max = kNegInf;
  uint32_t rfl = 0u;
  int32_t ninf_row = 0;
  int npub_s[kMaxSlices];
#pragma unroll
  for (int s = 0; s < kMaxSlices; ++s) {
    const bool in = s < G;
    const uint32_t f = in ? L.hflags[s] : 0u;
    const float hx = L.hmax[s];
    npub_s[s] = in ? L.hnpub[s] : 0;
    rfl |= f;
    row_max = __builtin_fmaxf(row_max, (f & kFLive) ? hx : kNegInf);
    total += npub_s[s];
    ninf_row += in ? L.hninf[s] : 0;
  }
  // (LP) The row's raw log-sum-exp from the slices' raw headers (NaN when a
  // logit is NaN, +inf when one is +inf, -inf when all are -inf); every
  // thread computes it.
  double lse = 0.0;
  if constexpr (LP) {
    float mx = kNegInf;
    uint32_t rf = 0u;
#pragma unroll
    for (int s = 0; s < kMaxSlices; ++s) {
      const bool in = s < G;
      rf |= in ? L.hflags[s] : 0u;
      mx = __builtin_fmaxf(mx, in ? L.hrmax[s] : kNegInf);
    }
    if (rf & kFRawNaN) {
      lse = __builtin_nan("");
    } else if (rf & kFRawPosInf) {
      lse = __builtin_huge_val();
    } else if (mx == kNegInf) {
      lse = -__builtin_huge_val();
    } else {
      double z = 0.0;
#pragma unroll
      for (int s = 0; s < kMaxSlices; ++s) {
        const float hx = L.hrmax[s];
        z += (s < G && hx > kNegInf)
                 ? (double)L.hrz[s] * (double)__builtin_amdgcn_exp2f((hx - mx) * kLog2e)
                 : 0.0;
      }
      lse = (double)mx + (double)__builtin_logf((float)z);
    }
  }
  // (LP) The raw keys, by waves 1..4 once the row's keys are merged, while
  // wave 0 draws: each of those waves reads every other slice's raw list
  // (lane l polls word l; each slice lists min(k, its length) keys, sorted;
  // the waves store the same values), then each lane ranks the key of one
  // list slot by counting the keys above it; the ranks below k write their
  // outputs.  A list given up on (bounded
  // polls) leaves the row's raw outputs NaN / -1 and raises the sticky
  // status bit.
  auto raw_merge = [&]() {
    const int Kr = LPo.k;
    if (Kr > 0 && wv >= 1 && wv <= kMaxSlices * kTopkMaxLp / 64) {
      int nr_s[kMaxSlices];
#pragma unroll
      for (int s = 0; s < kMaxSlices; ++s) {
        const int64_t len = s == G - 1 ? V - (int64_t)s * P.slice_len : (int64_t)P.slice_len;
        nr_s[s] = s < G ? (len < Kr ? (int)len : Kr) : 0;
      }
      const uint64_t* praw = T.pub + (size_t)row * kMaxSlices * kTopkWords + kTopkWordsBase + l;
      uint64_t w8[kMaxSlices];
      bool want[kMaxSlices];
#pragma unroll
      for (int s = 0; s < kMaxSlices; ++s) {
        want[s] = s < G && s != slice && l < 2 * nr_s[s];
        w8[s] = want[s] ? ld_coherent(praw + s * kTopkWords) : ((uint64_t)tag << 32);
      }
      const int lim = spin_test > 0 ? spin_test : kSpin;
      bool rlost = false;
      for (int it = 0;; ++it) {
        bool all = spin_test <= 0;
#pragma unroll
        for (int s = 0; s < kMaxSlices; ++s) all = all && (uint32_t)(w8[s] >> 32) == tag;
        if (all) break;
        if (it >= lim) {
          rlost = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int s = 0; s < kMaxSlices; ++s)
          if ((uint32_t)(w8[s] >> 32) != tag) w8[s] = ld_coherent(praw + s * kTopkWords);
      }
#pragma unroll
      for (int s = 0; s < kMaxSlices; ++s) {
        if (want[s]) {
          uint32_t* half = reinterpret_cast<uint32_t*>(&L.rbest[s * kTopkMaxLp + (l >> 1)]);
          half[l & 1 ? 0 : 1] = (uint32_t)w8[s];
        }
      }
      const bool gone = __ballot(rlost) != 0ull || L.lost != 0;
      if (gone && wv == 1 && l == 0) atomicOr(T.status, kStatusSpinTimeout);
      __builtin_amdgcn_wave_barrier();
      // this lane's list slot j, ranked by counting the keys above it in
      // every list (broadcast reads, eight at a time)
      const int j = (wv - 1) * 64 + l, sj = j / kTopkMaxLp, pj = j - sj * kTopkMaxLp;
      if (sj < G && pj < nr_s[sj]) {
        const uint64_t key = L.rbest[j];
        int r = 0;
        for (int s2 = 0; s2 < G; ++s2) {
          const uint64_t* lst = L.rbest + s2 * kTopkMaxLp;
          for (int p0 = 0; p0 < nr_s[s2]; p0 += 8) {
            uint64_t kj[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) kj[q] = lst[p0 + q];
#pragma unroll
            for (int q = 0; q < 8; ++q) r += (p0 + q < nr_s[s2] && kj[q] > key) ? 1 : 0;
          }
        }
        if (r < Kr) {
          // a row whose log-sum-exp is not finite fails closed, as a list
          // given up on does (CBv2NonFiniteLogits.swift:8-34)
          const bool closed = gone || !__builtin_isfinite(lse);
          const size_t o = (size_t)row * (size_t)Kr + (size_t)r;
          LPo.ids[o] = closed ? -1 : key_id(key);
          LPo.values[o] = closed ? __builtin_nanf("") : (float)((double)key_y(key) - lse);
        }
      }
    }
  };
  // The row's best keys in order, in L.merged.  At most 64 keys in all
  // (every slice's list short, as min-p makes them): one wave ranks them.
  // More: each slice's wave counts, for each of its keys, the keys above it
  // in the other slices' sorted lists (binary searches).
  static_assert(kTopkMaxK == 64, "one wave per slice list");
  if (total <= 64) {
    if (tid >= 64) {
      if constexpr (LP) raw_merge();
      if (tid == 64) {
        gmem(T.ticket)[row] = 0u;
        gmem(T.epoch)[row] = tag;
      }
      return;
    }
    // lane l's candidate: the l-th key of the lists laid end to end; its
    // rank is the number of keys above it (compares against all of them,
    // broadcast reads eight at a time), and it moves to that position
    int sl = 0, pl = l;
#pragma unroll
    for (int s = 0; s < kMaxSlices; ++s) {
      if (pl >= npub_s[s] && sl == s) {
        pl -= npub_s[s];
        sl = s + 1;
      }
    }
    const uint64_t key = l < total ? L.best[sl * kTopkMaxK + pl] : 0ull;
    L.cand[l] = key;
    __builtin_amdgcn_wave_barrier();
    int rk = 0;
    for (int j0 = 0; j0 < total; j0 += 8) {
      uint64_t kj[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) kj[q] = L.cand[j0 + q];
#pragma unroll
      for (int q = 0; q < 8; ++q) rk += (j0 + q < total && kj[q] > key) ? 1 : 0;
    }
    if (l < total) L.merged[rk] = key;
    __builtin_amdgcn_wave_barrier();
  } else {
    const int s = __builtin_amdgcn_readfirstlane(tid) >> 6, p = l;
    if (s < G && p < L.hnpub[s]) {
      const uint64_t key = L.best[s * kTopkMaxK + p];
      int r = p;
      for (int s2 = 0; s2 < G; ++s2) {
        if (s2 == s) continue;
        const uint64_t* lst = L.best + s2 * kTopkMaxK;
        int lo = 0, hi = L.hnpub[s2];
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (lst[mid] > key) lo = mid + 1; else hi = mid;
        }
        r += lo;
      }
      if (r < kTopkMaxK) L.merged[r] = key;
    }
    __syncthreads();
    if (tid >= 64) {
      if constexpr (LP) raw_merge();
      if (tid == 64) {
        gmem(T.ticket)[row] = 0u;
        gmem(T.epoch)[row] = tag;
      }
      return;
    }
  }

  // ---------------------------------------------------------- J: the row
  // the row's mass relative to its maximum (each slice's mass is relative to
  // its own maximum)
  double z = 0.0;
  if (c.kind != LSAMP_KIND_ARGMAX && row_max > kNegInf && row_max < kPosInf) {
#pragma unroll
    for (int s = 0; s < kMaxSlices; ++s) {
      const float hx = L.hmax[s];
      const double hz = L.hz[s];
      const bool live = s < G && (L.hflags[s] & kFLive) && hx > kNegInf;
      z += live ? hz * (double)__builtin_amdgcn_exp2f((hx - row_max) * lgz) : 0.0;
    }
  }
  const bool any = (rfl & kFLive) != 0u;
  const bool lost = L.lost != 0;
  uint32_t flags = (rfl & kFNonfinite) ? LSAMP_ROW_NONFINITE : 0u;
  float u = u_in;
  if (!P.uniforms && P.philox_keys) u = philox_uniform(key_in, 0u);
  uint8_t* kr = P.keep ? P.keep + (size_t)row * (size_t)V : nullptr;

  int32_t token = -1;
  float cx = 0.0f;      // (LP) the chosen token's raw logit
  bool cx_ok = false;
  uint64_t W = 0ull, probe_w = 0ull;
  int32_t kept_c = 0;
  float cmin = kPosInf;
  double cent = 0.0;
  float y_max = any ? to_filter(c, row_max) : 0.0f;
  const bool inf_mode = any && row_max == kPosInf && c.kind == LSAMP_KIND_FILTERED;
  if (lost) {
    flags |= LSAMP_ROW_TIMEOUT;
  } else if (bad_row || (rfl & kFEntOverflow)) {
    flags |= LSAMP_ROW_OVERFLOW;
  } else if (!any) {
    flags |= LSAMP_ROW_EMPTY;
  } else if (inf_mode) {
    // the +inf tokens, equally weighted: the token at index (U n) >> 32 of
    // the row's +inf tokens in id order; each slice listed its first ones
    y_max = kPosInf;
    W = (uint64_t)ninf_row << 40;
    const uint64_t j = ((uint64_t)uniform_u32(u) * (uint64_t)ninf_row) >> 32;
    int64_t pre = 0;
    int32_t tk = -1;
    bool beyond = false;
    for (int s = 0; s < G; ++s) {
      const int64_t ns = L.hninf[s];
      if ((int64_t)j < pre + ns) {
        const int jj = (int)((int64_t)j - pre);
        if (jj < L.hnpub[s]) tk = key_id(L.best[s * kTopkMaxK + jj]);
        else beyond = true;
        break;
      }
      pre += ns;
    }
    if (beyond) {
      // more +inf tokens in one slice than it lists: fail closed
      flags |= LSAMP_ROW_OVERFLOW;
      W = 0ull;
    } else {
      token = tk;
      kept_c = ninf_row;
      cmin = kPosInf;
      cent = 0.0;
    }
  } else {
    // the keep rule over the row's best keys (CBv2: rank < k, exclusive mass
    // <= top-p of the total, p >= min-p of the top; argmax rows: the first)
    const int nc = total < K ? total : K;
    const bool in = l < nc;
    const uint64_t key = in ? L.merged[l] : 0ull;
    const float y = key_y(key);
    const int32_t id = key_id(key);
    // (LP) each listed token's raw logit, requested now, read after the draw
    const float rawx = LP && in ? load_scalar<DT>(rowp, id) : 0.0f;
    const double P_lim = top_p_limit(P, c, prm, z);
    const bool p_on = P_lim >= 0.0;
    const int32_t k_lim = c.kind == LSAMP_KIND_ARGMAX ? 1 : prm.top_k;
    const double e = in ? (double)__builtin_expf(y - y_max) : 0.0;
    const double e_excl = wave_incl_scan(e) - e;
    bool keep_p = true, keep_m = true;
    if (p_on) keep_p = e_excl <= P_lim;
    if (m_on) keep_m = __builtin_expf(y - y_max) >= mp;
    if (l >= k_lim) keep_p = false;
    const bool keep = in && keep_p && keep_m;
    kept_c = (int32_t)__popcll(__ballot(keep));  // each rule keeps a prefix
    const uint64_t w = keep ? weight(y, y_max, c.scale) : 0ull;
    // the kept in id order, then a running sum: the token is the one whose
    // run crosses the target
    uint64_t* dw = L.cand;                              // [64] weights by id rank
    int32_t* sid = reinterpret_cast<int32_t*>(L.racc);  // [64] kept ids, then by id rank
    if (keep) sid[l] = id;
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
    int32_t* sid2 = sid + 64;
    if (keep) {
      dw[pos] = w;
      sid2[pos] = id;
    }
    __builtin_amdgcn_wave_barrier();
    const uint64_t wo = l < kept_c ? dw[l] : 0ull;
    const int32_t io = l < kept_c ? sid2[l] : -1;
    const uint64_t cum = wave_incl_scan(wo);
    W = read_lane(cum, 63);
    const uint64_t target = W ? scaled_target(uniform_u32(u), W) : 0ull;
    const uint64_t hm = __ballot(wo != 0ull && cum > target && cum - wo <= target);
    token = hm ? read_lane(io, __builtin_ctzll(hm)) : -1;
    if constexpr (LP) {
      const uint64_t hc = __ballot(in && id == token);
      if (hc) {
        cx = read_lane(rawx, __builtin_ctzll(hc));
        cx_ok = true;
      }
    }
    const uint64_t hp = __ballot(keep && probe >= 0 && id == probe);
    probe_w = hp ? read_lane(w, __builtin_ctzll(hp)) : 0ull;
    if (P.stats) {
      cent = wave_sum(keep ? (double)w * (1.0 / 1099511627776.0) * (double)weight_arg(y, y_max, c.scale)
                           : 0.0);
      cmin = wave_min(keep ? y : kPosInf);
    }
    if (kr && in && keep) kr[id] = 1;
    if (token < 0 || W == 0ull) flags |= LSAMP_ROW_EMPTY;
  }
  if constexpr (LP) {
    if (token >= 0 && !cx_ok) cx = load_scalar<DT>(rowp, token);
    if (l == 0)
      LPo.chosen[row] = token >= 0 && __builtin_isfinite(lse) ? (float)((double)cx - lse)
                                                              : __builtin_nanf("");
  }
  if (l == 0) {
    if (lost) atomicOr(T.status, kStatusSpinTimeout);
    gmem(P.tokens)[row] = token;
    if (P.row_flags) gmem(P.row_flags)[row] = flags;
    if (P.stats) {
      lsamp_row_stats st;
      st.max_value = y_max;
      st.log_normalizer = z > 0.0 ? __builtin_logf((float)z) : 0.0f;
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
  }
}

template <int DT, bool LP>
__global__ __launch_bounds__(kThreads) void k_topk(SamplePlan Pk, TopkWs Tk, TopkLp Lk) {
  __shared__ TopkLds L;
  const SamplePlan& P = Pk;
  const TopkWs& T = Tk;
  // work-group b runs on XCD b % 8; that XCD's rows are b % 8, + 8, + 16, ...
  const int b = (int)blockIdx.x;
  const int loc = b >> 3;
  const int row = (b & 7) + 8 * (loc / P.slices);
  const int slice = loc % P.slices;
  if (row < P.rows) topk_task<DT, LP>(P, T, Lk, row, slice, L);
}

template <int DT>
int launch_topk_dt(const SamplePlan& P, const TopkWs& T, const TopkLp& lp, hipStream_t st,
                   void* const* events) {
  auto mark = [&](int i) {
    if (events) (void)hipEventRecord(reinterpret_cast<hipEvent_t>(events[i]), st);
  };
  const int rows8 = (P.rows + 7) / 8 * 8;
  const dim3 grid((unsigned)(rows8 * P.slices));
  mark(0);
  // (raw log-probabilities in the same pass for 16-bit logits only: the fp32
  // slab leaves no registers for them, and lsamp_step then ranks the raw
  // logits in a second pass)
  if constexpr (DT != LSAMP_DTYPE_F32) {
    if (lp.k >= 0)
      hipLaunchKernelGGL((k_topk<DT, true>), grid, dim3(kThreads), 0, st, P, T, lp);
    else
      hipLaunchKernelGGL((k_topk<DT, false>), grid, dim3(kThreads), 0, st, P, T, lp);
  } else {
    hipLaunchKernelGGL((k_topk<DT, false>), grid, dim3(kThreads), 0, st, P, T, lp);
  }
  mark(1);
  mark(2);
  return (int)hipGetLastError();
}

template <int DT>
int topk_blocks_dt() {
  int n = 0;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_topk<DT, false>, kThreads, 0) ==
                 hipSuccess
             ? n
             : 0;
}

}  // namespace

int launch_topk(const SamplePlan& P, const TopkWs& T, const TopkLp& lp, void* stream,
                void* const* events) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (P.dtype) {
    case LSAMP_DTYPE_F32: return launch_topk_dt<LSAMP_DTYPE_F32>(P, T, lp, st, events);
    case LSAMP_DTYPE_BF16: return launch_topk_dt<LSAMP_DTYPE_BF16>(P, T, lp, st, events);
    default: return launch_topk_dt<LSAMP_DTYPE_F16>(P, T, lp, st, events);
  }
}

int set_topk_spin_test(int32_t polls) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_topk_spin_test), &polls, sizeof polls, 0,
                                hipMemcpyHostToDevice);
}

int topk_blocks_per_cu(int dtype) {
  switch (dtype) {
    case LSAMP_DTYPE_F32: return topk_blocks_dt<LSAMP_DTYPE_F32>();
    case LSAMP_DTYPE_BF16: return topk_blocks_dt<LSAMP_DTYPE_BF16>();
    default: return topk_blocks_dt<LSAMP_DTYPE_F16>();
  }
}

}  // namespace lsamp
