// lsamp_rank.hip — exact top-k of raw logits and their log-probabilities.
//
// The order is the one of the reference's shared top-2 reduction
// (Libraries/MLXLMCommon/ContinuousBatchingV2/CBv2TopTwo.swift:29-47): value
// descending, token id ascending on exact ties (+0 and -0 tie), NaNs last.
// Every token gets a 64-bit sort key with that order: the high word orders
// the value (0 for NaN, 0x80000000 +- magnitude bits otherwise), the low word
// is ~id.  Keys are distinct, so "the k largest keys" is the answer.
//
// One 512-thread work-group owns one slice of one row and keeps the slice's
// logits in registers (one pass over HBM):
//   1. each thread takes its largest key (and, for log-probabilities, the
//      sum of exp(x - m) over its logits, m its largest non-NaN logit);
//   2. tau = the k-th largest of the 512 thread maxima: a rank inside each
//      wave (a count over the wave's 64 maxima in LDS), then a rank in the 8
//      sorted wave lists (binary searches);
//   3. every key >= tau is a candidate: they include the slice's top k (the k
//      threads at or above tau hold k distinct keys >= tau) and come from k
//      threads only, so there are at most k * (tokens per thread).  Those
//      threads copy their logits to LDS and all threads scan the copies;
//   4. each candidate's rank is its count of larger candidates; the k best
//      go to the row's slice record with the log-sum-exp partial.
// The last work-group of the row to arrive merges the slice records (a rank
// by binary search in the sorted lists) and writes ids, values (the sort key
// carries the value) and the chosen token's log-probability (its logit
// travels in the record of the slice that holds it).
//
// Work that only the few waves holding the candidates would run (unrolled
// passes over their registers) is a long dependent chain with nothing to
// overlap it, so the once-per-slice steps spread their work over all the
// threads through LDS.
#include <hip/hip_runtime.h>

#include "lsamp_device.h"
#include "lsamp_internal.h"

namespace lsamp {
namespace {

using namespace dev;

template <int DT>
struct RankBits {
  static constexpr int W = DT == LSAMP_DTYPE_F32 ? 32 : 16;  // bits per logit
  static constexpr uint32_t MAG = W == 32 ? 0x7fffffffu : 0x7fffu;
  static constexpr uint32_t SIGN = W == 32 ? 0x80000000u : 0x8000u;
  static constexpr uint32_t ZERO = SIGN;  // key of +0 and -0
  static constexpr uint32_t INF =
      DT == LSAMP_DTYPE_F32 ? 0x7f800000u : (DT == LSAMP_DTYPE_BF16 ? 0x7f80u : 0x7c00u);
  static constexpr int N = Vec<DT>::N;  // logits per 16-byte vector
};

// Order key of a logit's bits that are not NaN: ZERO + magnitude for a
// non-negative value, ZERO - magnitude for a negative one (>= 1 for -inf).
template <int DT>
__device__ __forceinline__ uint32_t key_nn(uint32_t b) {
  using B = RankBits<DT>;
  const uint32_t mag = b & B::MAG;
  const uint32_t s = (uint32_t)((int32_t)(b << (32 - B::W)) >> 31);
  return B::ZERO + ((mag ^ s) - s);
}
// Same with NaN -> 0.
template <int DT>
__device__ __forceinline__ uint32_t key_of(uint32_t b) {
  return (b & RankBits<DT>::MAG) > RankBits<DT>::INF ? 0u : key_nn<DT>(b);
}
__device__ __forceinline__ float bits_value_f(uint32_t b, int dt) {
  if (dt == LSAMP_DTYPE_F32) return __uint_as_float(b);
  if (dt == LSAMP_DTYPE_BF16) return __uint_as_float(b << 16);
  return half_bits_to_f32(b);
}
template <int DT>
__device__ __forceinline__ float bits_value(uint32_t b) {
  return bits_value_f(b, DT);
}
// Logit value of a non-zero key.
template <int DT>
__device__ __forceinline__ float key_value(uint32_t key) {
  using B = RankBits<DT>;
  const uint32_t b = key >= B::ZERO ? key - B::ZERO : (B::ZERO - key) | B::SIGN;
  return bits_value<DT>(b);
}
// Bits of element e of a 16-byte vector.
template <int DT>
__device__ __forceinline__ uint32_t elem_bits(const uint4& r, int e) {
  if constexpr (DT == LSAMP_DTYPE_F32) {
    return e == 0 ? r.x : (e == 1 ? r.y : (e == 2 ? r.z : r.w));
  } else {
    const int q = e >> 1;
    const uint32_t w = q == 0 ? r.x : (q == 1 ? r.y : (q == 2 ? r.z : r.w));
    return (e & 1) ? w >> 16 : w & 0xffffu;
  }
}

// A thread's best (key, position): for 16-bit logits key << 16 | (0xffff -
// position), for fp32 key << 32 | (0xffffffff - position); the position
// (vector * N + element) grows with the token id, so the largest packed value
// is the thread's largest key at its lowest id.  0 = no token.
template <int DT>
struct Best {
  using T = typename std::conditional<DT == LSAMP_DTYPE_F32, uint64_t, uint32_t>::type;
  static constexpr int SHIFT = DT == LSAMP_DTYPE_F32 ? 32 : 16;
  static constexpr T LOW = DT == LSAMP_DTYPE_F32 ? 0xffffffffull : 0xffffu;
  static __device__ __forceinline__ T pack(uint32_t key, int pos) {
    return ((T)key << SHIFT) | (LOW - (T)pos);
  }
  static __device__ __forceinline__ uint32_t key(T b) { return (uint32_t)(b >> SHIFT); }
  static __device__ __forceinline__ int pos(T b) { return (int)(LOW - (b & LOW)); }
};

// Sort key of a token: the order key in the high word; in the low word
// (0x7ffff - id) in bits 13..31 (ids < 2^19), a marker bit 12 (so a real key
// exceeds the placeholders 0 .. 512 below) and in bit 0 the sign of a zero.
// Distinct ids give distinct keys and the low bits under the id field never
// decide an order.
__device__ __forceinline__ uint64_t sort_key(uint32_t key, int32_t id, uint32_t negzero) {
  return ((uint64_t)key << 32) | ((uint32_t)(0x7ffff - id) << 13) | 0x1000u | negzero;
}
__device__ __forceinline__ int32_t key_id(uint64_t k) {
  return 0x7ffff - (int32_t)((uint32_t)k >> 13);
}
// The logit (as float32) that a sort key stands for; a NaN comes back as the
// default quiet NaN.
template <int DT>
__device__ __forceinline__ float sort_key_value(uint64_t k) {
  const uint32_t key = (uint32_t)(k >> 32);
  if (key == 0u) return __builtin_nanf("");
  if (key == RankBits<DT>::ZERO) return (k & 1u) ? -0.0f : 0.0f;
  return key_value<DT>(key);
}
template <int DT>
__device__ __forceinline__ uint32_t negzero_bit(uint32_t b) {
  return b == RankBits<DT>::SIGN ? 1u : 0u;
}

constexpr int kRankCandCap = kRankMaxK * (rank_slice_len(kRankOptions - 1) / kThreads);

// 16-byte vectors per thread of the largest slice
constexpr int kRankMaxVecs = rank_slice_len(kRankOptions - 1) / kThreads / 4;

struct alignas(16) RankLds {
  union {
    uint64_t cand[kRankCandCap];                // slice candidates (0-padded)
    uint64_t lists[kRankMaxSlices][kRankMaxK];  // finalize: the slices' lists
  } u;
  uint4 stage[kRankMaxK * kRankMaxVecs];  // logits of the threads at or above tau
  int32_t stage_tid[kRankMaxK];
  uint64_t wt[kWaves][64];           // each wave's thread maxima
  uint64_t tops[kWaves][kRankMaxK];  // each wave's largest thread maxima (0-padded)
  uint64_t out[kRankMaxK];           // finalize: the row's top k
  float wm[kWaves];                  // per wave: largest finite thread maximum
  double wsum[kWaves];               //   sum exp(x - wm) over its finite logits
  uint32_t wflags[kWaves];
  uint32_t tok_bits;
  uint64_t tau;
  double lse;
  int32_t ncand;
  int32_t nstage;
  int32_t last;
};

// Count of the entries of a 0-padded LDS list larger than v, over `blocks`
// blocks of 16 entries (eight 16-byte reads in flight per block).
__device__ __forceinline__ int count_gt16(const uint64_t* a, int blocks, uint64_t v) {
  int c = 0;
  const ulonglong2* p = reinterpret_cast<const ulonglong2*>(a);
  for (int b = 0; b < blocks; ++b) {
    ulonglong2 w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = p[b * 8 + j];
#pragma unroll
    for (int j = 0; j < 8; ++j) c += (w[j].x > v ? 1 : 0) + (w[j].y > v ? 1 : 0);
  }
  return c;
}

// Rank of v among the union of up to LISTS lists of kRankMaxK entries each,
// sorted descending and 0-padded (list o counts only if o < nlists): the
// number of entries larger than v.  A branch-free lower bound per list, the
// lists' probes interleaved so each round's LDS reads are all in flight.
template <int LISTS>
__device__ __forceinline__ int rank_in_sorted(const uint64_t (*a)[kRankMaxK], int nlists,
                                              uint64_t v) {
  static_assert(kRankMaxK == 32, "five halving steps and a last probe");
  int pos[LISTS];
#pragma unroll
  for (int o = 0; o < LISTS; ++o) pos[o] = 0;
#pragma unroll
  for (int step = 16; step >= 1; step >>= 1) {
#pragma unroll
    for (int o = 0; o < LISTS; ++o) pos[o] += a[o][pos[o] + step - 1] > v ? step : 0;
  }
  int r = 0;
#pragma unroll
  for (int o = 0; o < LISTS; ++o)
    if (o < nlists) r += pos[o] + (a[o][pos[o]] > v ? 1 : 0);
  return r;
}

template <int DT, int OPT, bool VEC>
__global__ __launch_bounds__(kThreads) void k_rank(RankPlan P) {
  using B = RankBits<DT>;
  using BT = Best<DT>;
  constexpr int N = B::N;
  constexpr int ES = Vec<DT>::ESIZE;
  constexpr int SL = rank_slice_len(OPT);
  constexpr int Q = SL / (kThreads * N);  // 16-byte vectors per thread
  constexpr float kLog2e = 1.4426950408889634f;
  __shared__ RankLds L;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int G = P.slices;
  const int row = blockIdx.x / G, slice = blockIdx.x - row * G;
  const int32_t s0 = slice * SL;
  const int32_t ns = min(SL, P.vocab - s0);  // tokens in this slice
  const bool tail = ns < SL;
  const int k = P.k;
  const char* rowp =
      reinterpret_cast<const char*>(P.logits) + (size_t)row * (size_t)P.row_stride * ES;
  RankSlice* part = P.part + (size_t)row * kRankMaxSlices;

  // the chosen token's logit, read early by the slice that holds it
  const int32_t tok = P.tokens ? P.tokens[row] : -1;
  uint32_t tok_bits = 0u;
  if (tid == 0 && tok >= s0 && tok < s0 + ns)
    tok_bits = load_raw_bits<DT>(rowp, (int64_t)tok * P.col_stride);

  // ---- the slice's logits
  uint4 r[Q];
  if constexpr (VEC) {
    const int32_t full = ns / N;  // whole vectors inside the slice
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(rowp) + (size_t)s0 * ES, 0, full * 16, kBufferWord3);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs, tid * 16, q * kThreads * 16, 0);
      r[q] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    if (tail && (ns % N) != 0 && (full % kThreads) == tid) {
      // the slice's last partial vector, element by element
      const int qp = full / kThreads;
      const int32_t i0 = s0 + full * N;
      uint32_t b[N];
#pragma unroll
      for (int e = 0; e < N; ++e)
        b[e] = full * N + e < ns ? load_raw_bits<DT>(rowp, i0 + e) : 0u;
      uint4 v;
      if constexpr (N == 4) {
        v = make_uint4(b[0], b[1], b[2], b[3]);
      } else {
        v = make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16),
                       b[6] | (b[7] << 16));
      }
#pragma unroll
      for (int q = 0; q < Q; ++q)
        if (q == qp) r[q] = v;
    }
  } else {
    const int64_t cs = P.col_stride;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int32_t l0 = (q * kThreads + tid) * N;
      uint32_t b[N];
#pragma unroll
      for (int e = 0; e < N; ++e)
        b[e] = l0 + e < ns ? load_raw_bits<DT>(rowp, (int64_t)(s0 + l0 + e) * cs) : 0u;
      if constexpr (N == 4) {
        r[q] = make_uint4(b[0], b[1], b[2], b[3]);
      } else {
        r[q] = make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16),
                          b[6] | (b[7] << 16));
      }
    }
  }
  // while the logits stream in: the candidate list starts 0-padded
  if (k > 0) {
    ulonglong2* c2 = reinterpret_cast<ulonglong2*>(L.u.cand);
#pragma unroll
    for (int i = 0; i < kRankCandCap / 2 / kThreads; ++i) c2[tid + i * kThreads] = ulonglong2{0, 0};
  }
  if (tid == 0) {
    L.ncand = 0;
    L.nstage = 0;
  }

  // ---- 1. the thread's best key (and largest magnitude, for NaN / inf)
  typename BT::T best = 0;
  uint32_t magmax = 0;
  if (!tail) {
#pragma unroll
    for (int q = 0; q < Q; ++q) {
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const uint32_t b = elem_bits<DT>(r[q], e);
        magmax = max(magmax, b & B::MAG);
        const typename BT::T c = BT::pack(key_nn<DT>(b), q * N + e);
        best = c > best ? c : best;
      }
    }
  }
  // a tail slice, or a thread that holds a NaN: again, NaN-aware and masked
  const bool safe = tail || magmax > B::INF;
  if (safe) {
    best = 0;
    magmax = 0;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
#pragma unroll
      for (int e = 0; e < N; ++e) {
        if ((q * kThreads + tid) * N + e < ns) {
          const uint32_t b = elem_bits<DT>(r[q], e);
          magmax = max(magmax, b & B::MAG);
          const typename BT::T c = BT::pack(key_of<DT>(b), q * N + e);
          best = c > best ? c : best;
        }
      }
    }
  }
  const uint32_t bkey = BT::key(best);
  uint64_t tcomp;  // the thread's largest sort key (1 + tid when it holds no token)
  if (best != 0) {
    const int pos = BT::pos(best);
    const int32_t id = s0 + ((pos / N) * kThreads + tid) * N + pos % N;
    tcomp = sort_key(bkey, id, 0u);
  } else {
    tcomp = 1u + (uint32_t)tid;
  }
  const float m_t = (best != 0 && bkey != 0) ? key_value<DT>(bkey) : kNegInf;

  // log-sum-exp partial: sum exp(x - m_t) over the thread's finite logits
  float s_t = 0.f;
  if (P.lse && m_t > kNegInf && m_t < kPosInf) {
    if (!safe) {
#pragma unroll
      for (int q = 0; q < Q; ++q) {
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const float x = bits_value<DT>(elem_bits<DT>(r[q], e));
          s_t += __builtin_amdgcn_exp2f((x - m_t) * kLog2e);
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < Q; ++q) {
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const uint32_t b = elem_bits<DT>(r[q], e);
          const bool ok = (q * kThreads + tid) * N + e < ns && (b & B::MAG) <= B::INF;
          const float x = ok ? bits_value<DT>(b) : kNegInf;
          s_t += __builtin_amdgcn_exp2f((x - m_t) * kLog2e);
        }
      }
    }
  }

  // ---- per wave: flags, the log-sum-exp partial, the rank of each lane's maximum
  {
    const uint32_t f = (__ballot(magmax > B::INF) ? kRankNaN : 0u) |
                       (__ballot(magmax >= B::INF) ? kRankNonfinite : 0u) |
                       (__ballot(m_t == kPosInf) ? kRankPosInf : 0u);
    float wm = kNegInf;
    double wsum = 0.0;
    if (P.lse) {
      const float mf = m_t < kPosInf ? m_t : kNegInf;  // finite maxima only
      wm = wave_max(mf);
      const double term =
          mf > kNegInf ? (double)(s_t * __builtin_amdgcn_exp2f((mf - wm) * kLog2e)) : 0.0;
      wsum = wave_sum(term);
    }
    if (k > 0) {
      // (the wave's own LDS row: its writes are visible to its reads)
      L.wt[wv][lane] = tcomp;
      __builtin_amdgcn_wave_barrier();
      const int rank = count_gt16(L.wt[wv], 64 / 16, tcomp);
      if (rank < kRankMaxK) L.tops[wv][rank] = rank < k ? tcomp : 0ull;
    }
    if (lane == 0) {
      L.wm[wv] = wm;
      L.wsum[wv] = wsum;
      L.wflags[wv] = f;
    }
  }
  lds_barrier();

  // ---- 2. tau: the k-th largest thread maximum (the merge of the wave lists)
  if (k > 0 && tid < kWaves * k) {
    const int w = tid / k, rr = tid - w * k;
    const uint64_t v = L.tops[w][rr];
    if (rank_in_sorted<kWaves>(L.tops, kWaves, v) == k - 1) L.tau = v;
  }
  float M = kNegInf;
  double S = 0.0;
  uint32_t sflags = 0u;
#pragma unroll
  for (int o = 0; o < kWaves; ++o) {
    sflags |= L.wflags[o];
    M = fmaxf(M, L.wm[o]);
  }
  if (P.lse && M > kNegInf) {
#pragma unroll
    for (int o = 0; o < kWaves; ++o)
      if (L.wm[o] > kNegInf)
        S += L.wsum[o] * (double)__builtin_amdgcn_exp2f((L.wm[o] - M) * kLog2e);
  }
  if (sflags & kRankPosInf) M = kPosInf;

  if (k > 0) {
    lds_barrier();
    const uint64_t tau = L.tau;
    // ---- 3. candidates: the slice's keys >= tau.  They sit in the threads
    // at or above tau (k of them at most), which copy their logits to LDS;
    // then every thread scans a share of the copies.
    if (tcomp >= tau && best != 0) {
      const int slot = atomicAdd(&L.nstage, 1);
      L.stage_tid[slot] = tid;
#pragma unroll
      for (int q = 0; q < Q; ++q) L.stage[slot * Q + q] = r[q];
    }
    lds_barrier();
    const int nvec = L.nstage * Q;
    for (int v = tid; v < nvec; v += kThreads) {
      const int slot = v / Q, q = v - slot * Q;
      const int32_t l0 = (q * kThreads + L.stage_tid[slot]) * N;
      const uint4 x = L.stage[v];
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const uint32_t b = elem_bits<DT>(x, e);
        const uint64_t c = sort_key(key_of<DT>(b), s0 + l0 + e, negzero_bit<DT>(b));
        if (l0 + e < ns && c >= tau) {
          const int at = atomicAdd(&L.ncand, 1);
          if (at < kRankCandCap) L.u.cand[at] = c;
        }
      }
    }
    lds_barrier();
    // ---- 4. each candidate's rank: its count of larger candidates
    const int n = min(L.ncand, kRankCandCap);
    const int nblocks = (n + 15) >> 4;
    for (int j = tid; j < n; j += kThreads) {
      const uint64_t v = L.u.cand[j];
      const int rk = count_gt16(L.u.cand, nblocks, v);
      if (rk < k) st_coherent(&part[slice].top[rk], v);
    }
    for (int j = n + tid; j < k; j += kThreads) st_coherent(&part[slice].top[j], (uint64_t)0);
  }
  if (tid == 0) {
    st_coherent_f32(&part[slice].m, M);
    st_coherent_f64(&part[slice].s, S);
    st_coherent(&part[slice].flags, sflags);
    st_coherent(&part[slice].tok_bits, tok_bits);
  }
  if (!arrive_last(&P.arrive[row], (uint32_t)G, &L.last)) return;

  // ---- the row's last work-group: every slice record in one round of reads
  for (int i = tid; i < G * kRankMaxK; i += kThreads) {
    const int g = i / kRankMaxK, rr = i - g * kRankMaxK;
    L.u.lists[g][rr] = rr < k ? ld_coherent(&part[g].top[rr]) : 0ull;
  }
  // (wave 0 keeps the slices' log-sum-exp partials in registers, lane g for
  // slice g)
  float mg = kNegInf;
  double sg = 0.0;
  uint32_t fg = 0u;
  if (tid < G) {
    mg = __uint_as_float(ld_coherent(reinterpret_cast<const uint32_t*>(&part[tid].m)));
    sg = __builtin_bit_cast(double, ld_coherent(reinterpret_cast<const uint64_t*>(&part[tid].s)));
    fg = ld_coherent(&part[tid].flags);
    if (tok >= tid * SL && tok < (tid + 1) * SL) L.tok_bits = ld_coherent(&part[tid].tok_bits);
  }
  __syncthreads();
  for (int i = tid; i < G * k; i += kThreads) {
    const int g = i / k, rr = i - g * k;
    const uint64_t v = L.u.lists[g][rr];
    if (v != 0ull) {
      const int rk = G <= 8 ? rank_in_sorted<8>(L.u.lists, G, v)
                            : rank_in_sorted<kRankMaxSlices>(L.u.lists, G, v);
      if (rk < k) L.out[rk] = v;
    }
  }
  if (wv == 0) {
    const uint32_t rflags = (__ballot(fg & kRankNaN) ? kRankNaN : 0u) |
                            (__ballot(fg & kRankPosInf) ? kRankPosInf : 0u) |
                            (__ballot(fg & kRankNonfinite) ? kRankNonfinite : 0u);
    double lse = 0.0;
    if (P.lse) {
      const float mx = wave_max(mg);
      const double z = wave_sum(
          mg > kNegInf ? sg * (double)__builtin_amdgcn_exp2f((mg - mx) * kLog2e) : 0.0);
      if (rflags & kRankNaN)
        lse = __builtin_nan("");
      else if (rflags & kRankPosInf)
        lse = __builtin_huge_val();
      else if (mx == kNegInf)
        lse = -__builtin_huge_val();
      else
        lse = (double)mx + (double)__builtin_logf((float)z);
    }
    if (tid == 0) {
      L.lse = lse;
      uint32_t of = (rflags & kRankNonfinite) ? LSAMP_ROW_NONFINITE : 0u;
      if (P.tokens) {
        // a row whose log-sum-exp is not finite fails closed (NaN)
        float c = __builtin_nanf("");
        if (tok < 0 || tok >= P.vocab)
          of |= LSAMP_ROW_TOKEN_RANGE;
        else if (__builtin_isfinite(lse))
          c = (float)((double)bits_value<DT>(L.tok_bits) - lse);
        P.chosen[row] = c;
      }
      if (P.row_flags) P.row_flags[row] = of;
      st_coherent(&P.arrive[row], 0u);
    }
  }
  __syncthreads();
  if (tid < k) {
    // Log-probabilities of a row whose log-sum-exp is not finite (a NaN or
    // +inf logit, or every logit -inf) are undefined: the row fails closed
    // with ids -1 and NaN values, as the reference fails a non-finite row
    // (CBv2NonFiniteLogits.swift:8-34).  The exact top-2 ranks it as is.
    const uint64_t v = L.out[tid];
    const float x = sort_key_value<DT>(v);
    const bool closed = !P.raw_values && !__builtin_isfinite(L.lse);
    P.ids[(size_t)row * k + tid] = closed ? -1 : key_id(v);
    P.values[(size_t)row * k + tid] =
        P.raw_values ? x : closed ? __builtin_nanf("") : (float)((double)x - L.lse);
  }
}

template <int DT, int OPT>
void launch_rank_t(const RankPlan& P, hipStream_t st) {
  const dim3 grid((unsigned)(P.rows * P.slices));
  if (P.vec)
    hipLaunchKernelGGL((k_rank<DT, OPT, true>), grid, dim3(kThreads), 0, st, P);
  else
    hipLaunchKernelGGL((k_rank<DT, OPT, false>), grid, dim3(kThreads), 0, st, P);
}

template <int DT>
void launch_rank_dt(const RankPlan& P, hipStream_t st) {
  switch (P.option) {
    case 0: launch_rank_t<DT, 0>(P, st); break;
    case 1: launch_rank_t<DT, 1>(P, st); break;
    default: launch_rank_t<DT, 2>(P, st); break;
  }
}

}  // namespace

int launch_rank(const RankPlan& P, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (P.dtype) {
    case LSAMP_DTYPE_F32: launch_rank_dt<LSAMP_DTYPE_F32>(P, st); break;
    case LSAMP_DTYPE_BF16: launch_rank_dt<LSAMP_DTYPE_BF16>(P, st); break;
    default: launch_rank_dt<LSAMP_DTYPE_F16>(P, st); break;
  }
  return (int)hipGetLastError();
}

}  // namespace lsamp
