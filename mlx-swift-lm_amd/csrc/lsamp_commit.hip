// lsamp_commit.hip — the incremental penalty-state update after a draw, on
// the device (LogitsPipelineV2.commit, LogitsPipelineV2.swift:357-384).
//
// The reference keeps dense [B, vocab] float tensors (outputCounts,
// repWindowCounts) and a [B, W] ring, and scatter-adds into them once per
// step.  Here the same state is a fixed-capacity sparse table per row (one
// entry per token that carries a count, the repetition flag or a bias), the
// layout lsamp_sample reads, so a decode loop alternates lsamp_sample and
// lsamp_commit without a host round trip.
//
// One wave per row, in two rounds of memory reads: first the row's
// bookkeeping and its window row (the evicted token is a lane read), then the
// row's entries and window counts into registers, 64 lanes apart.  The lanes
// holding the sampled token, the evicted token and the run's last entry hand
// them to lane 0 (lane reads), which applies the update in the reference's
// order (output count, eviction, insertion into the window, ring position)
// and writes the changed entries back.  The row's tokens live in one
// contiguous run of entries; an entry that ends with no count, no flag and no
// bias leaves the run (the run's last entry moves into its slot).
#include <hip/hip_runtime.h>

#include "lsamp_device.h"
#include "lsamp_internal.h"

namespace lsamp {
namespace {

using namespace dev;

__device__ __forceinline__ bool neutral(const lsamp_penalty_entry& e) {
  return e.count == 0 && e.flags == 0u && e.bias == 0.0f;
}

// Entries a lane holds in registers during the scan (the row's run of
// entries, 64 lanes apart); longer runs are scanned again from memory.
constexpr int kCommitRegs = 16;

struct Found {
  int32_t idx;  // -1: absent
  lsamp_penalty_entry e;
  int32_t wc;
};

// The entry that lane `src` (wave-uniform) holds, read by every lane.
__device__ __forceinline__ Found take_from(int src, int32_t idx, const lsamp_penalty_entry& e,
                                           int32_t wc) {
  Found f;
  f.idx = read_lane(idx, src);
  f.e.token = read_lane(e.token, src);
  f.e.count = read_lane(e.count, src);
  f.e.flags = read_lane(e.flags, src);
  f.e.bias = read_lane(e.bias, src);
  f.wc = read_lane(wc, src);
  return f;
}

__global__ __launch_bounds__(64) void k_commit(lsamp_commit_args a) {
  const lsamp_penalty_table& T = a.table;
  const int r = blockIdx.x, lane = threadIdx.x;
  // first memory round trip: the row's bookkeeping and its whole window row, all independent
  const int32_t t = a.tokens[r];
  const uint32_t mode = T.mode[r];
  const int32_t len0 = T.row_len[r];
  const int32_t W = T.window_size[r];
  const int32_t pos = T.ring_pos[r];
  int32_t* win = T.window + (size_t)r * (size_t)T.window_capacity;
  const int32_t wlane = lane < T.window_capacity ? win[lane] : -1;
  lsamp_penalty_entry* ent = T.entries + (size_t)r * (size_t)T.capacity;
  int32_t* wcnt = T.window_count + (size_t)r * (size_t)T.capacity;
  const bool rep = (mode & LSAMP_STATE_REPETITION) != 0u;
  // a table whose bookkeeping is out of range is left alone (and reported)
  const bool sane = len0 >= 0 && len0 <= T.capacity &&
                    (!rep || (W >= 1 && W <= T.window_capacity && pos >= 0 && pos < W));
  if (!sane || t < 0 || t >= a.vocab ||
      (mode & (LSAMP_STATE_COUNTS | LSAMP_STATE_REPETITION)) == 0u) {
    if (lane == 0 && a.row_flags) a.row_flags[r] = sane ? 0u : LSAMP_ROW_OVERFLOW;
    return;
  }
  // the token this write evicts (slot pos of the ring)
  const int32_t ev = !rep ? -1 : pos < 64 ? read_lane(wlane, pos) : win[pos];

  // second memory round trip: the row's entries and window counts, in registers
  lsamp_penalty_entry e[kCommitRegs];
  int32_t wc[kCommitRegs];
#pragma unroll
  for (int i = 0; i < kCommitRegs; ++i) {
    const int j = lane + 64 * i;
    if (j < len0) {
      e[i] = ent[j];
      wc[i] = wcnt[j];
    } else {
      e[i] = lsamp_penalty_entry{-1, 0, 0u, 0.0f};
      wc[i] = 0;
    }
  }
  int32_t it = -1, iev = -1;
#pragma unroll
  for (int i = 0; i < kCommitRegs; ++i) {
    if (e[i].token == t) it = lane + 64 * i;
    if (ev >= 0 && e[i].token == ev) iev = lane + 64 * i;
  }
  for (int j = lane + 64 * kCommitRegs; j < len0; j += 64) {  // runs past the registers
    const int32_t tok = ent[j].token;
    if (tok == t) it = j;
    if (ev >= 0 && tok == ev) iev = j;
  }
  it = wave_max(it);
  iev = wave_max(iev);
  // the found entries and the run's last entry, from the lanes that hold them
  auto fetch = [&](int32_t idx) -> Found {
    Found f{-1, {0, 0, 0u, 0.0f}, 0};
    if (idx < 0) return f;
    if (idx < 64 * kCommitRegs) {
      const int src = idx & 63, slot = idx >> 6;
      lsamp_penalty_entry mine{0, 0, 0u, 0.0f};
      int32_t mwc = 0;
#pragma unroll
      for (int i = 0; i < kCommitRegs; ++i)
        if (i == slot) {
          mine = e[i];
          mwc = wc[i];
        }
      return take_from(src, idx, mine, mwc);
    }
    f.idx = idx;
    f.e = ent[idx];
    f.wc = wcnt[idx];
    return f;
  };
  Found ft = fetch(it), fe = fetch(iev), fl = fetch(len0 - 1);
  if (lane != 0) return;

  // lane 0 applies the update in the reference's order
  int32_t len = len0;
  bool overflow = false;
  auto insert = [&](Found& f) {
    if (len >= T.capacity) {
      overflow = true;
      return;
    }
    f.idx = len++;
    f.e = lsamp_penalty_entry{t, 0, 0u, 0.0f};
    f.wc = 0;
  };
  // outputCounts[row, token] += 1                               (:364-366)
  if (mode & LSAMP_STATE_COUNTS) {
    if (ft.idx < 0) insert(ft);
    if (ft.idx >= 0) ft.e.count += 1;
  }
  bool drop_ev = false;
  if (rep && ev != t) {
    // repWindowCounts[row, evicted] -= 1 for a real evicted id  (:371-375)
    if (fe.idx >= 0) {
      fe.wc = fe.wc > 1 ? fe.wc - 1 : 0;
      if (fe.wc == 0) fe.e.flags &= ~LSAMP_PEN_REPETITION;
      drop_ev = neutral(fe.e);
    }
    // repWindowCounts[row, token] += 1                        (:376)
    if (ft.idx < 0) insert(ft);
    if (ft.idx >= 0) {
      ft.wc += 1;
      ft.e.flags |= LSAMP_PEN_REPETITION;
    }
  }
  // write back; an evicted entry left with nothing leaves the run, the
  // run's last entry (possibly the one just inserted) taking its slot
  if (drop_ev) {
    const int32_t last = len - 1;
    Found mv = last == ft.idx ? ft : (last == fl.idx ? fl : fetch(-1));
    if (last != fe.idx) {
      if (last == ft.idx) ft.idx = fe.idx;
      ent[fe.idx] = mv.e;
      wcnt[fe.idx] = mv.wc;
    }
    --len;
  } else if (fe.idx >= 0) {
    ent[fe.idx] = fe.e;
    wcnt[fe.idx] = fe.wc;
  }
  if (ft.idx >= 0) {
    ent[ft.idx] = ft.e;
    wcnt[ft.idx] = ft.wc;
  }
  // repWindow[row, slot] = token; ringPos = (ringPos + 1) % W  (:377-380)
  if (rep) {
    win[pos] = t;
    T.ring_pos[r] = pos + 1 == W ? 0 : pos + 1;
  }
  T.row_len[r] = len;
  if (a.row_flags) a.row_flags[r] = overflow ? LSAMP_ROW_OVERFLOW : 0u;
}

// ---------------------------------------------------------------------------
// Penalty-aware verify windows (CBv2DefaultSampler.applyWindowPenalties,
// DefaultSamplerV2.swift:503-580).  The reference broadcasts each sequence's
// dense [vocab] output counts over the window and adds a cumulative one-hot
// of the drafts ([B, W, vocab] floats).  Here each window position gets a
// sparse run of entries: the sequence's entries with their counts raised by
// the drafts before the position, then the drafts that are not among them.
// Four waves per position (a row's entry loads all in flight at once); the
// drafts sit in LDS and every thread compares its entries with all of them.

constexpr int kMaxWindowDrafts = 64;
constexpr int kWindowThreads = 256;

__global__ __launch_bounds__(kWindowThreads) void k_window_entries(WindowEntriesPlan P) {
  __shared__ int32_t drafts[kMaxWindowDrafts];
  __shared__ unsigned long long found;  // drafts some entry matched
  const int row = blockIdx.x, lane = threadIdx.x;
  const int s = row / P.window, j = row - s * P.window;
  const int nd = P.column_offset + j;  // drafts before this position
  if (lane < nd) drafts[lane] = P.drafts[(size_t)s * (size_t)P.drafts_stride + lane];
  if (lane == 0) found = 0ull;
  __syncthreads();
  const int32_t e0 = P.row_ptr[s];
  const int32_t len = P.row_len ? P.row_len[s] : P.row_ptr[s + 1] - e0;
  lsamp_penalty_entry* out = P.out + (size_t)row * (size_t)P.cap;
  unsigned long long hit = 0ull;
#pragma unroll 4
  for (int k = lane; k < len; k += kWindowThreads) {
    const lsamp_penalty_entry e = P.entries[e0 + k];
    int32_t add = 0;
    for (int i = 0; i < nd; ++i) {
      if (drafts[i] == e.token) {
        ++add;
        hit |= 1ull << i;
      }
    }
    // counts only: the verify window applies frequency / presence alone
    if (k < P.cap) out[k] = lsamp_penalty_entry{e.token, e.count + add, 0u, 0.0f};
  }
  if (hit) atomicOr(&found, hit);
  __syncthreads();
  if (lane != 0) return;
  // drafts no entry holds: one new entry per distinct token, its count the
  // number of times it occurs among the drafts before the position
  int32_t n = len;
  bool over = len > P.cap;
  const unsigned long long f = found;
  for (int i = 0; i < nd; ++i) {
    const int32_t d = drafts[i];
    if (((f >> i) & 1ull) || d < 0 || d >= P.vocab) continue;
    bool seen = false;
    int32_t c = 0;
    for (int i2 = 0; i2 < nd; ++i2) {
      if (drafts[i2] != d) continue;
      if (i2 < i) seen = true;
      ++c;
    }
    if (seen) continue;
    if (n < P.cap)
      out[n] = lsamp_penalty_entry{d, c, 0u, 0.0f};
    else
      over = true;
    ++n;
  }
  P.out_ptr[row] = row * P.cap;
  P.out_len[row] = n < P.cap ? n : P.cap;
  if (over) atomicOr(P.status, kStatusPenaltyCapacity);
}

}  // namespace

int launch_window_entries(const WindowEntriesPlan& plan, void* stream) {
  hipLaunchKernelGGL(k_window_entries, dim3((unsigned)(plan.sequences * plan.window)),
                     dim3(kWindowThreads), 0, reinterpret_cast<hipStream_t>(stream), plan);
  return (int)hipGetLastError();
}

int launch_commit(const lsamp_commit_args& args, void* stream) {
  hipLaunchKernelGGL(k_commit, dim3((unsigned)args.table.rows), dim3(64), 0,
                     reinterpret_cast<hipStream_t>(stream), args);
  return (int)hipGetLastError();
}

}  // namespace lsamp
