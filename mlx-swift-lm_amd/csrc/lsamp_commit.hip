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
// One wave per row: the lanes scan the row's entries for the sampled token
// and for the token the ring evicts (ids are unique within a row), then lane
// 0 applies the update in the reference's order: output count, eviction,
// insertion into the window, ring position.  The row's tokens live in one
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

__global__ __launch_bounds__(64) void k_commit(lsamp_commit_args a) {
  const lsamp_penalty_table& T = a.table;
  const int r = blockIdx.x, lane = threadIdx.x;
  const int32_t t = a.tokens[r];
  const uint32_t mode = T.mode[r];
  int32_t len = T.row_len[r];
  lsamp_penalty_entry* ent = T.entries + (size_t)r * (size_t)T.capacity;
  int32_t* wcnt = T.window_count + (size_t)r * (size_t)T.capacity;
  int32_t* win = T.window + (size_t)r * (size_t)T.window_capacity;
  const bool rep = (mode & LSAMP_STATE_REPETITION) != 0u;
  const int32_t W = T.window_size[r];
  const int32_t pos = rep ? T.ring_pos[r] : 0;
  // a table whose bookkeeping is out of range is left alone (and reported)
  const bool sane = len >= 0 && len <= T.capacity &&
                    (!rep || (W >= 1 && W <= T.window_capacity && pos >= 0 && pos < W));
  if (!sane || t < 0 || t >= a.vocab || (mode & (LSAMP_STATE_COUNTS | LSAMP_STATE_REPETITION)) == 0u) {
    if (lane == 0 && a.row_flags) a.row_flags[r] = sane ? 0u : LSAMP_ROW_OVERFLOW;
    return;
  }
  const int32_t ev = rep ? win[pos] : -1;  // the token this write evicts

  int32_t it = -1, iev = -1;
  for (int j = lane; j < len; j += 64) {
    const int32_t tok = ent[j].token;
    if (tok == t) it = j;
    if (tok == ev) iev = j;
  }
  it = wave_max(it);
  iev = wave_max(iev);
  if (lane != 0) return;

  bool overflow = false;
  auto insert = [&]() -> int32_t {
    if (len >= T.capacity) {
      overflow = true;
      return -1;
    }
    ent[len] = lsamp_penalty_entry{t, 0, 0u, 0.0f};
    wcnt[len] = 0;
    return len++;
  };
  // outputCounts[row, token] += 1                               (:364-366)
  if (mode & LSAMP_STATE_COUNTS) {
    if (it < 0) it = insert();
    if (it >= 0) ent[it].count += 1;
  }
  if (rep) {
    if (ev != t) {
      // repWindowCounts[row, evicted] -= 1 for a real evicted id  (:371-375)
      if (ev >= 0 && iev >= 0) {
        const int32_t c = wcnt[iev] - 1;
        wcnt[iev] = c;
        if (c <= 0) {
          wcnt[iev] = 0;
          ent[iev].flags &= ~LSAMP_PEN_REPETITION;
          if (neutral(ent[iev])) {
            const int32_t last = len - 1;
            if (iev != last) {
              ent[iev] = ent[last];
              wcnt[iev] = wcnt[last];
              if (it == last) it = iev;
            }
            --len;
          }
        }
      }
      // repWindowCounts[row, token] += 1                        (:376)
      if (it < 0) it = insert();
      if (it >= 0) {
        wcnt[it] += 1;
        ent[it].flags |= LSAMP_PEN_REPETITION;
      }
    }
    // repWindow[row, slot] = token; ringPos = (ringPos + 1) % W  (:377-380)
    win[pos] = t;
    T.ring_pos[r] = pos + 1 == W ? 0 : pos + 1;
  }
  T.row_len[r] = len;
  if (a.row_flags) a.row_flags[r] = overflow ? LSAMP_ROW_OVERFLOW : 0u;
}

}  // namespace

int launch_commit(const lsamp_commit_args& args, void* stream) {
  hipLaunchKernelGGL(k_commit, dim3((unsigned)args.table.rows), dim3(64), 0,
                     reinterpret_cast<hipStream_t>(stream), args);
  return (int)hipGetLastError();
}

}  // namespace lsamp
