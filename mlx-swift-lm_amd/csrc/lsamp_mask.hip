// lsamp_mask.hip — a decode step's grammar bitmask assembled on the device
// from cached pool rows (CBv2TokenConstraintSampler.mask,
// TokenConstraintSamplerV2.swift:131-182; deviceMask / open, :187-199).
//
// The reference keeps a [1, vocab] bool row per cached mask and builds a miss
// on the host (O(vocab) flags, then an upload).  Here a mask row is the packed
// LSB-first bitmask lsamp_sample consumes, a miss uploads only the allowed
// ids, and the work-groups of an output row either
//   * set the allowed ids' bits in an LDS copy of the row and write the row
//     to its pool slot and to the output (a build: one work-group),
//   * copy its pool row to the output, four work-groups a row (a cached row), or
//   * write all ones (an open row).
#include <hip/hip_runtime.h>

#include "lsamp_device.h"
#include "lsamp_internal.h"

namespace lsamp {
namespace {

constexpr int kMaskThreads = 1024;
constexpr int kMaskParts = 4;  // work-groups per row (cached and open rows split the copy)

__global__ __launch_bounds__(kMaskThreads) void k_mask_assemble(MaskAssemblePlan P) {
  extern __shared__ uint32_t bits[];  // [words]: the row being built
  __shared__ int bad;
  const int r = blockIdx.x / kMaskParts, part = blockIdx.x % kMaskParts;
  const int tid = threadIdx.x;
  const int32_t src = P.inline_rows ? P.src_inline[r] : P.row_source[r];
  const int W = P.words;
  uint32_t* out = P.out + (size_t)r * (size_t)W;
  if (src < 0 || P.inline_rows || !P.row_build[r]) {
    // this work-group's quarter of the row
    const uint32_t* prow = src < 0 ? nullptr : P.pool + (size_t)src * (size_t)W;
    if (P.vec) {
      const int n4 = W / 4, q0 = part * n4 / kMaskParts, q1 = (part + 1) * n4 / kMaskParts;
      uint4* o4 = reinterpret_cast<uint4*>(out);
      const uint4* p4 = reinterpret_cast<const uint4*>(prow);
      const uint4 ones = make_uint4(~0u, ~0u, ~0u, ~0u);
      if (prow)
        for (int i = q0 + tid; i < q1; i += kMaskThreads) o4[i] = p4[i];
      else
        for (int i = q0 + tid; i < q1; i += kMaskThreads) o4[i] = ones;
    } else {
      const int q0 = part * W / kMaskParts, q1 = (part + 1) * W / kMaskParts;
      if (prow)
        for (int i = q0 + tid; i < q1; i += kMaskThreads) out[i] = prow[i];
      else
        for (int i = q0 + tid; i < q1; i += kMaskThreads) out[i] = ~0u;
    }
    if (part == 0 && tid == 0 && P.row_flags) P.row_flags[r] = 0u;
    return;
  }
  if (part != 0) return;  // a build is one work-group's (the row sits in its LDS)
  for (int i = tid; i < W; i += kMaskThreads) bits[i] = 0u;
  if (tid == 0) bad = 0;
  __syncthreads();
  const int32_t a = P.ids_ptr[r], b = P.ids_ptr[r + 1];
  const int lane = tid & 63;
  bool mybad = false;
  // 64 ids per wave and pass; lanes whose ids share a word OR their bits
  // together first (a segmented suffix OR over runs of equal words), so a
  // sorted dense list costs a few LDS atomics per wave instead of 64
  constexpr int kAhead = 4;  // passes whose ids are loaded before the first is combined
  for (int32_t k00 = a + (tid & ~63); k00 < b; k00 += kAhead * kMaskThreads) {
    int32_t idv[kAhead];
#pragma unroll
    for (int u = 0; u < kAhead; ++u) {
      const int32_t k = k00 + u * kMaskThreads + lane;
      idv[u] = k < b ? P.ids[k] : 0;
    }
#pragma unroll
    for (int u = 0; u < kAhead; ++u) {
      const int32_t k0 = k00 + u * kMaskThreads;  // wave-uniform
      if (k0 >= b) continue;
      const int32_t k = k0 + lane;
      const bool in = k < b;
      const int32_t id = idv[u];
      const bool ok = in && id >= 0 && id < P.vocab;
      mybad |= in && !ok;
      const int32_t w = ok ? (id >> 5) : -1 - lane;  // a lane without an id is a run of its own
      uint32_t v = ok ? 1u << (id & 31) : 0u;
      // every lane shuffles (a lane outside the exec mask would read as 0)
      const int32_t wn = __shfl_down(w, 1, 64);
      bool end = lane == 63 || wn != w;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const uint32_t v2 = __shfl_down(v, d, 64);
        const int e2 = __shfl_down((int)end, d, 64);
        if (!end) {
          v |= v2;
          end = e2 != 0;
        }
      }
      const int32_t wp = __shfl_up(w, 1, 64);
      if (ok && (lane == 0 || wp != w)) atomicOr(&bits[w], v);
    }
  }
  if (mybad) bad = 1;  // every writer stores the same value
  __syncthreads();
  // an out-of-range id leaves the whole row false (deviceMask, :189-191)
  const bool zero = bad != 0;
  uint32_t* prow = P.pool + (size_t)src * (size_t)W;
  for (int i = tid; i < W; i += kMaskThreads) {
    const uint32_t x = zero ? 0u : bits[i];
    prow[i] = x;
    out[i] = x;
  }
  if (tid == 0 && P.row_flags) P.row_flags[r] = zero ? LSAMP_MASK_ID_RANGE : 0u;
}

// Suppressed ids (SuppressTokensProcessor, SuppressTokens.swift:67-81) folded
// into the step's bitmask.  A work-group owns kSupWords consecutive words of
// every row in its slice of rows: it clears the suppressed bits of its words
// in LDS (the whole id list is read by every work-group; lists are short),
// then writes caller word & LDS word for each row.
constexpr int kSupThreads = 256;
constexpr int kSupWords = 256;
constexpr int kSupRowsPerGroup = 16;
static_assert(kSupWords == kSupThreads, "one word per thread");

__global__ __launch_bounds__(kSupThreads) void k_suppress_mask(SuppressPlan P) {
  __shared__ uint32_t sup[kSupWords];
  const int tid = threadIdx.x;
  const int w0 = blockIdx.x * kSupWords;
  sup[tid] = ~0u;
  __syncthreads();
  for (int j = tid; j < P.n; j += kSupThreads) {
    const int32_t id = P.ids[j];
    if (id < 0 || id >= P.vocab) continue;
    const int w = (id >> 5) - w0;
    if (w >= 0 && w < kSupWords) atomicAnd(&sup[w], ~(1u << (id & 31)));
  }
  __syncthreads();
  const int w = w0 + tid;
  if (w >= P.words) return;
  // bits of this word that name tokens inside the vocabulary
  const int32_t nv = P.vocab - 32 * w;
  const uint32_t in_vocab = nv >= 32 ? ~0u : ((1u << nv) - 1u);
  // caller's bits: a word past mask_words, or a bit at or past mask_bits,
  // follows the tail policy
  int32_t nin = w < P.mask_words ? P.mask_bits - 32 * w : 0;
  nin = nin < 0 ? 0 : (nin > 32 ? 32 : nin);
  const uint32_t in_mask = nin >= 32 ? ~0u : ((1u << nin) - 1u);
  const uint32_t tail = P.mask_tail == LSAMP_MASK_TAIL_KEEP ? ~in_mask : 0u;
  const uint32_t keep = sup[tid] & in_vocab;
  const int r0 = blockIdx.y * kSupRowsPerGroup;
  const int r1 = r0 + kSupRowsPerGroup < P.rows ? r0 + kSupRowsPerGroup : P.rows;
  for (int r = r0; r < r1; ++r) {
    uint32_t allow = ~0u;
    if (P.bitmask) {
      const uint32_t word = w < P.mask_words ? P.bitmask[(size_t)r * P.mask_words + w] : 0u;
      allow = (word & in_mask) | tail;
    }
    P.out[(size_t)r * P.words + w] = allow & keep;
  }
}

}  // namespace

int launch_suppress_mask(const SuppressPlan& plan, void* stream) {
  const unsigned gx = (unsigned)((plan.words + kSupWords - 1) / kSupWords);
  const unsigned gy = (unsigned)((plan.rows + kSupRowsPerGroup - 1) / kSupRowsPerGroup);
  hipLaunchKernelGGL(k_suppress_mask, dim3(gx, gy), dim3(kSupThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), plan);
  return (int)hipGetLastError();
}

int launch_mask_assemble(const MaskAssemblePlan& plan, void* stream) {
  hipLaunchKernelGGL(k_mask_assemble, dim3((unsigned)(plan.rows * kMaskParts)), dim3(kMaskThreads),
                     (size_t)plan.words * sizeof(uint32_t), reinterpret_cast<hipStream_t>(stream),
                     plan);
  return (int)hipGetLastError();
}

}  // namespace lsamp
