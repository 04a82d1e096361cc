// lsamp_mask.hip — a decode step's grammar bitmask assembled on the device
// from cached pool rows (CBv2TokenConstraintSampler.mask,
// TokenConstraintSamplerV2.swift:131-182; deviceMask / open, :187-199).
//
// The reference keeps a [1, vocab] bool row per cached mask and builds a miss
// on the host (O(vocab) flags, then an upload).  Here a mask row is the packed
// LSB-first bitmask lsamp_sample consumes, a miss uploads only the allowed
// ids, and one work-group per output row either
//   * sets the allowed ids' bits in an LDS copy of the row and writes the row
//     to its pool slot and to the output (a build),
//   * copies its pool row to the output (a cached row), or
//   * writes all ones (an open row).
#include <hip/hip_runtime.h>

#include "lsamp_device.h"
#include "lsamp_internal.h"

namespace lsamp {
namespace {

constexpr int kMaskThreads = 256;

__global__ __launch_bounds__(kMaskThreads) void k_mask_assemble(MaskAssemblePlan P) {
  extern __shared__ uint32_t bits[];  // [words]: the row being built
  __shared__ int bad;
  const int r = blockIdx.x, tid = threadIdx.x;
  const int32_t src = P.row_source[r];
  const int W = P.words;
  uint32_t* out = P.out + (size_t)r * (size_t)W;
  if (src < 0 || !P.row_build[r]) {
    const uint32_t* prow = src < 0 ? nullptr : P.pool + (size_t)src * (size_t)W;
    if (P.vec) {
      uint4* o4 = reinterpret_cast<uint4*>(out);
      const uint4* p4 = reinterpret_cast<const uint4*>(prow);
      const uint4 ones = make_uint4(~0u, ~0u, ~0u, ~0u);
      for (int i = tid; i < W / 4; i += kMaskThreads) o4[i] = prow ? p4[i] : ones;
    } else {
      for (int i = tid; i < W; i += kMaskThreads) out[i] = prow ? prow[i] : ~0u;
    }
    if (tid == 0 && P.row_flags) P.row_flags[r] = 0u;
    return;
  }
  for (int i = tid; i < W; i += kMaskThreads) bits[i] = 0u;
  if (tid == 0) bad = 0;
  __syncthreads();
  const int32_t a = P.ids_ptr[r], b = P.ids_ptr[r + 1];
  bool mybad = false;
  for (int32_t k = a + tid; k < b; k += kMaskThreads) {
    const int32_t id = P.ids[k];
    if (id < 0 || id >= P.vocab) {
      mybad = true;
      continue;
    }
    atomicOr(&bits[id >> 5], 1u << (id & 31));
  }
  if (mybad) bad = 1;  // every writer stores the same value
  __syncthreads();
  // an out-of-range id leaves the whole row false (deviceMask, :189-191)
  const bool zero = bad != 0;
  uint32_t* prow = P.pool + (size_t)src * (size_t)W;
  for (int i = tid; i < W; i += kMaskThreads) {
    const uint32_t w = zero ? 0u : bits[i];
    prow[i] = w;
    out[i] = w;
  }
  if (tid == 0 && P.row_flags) P.row_flags[r] = zero ? LSAMP_MASK_ID_RANGE : 0u;
}

}  // namespace

int launch_mask_assemble(const MaskAssemblePlan& plan, void* stream) {
  hipLaunchKernelGGL(k_mask_assemble, dim3((unsigned)plan.rows), dim3(kMaskThreads),
                     (size_t)plan.words * sizeof(uint32_t), reinterpret_cast<hipStream_t>(stream),
                     plan);
  return (int)hipGetLastError();
}

}  // namespace lsamp
