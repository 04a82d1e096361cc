// lsamp_penalize.hip — the mlx-lm penalty processor as its own pass.
//
// PenaltyProcessor.process (Evaluate.swift:687-693) for a processor chain in
// which another processor sits between the penalties and the sampler
// (GenerationComponents.swift:112-141).  Two launches on the caller's stream:
// a copy of every logit into the output dtype (bandwidth-bound, 16 bytes a
// lane), then one thread per penalty entry writing the patched value of its
// token (patch_value, the same arithmetic as the sampling kernels: the
// repetition and presence penalties in the logits' dtype, the frequency
// penalty in float32).  Stream order puts every entry's write after the copy.
#include <hip/hip_runtime.h>

#include "lsamp_device.h"
#include "lsamp_internal.h"
#include "lsamp_row.h"

namespace lsamp {
namespace {

using namespace dev;
using namespace rowops;

constexpr int kPenThreads = 256;

template <int OT>
__device__ __forceinline__ void store_out(void* out, size_t i, float x) {
  if constexpr (OT == LSAMP_DTYPE_F32) {
    gmem(reinterpret_cast<float*>(out))[i] = x;
  } else if constexpr (OT == LSAMP_DTYPE_BF16) {
    gmem(reinterpret_cast<uint16_t*>(out))[i] = (uint16_t)(__float_as_uint(round_bf16(x)) >> 16);
  } else {
    gmem(reinterpret_cast<uint16_t*>(out))[i] =
        __builtin_bit_cast(uint16_t, (_Float16)x);
  }
}

// Every logit, converted (exactly: the output dtype is the input's or wider).
template <int DT, int OT>
__global__ __launch_bounds__(kPenThreads) void k_penalize_copy(PenalizePlan P) {
  const int row = (int)blockIdx.y;
  const char* rowp = reinterpret_cast<const char*>(P.logits) +
                     (size_t)row * (size_t)P.row_stride * (DT == LSAMP_DTYPE_F32 ? 4 : 2);
  const size_t obase = (size_t)row * (size_t)P.vocab;
  for (int64_t i = (int64_t)blockIdx.x * kPenThreads + threadIdx.x; i < P.vocab;
       i += (int64_t)gridDim.x * kPenThreads) {
    if constexpr (DT == OT) {
      if constexpr (DT == LSAMP_DTYPE_F32)
        gmem(reinterpret_cast<uint32_t*>(P.out))[obase + i] = load_raw_bits<DT>(rowp, i);
      else
        gmem(reinterpret_cast<uint16_t*>(P.out))[obase + i] = (uint16_t)load_raw_bits<DT>(rowp, i);
    } else {
      store_out<OT>(P.out, obase + (size_t)i, load_scalar<DT>(rowp, i));
    }
  }
}

// One work-group per row, one thread per entry: the token's patched value.
// (The penalties apply whatever the row's sampler, ArgMaxSampler rows too.)
template <int DT, int OT>
__global__ __launch_bounds__(kPenThreads) void k_penalize_entries(PenalizePlan P) {
  const int row = (int)blockIdx.x;
  const int32_t e0 = gmem(P.row_ptr)[row];
  const int32_t e1 = P.row_len ? e0 + gmem(P.row_len)[row] : gmem(P.row_ptr)[row + 1];
  const char* rowp = reinterpret_cast<const char*>(P.logits) +
                     (size_t)row * (size_t)P.row_stride * (DT == LSAMP_DTYPE_F32 ? 4 : 2);
  const lsamp_row_params prm = P.params[row];
  const RowCtx c = make_ctx(LSAMP_SEM_MLXLM, prm);
  for (int32_t e = e0 + (int32_t)threadIdx.x; e < e1; e += kPenThreads) {
    const lsamp_penalty_entry ent = gload16(P.entries + e);
    if (ent.token < 0 || ent.token >= P.vocab) continue;
    const float x = patch_value(c, prm, load_scalar<DT>(rowp, ent.token), ent, DT);
    store_out<OT>(P.out, (size_t)row * (size_t)P.vocab + (size_t)ent.token, x);
  }
}

template <int DT, int OT>
int launch_dt(const PenalizePlan& P, hipStream_t st) {
  const unsigned bx = (unsigned)((P.vocab + kPenThreads * 8 - 1) / (kPenThreads * 8));
  hipLaunchKernelGGL((k_penalize_copy<DT, OT>), dim3(bx, (unsigned)P.rows), dim3(kPenThreads), 0,
                     st, P);
  if (P.entries && P.row_ptr)
    hipLaunchKernelGGL((k_penalize_entries<DT, OT>), dim3((unsigned)P.rows), dim3(kPenThreads), 0,
                       st, P);
  return (int)hipGetLastError();
}

}  // namespace

int launch_penalize(const PenalizePlan& P, void* stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (P.dtype * 3 + P.out_dtype) {
    case LSAMP_DTYPE_F32 * 3 + LSAMP_DTYPE_F32: return launch_dt<LSAMP_DTYPE_F32, LSAMP_DTYPE_F32>(P, st);
    case LSAMP_DTYPE_BF16 * 3 + LSAMP_DTYPE_BF16: return launch_dt<LSAMP_DTYPE_BF16, LSAMP_DTYPE_BF16>(P, st);
    case LSAMP_DTYPE_BF16 * 3 + LSAMP_DTYPE_F32: return launch_dt<LSAMP_DTYPE_BF16, LSAMP_DTYPE_F32>(P, st);
    case LSAMP_DTYPE_F16 * 3 + LSAMP_DTYPE_F16: return launch_dt<LSAMP_DTYPE_F16, LSAMP_DTYPE_F16>(P, st);
    case LSAMP_DTYPE_F16 * 3 + LSAMP_DTYPE_F32: return launch_dt<LSAMP_DTYPE_F16, LSAMP_DTYPE_F32>(P, st);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace lsamp
