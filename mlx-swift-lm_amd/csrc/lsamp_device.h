// lsamp_device.h — device helpers shared by the kernels: dtype decoding,
// the deterministic exponential and fixed-point draw weights, Philox, and
// block-level reductions / scans for 512-thread work-groups.
#pragma once

#include <hip/hip_runtime.h>

#include <limits>

#include "lsamp_internal.h"

namespace lsamp {
namespace dev {

// Fourth word of a raw buffer descriptor on gfx9-family parts (32-bit data
// format; no swizzle, no stride).
constexpr int kBufferWord3 = 0x00020000;

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();

// ---------------------------------------------------------------- global memory
// Every pointer the kernels dereference addresses global memory, but the
// pointers reach them as generic ones (fields of a plan passed by value), and
// generic accesses compile to flat instructions.  A flat access may complete
// out of order with the vector loads, so after one the compiler waits for
// every load in flight (vmcnt(0)) before the next use of any of them, which
// serialises a slice's loads with the work on it.  Accesses through the
// global address space count only against the in-order vector counter, so a
// use of one load waits for that load alone.
template <typename T>
using gptr = __attribute__((address_space(1))) T*;

template <typename T>
__device__ __forceinline__ gptr<const T> gmem(const T* p) {
  return (gptr<const T>)p;
}
template <typename T>
__device__ __forceinline__ gptr<T> gmem(T* p) {
  return (gptr<T>)p;
}
// A 16-byte struct from global memory in one load (structs are read through
// a plain vector type: C++ cannot copy a class object out of another address
// space).
template <typename T>
__device__ __forceinline__ T gload16(const T* p) {
  static_assert(sizeof(T) == 16, "a 16-byte struct");
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(T, *gmem(reinterpret_cast<const u32x4*>(p)));
}

// ---------------------------------------------------------------- dtypes
template <int DT>
struct Vec {
  static constexpr int N = DT == LSAMP_DTYPE_F32 ? 4 : 8;  // elements per 16 bytes
  static constexpr int ESIZE = DT == LSAMP_DTYPE_F32 ? 4 : 2;
  static constexpr uint32_t NEG_INF_BITS =
      DT == LSAMP_DTYPE_F32 ? 0xff800000u : (DT == LSAMP_DTYPE_BF16 ? 0xff80u : 0xfc00u);
};

__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}

// Element k of a 16-byte vector.
template <int DT>
__device__ __forceinline__ float vec_elem(const uint4& r, int k) {
  if constexpr (DT == LSAMP_DTYPE_F32) {
    const uint32_t v = k == 0 ? r.x : (k == 1 ? r.y : (k == 2 ? r.z : r.w));
    return __uint_as_float(v);
  } else {
    const int q = k >> 1;
    const uint32_t word = q == 0 ? r.x : (q == 1 ? r.y : (q == 2 ? r.z : r.w));
    if constexpr (DT == LSAMP_DTYPE_BF16) {
      return (k & 1) ? __uint_as_float(word & 0xffff0000u) : __uint_as_float(word << 16);
    } else {
      return half_bits_to_f32((k & 1) ? (word >> 16) : (word & 0xffffu));
    }
  }
}

// Largest element of a 16-byte vector that holds no NaN (NaN-propagating
// maximum: no quieting moves are needed ahead of it).
template <int DT>
__device__ __forceinline__ float vec_max_nn(const uint4& r) {
  float m = vec_elem<DT>(r, 0);
#pragma unroll
  for (int k = 1; k < Vec<DT>::N; ++k) m = __builtin_elementwise_maximum(m, vec_elem<DT>(r, k));
  return m;
}

// Element e of a 16-byte vector, e not known at compile time.
template <int DT>
__device__ __forceinline__ float vec_elem_dyn(const uint4& r, int e) {
  if constexpr (DT == LSAMP_DTYPE_F32) {
    const uint32_t v = e == 0 ? r.x : (e == 1 ? r.y : (e == 2 ? r.z : r.w));
    return __uint_as_float(v);
  } else {
    const int q = e >> 1;
    const uint32_t word = q == 0 ? r.x : (q == 1 ? r.y : (q == 2 ? r.z : r.w));
    const uint32_t h = (e & 1) ? (word >> 16) : (word & 0xffffu);
    if constexpr (DT == LSAMP_DTYPE_BF16)
      return __uint_as_float(h << 16);
    else
      return half_bits_to_f32(h);
  }
}

// Replace the elements of a 16-byte vector whose bit is set in `excl` by -inf
// (branch-free: one mask per 32-bit word).
template <int DT>
__device__ __forceinline__ void exclude_elems(uint4& r, uint32_t excl) {
  uint32_t* w = reinterpret_cast<uint32_t*>(&r);
  if constexpr (DT == LSAMP_DTYPE_F32) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t m = 0u - ((excl >> k) & 1u);
      w[k] = (w[k] & ~m) | (Vec<DT>::NEG_INF_BITS & m);
    }
  } else {
    // bits 2k and 2k+1 of `excl` moved to bits 15 and 31 of a word, whose two
    // halves an arithmetic 16-bit shift turns into masks, then a bitfield
    // select from the -inf pair (three instructions a word, written out: the
    // compiler otherwise selects each half apart)
    const uint32_t pair = Vec<DT>::NEG_INF_BITS * 0x10001u;
    const uint32_t sp = excl | (excl << 15);  // bit j at j and at j + 15
    uint32_t m0, m1, m2, m3;
    // (the 16-bit shift counts are in a register: an inline constant would
    // reach only the low half)
    const uint32_t sh = 0x000f000fu;
    asm("v_lshlrev_b32 %0, 15, %8\n\t"
        "v_lshlrev_b32 %1, 13, %8\n\t"
        "v_lshlrev_b32 %2, 11, %8\n\t"
        "v_lshlrev_b32 %3, 9, %8\n\t"
        "v_pk_ashrrev_i16 %0, %10, %0\n\t"
        "v_pk_ashrrev_i16 %1, %10, %1\n\t"
        "v_pk_ashrrev_i16 %2, %10, %2\n\t"
        "v_pk_ashrrev_i16 %3, %10, %3\n\t"
        "v_bfi_b32 %4, %0, %9, %4\n\t"
        "v_bfi_b32 %5, %1, %9, %5\n\t"
        "v_bfi_b32 %6, %2, %9, %6\n\t"
        "v_bfi_b32 %7, %3, %9, %7"
        : "=&v"(m0), "=&v"(m1), "=&v"(m2), "=&v"(m3), "+v"(w[0]), "+v"(w[1]), "+v"(w[2]),
          "+v"(w[3])
        : "v"(sp), "s"(pair), "s"(sh));
  }
}

template <int DT>
__device__ __forceinline__ float load_scalar(const void* row, int64_t i) {
  if constexpr (DT == LSAMP_DTYPE_F32) {
    return gmem(reinterpret_cast<const float*>(row))[i];
  } else if constexpr (DT == LSAMP_DTYPE_BF16) {
    return __uint_as_float((uint32_t)gmem(reinterpret_cast<const uint16_t*>(row))[i] << 16);
  } else {
    return half_bits_to_f32(gmem(reinterpret_cast<const uint16_t*>(row))[i]);
  }
}

template <int DT>
__device__ __forceinline__ uint32_t load_raw_bits(const void* row, int64_t i) {
  if constexpr (DT == LSAMP_DTYPE_F32)
    return gmem(reinterpret_cast<const uint32_t*>(row))[i];
  else
    return gmem(reinterpret_cast<const uint16_t*>(row))[i];
}

// Load the 16-byte vector starting at token i0; lanes past `end` (or the whole
// vector when the row is not 16-byte aligned) are read one element at a time
// and out-of-range lanes are filled with -inf bits.
template <int DT>
__device__ __forceinline__ uint4 load_vec(const void* row, int64_t i0, int64_t end, bool aligned) {
  constexpr int N = Vec<DT>::N;
  if (aligned && i0 + N <= end) {
    return gload16(reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(row) +
                                                  i0 * Vec<DT>::ESIZE));
  }
  uint32_t b[N];
#pragma unroll
  for (int k = 0; k < N; ++k)
    b[k] = (i0 + k < end) ? load_raw_bits<DT>(row, i0 + k) : Vec<DT>::NEG_INF_BITS;
  uint4 r;
  if constexpr (DT == LSAMP_DTYPE_F32) {
    r.x = b[0];
    r.y = b[1];
    r.z = b[2];
    r.w = b[3];
  } else {
    r.x = b[0] | (b[1] << 16);
    r.y = b[2] | (b[3] << 16);
    r.z = b[4] | (b[5] << 16);
    r.w = b[6] | (b[7] << 16);
  }
  return r;
}

// Value an MLX array of `dt` holds after an op computed in float (RNE).
__device__ __forceinline__ float round_bf16(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return __uint_as_float(((b >> 16) | 0x40u) << 16);
  const uint32_t bias = 0x7fffu + ((b >> 16) & 1u);
  return __uint_as_float(((b + bias) >> 16) << 16);
}
__device__ __forceinline__ float round_dtype(float v, int dt) {
  if (dt == LSAMP_DTYPE_BF16) return round_bf16(v);
  if (dt == LSAMP_DTYPE_F16) return (float)(_Float16)v;
  return v;
}

// ------------------------------------------------------ deterministic math
// e^d for d <= 0 with a fixed sequence of IEEE fp32 operations: Cody & Waite
// (1980) range reduction with a two-part ln 2, Taylor polynomial of e^r to
// degree 7 in Horner form with fma, exact scaling by 2^n.  The host restates
// the same steps; results agree bit for bit.
__device__ __forceinline__ float dexp(float d) {
  if (!(d > -80.0f)) return 0.0f;
  if (d > 0.0f) d = 0.0f;
  const float n = __builtin_rintf(d * 1.44269504088896341f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, d);
  r = __builtin_fmaf(-n, 1.428606765330187e-06f, r);
  float p = 1.984126984e-04f;
  p = __builtin_fmaf(p, r, 1.388888889e-03f);
  p = __builtin_fmaf(p, r, 8.333333333e-03f);
  p = __builtin_fmaf(p, r, 4.166666667e-02f);
  p = __builtin_fmaf(p, r, 1.666666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n;
  return p * __uint_as_float((uint32_t)(ni + 127) << 23);
}

// Fixed-point draw weight 2^40 * dexp(fl(fl(y - y_max) * scale)).
__device__ __forceinline__ uint64_t weight(float y, float y_max, float scale) {
  if (!(y > kNegInf)) return 0ull;
  float d;
  if (y == y_max) {
    d = 0.0f;
  } else {
    const float diff = y - y_max;
    d = diff * scale;
  }
  const float e = dexp(d);
  return (uint64_t)(e * kWeightScale);
}

// The exponent argument used by `weight` (for entropy accumulation).
__device__ __forceinline__ float weight_arg(float y, float y_max, float scale) {
  if (y == y_max) return 0.0f;
  const float diff = y - y_max;
  return diff * scale;
}

__device__ __forceinline__ uint32_t uniform_u32(float u) {
  if (!(u > 0.0f)) return 0u;
  if (u >= 1.0f) return 0xffffffffu;
  return (uint32_t)(u * 4294967296.0f);
}

__device__ __forceinline__ uint64_t scaled_target(uint32_t U, uint64_t W) {
  const uint64_t hi = W >> 32, lo = W & 0xffffffffull;
  return (uint64_t)U * hi + (((uint64_t)U * lo) >> 32);
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11).
__device__ __forceinline__ uint32_t philox_x0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                              uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int round = 0; round < 10; ++round) {
    if (round > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0;
    const uint32_t n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return c0;
}

__device__ __forceinline__ float philox_uniform(uint64_t key, uint32_t purpose) {
  const uint32_t x0 = philox_x0(purpose, 0u, 0u, 0u, (uint32_t)key, (uint32_t)(key >> 32));
  return (float)(x0 >> 8) * 5.9604644775390625e-08f;
}

// Order-preserving key of a float (ascending).
__device__ __forceinline__ uint32_t ordered_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(b);
}

// Histogram bin of a transformed logit: floor(x * c32) with c32 = 32 / T,
// clamped so the integer conversion is defined for any finite x.
__device__ __forceinline__ float bin_pos(float x, float c32) {
  return __builtin_amdgcn_fmed3f(x * c32, -1.0e9f, 1.0e9f);
}
__device__ __forceinline__ int bin_of(float x, float c32) {
  return (int)__builtin_floorf(bin_pos(x, c32));
}

// ------------------------------------------------------------ wave ops
// Wave64 scans and reductions on DPP lane moves (row_shr within 16-lane rows,
// then row_bcast:15 / row_bcast:31 across rows).  All 64 lanes must be active.
// `id` is the operation's identity, read by lanes without a source.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp32(uint32_t v, uint32_t id) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, CTRL, ROWS, 0xf, false);
}
template <int CTRL, int ROWS, typename T>
__device__ __forceinline__ T dpp_move(T v, T id) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, dpp32<CTRL, ROWS>(__builtin_bit_cast(uint32_t, v),
                                                   __builtin_bit_cast(uint32_t, id)));
  } else {
    const uint64_t b = __builtin_bit_cast(uint64_t, v), i = __builtin_bit_cast(uint64_t, id);
    const uint32_t lo = dpp32<CTRL, ROWS>((uint32_t)b, (uint32_t)i);
    const uint32_t hi = dpp32<CTRL, ROWS>((uint32_t)(b >> 32), (uint32_t)(i >> 32));
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}
template <typename T>
__device__ __forceinline__ T read_lane(T v, int lane) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
  } else {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}
struct OpAdd {
  template <typename T> static __device__ __forceinline__ T f(T a, T b) { return a + b; }
};
struct OpMax {
  template <typename T> static __device__ __forceinline__ T f(T a, T b) { return a > b ? a : b; }
};
struct OpMin {
  template <typename T> static __device__ __forceinline__ T f(T a, T b) { return a < b ? a : b; }
};
// Inclusive scan in lane order.
template <typename Op, typename T>
__device__ __forceinline__ T wave_scan(T v, T id) {
  v = Op::f(v, dpp_move<0x111, 0xf>(v, id));
  v = Op::f(v, dpp_move<0x112, 0xf>(v, id));
  v = Op::f(v, dpp_move<0x114, 0xf>(v, id));
  v = Op::f(v, dpp_move<0x118, 0xf>(v, id));
  v = Op::f(v, dpp_move<0x142, 0xa>(v, id));
  v = Op::f(v, dpp_move<0x143, 0xc>(v, id));
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  return wave_scan<OpAdd>(v, T(0));
}
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  return read_lane(wave_scan<OpAdd>(v, T(0)), 63);
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
  const T id = std::numeric_limits<T>::has_infinity ? -std::numeric_limits<T>::infinity()
                                                    : std::numeric_limits<T>::lowest();
  return read_lane(wave_scan<OpMax>(v, id), 63);
}
template <typename T>
__device__ __forceinline__ T wave_min(T v) {
  const T id = std::numeric_limits<T>::has_infinity ? std::numeric_limits<T>::infinity()
                                                    : std::numeric_limits<T>::max();
  return read_lane(wave_scan<OpMin>(v, id), 63);
}

// ------------------------------------------------------------ block ops
// All helpers assume blockDim.x == kThreads and are called by every thread.
// scratch: at least kWaves elements of T.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* scratch) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r += scratch[i];
  __syncthreads();
  return r;
}
template <typename T>
__device__ __forceinline__ T block_max(T v, T* scratch) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r = scratch[i] > r ? scratch[i] : r;
  __syncthreads();
  return r;
}
template <typename T>
__device__ __forceinline__ T block_min(T v, T* scratch) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_min(v);
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) r = scratch[i] < r ? scratch[i] : r;
  __syncthreads();
  return r;
}

// Exclusive block scan in thread order; returns the exclusive prefix and
// writes the block total.  scratch: at least kWaves elements of T.
template <typename T>
__device__ __forceinline__ T block_excl_scan(T v, T* scratch, T* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const T incl = wave_incl_scan(v);
  __syncthreads();
  if (lane == 63) scratch[w] = incl;
  __syncthreads();
  T off = T(0), tot = T(0);
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    if (i < w) off += scratch[i];
    tot += scratch[i];
  }
  __syncthreads();
  *total = tot;
  return off + incl - v;
}

// Cross-work-group hand-off without fences.  An agent-scope fence on CDNA
// lowers to a walk of the whole L2 (write-back on release, invalidate on
// acquire), which serializes per XCD when hundreds of work-groups issue it.
// Instead, data another work-group will read is written with agent-scope
// relaxed atomic stores (write-through to the device coherence point), each
// wave waits for its stores to complete before the work-group barrier, the
// arrival counter is a returning agent-scope atomic, and the last arriver
// reads with agent-scope relaxed atomic loads (served from the coherence
// point, never from a stale L2 line).
template <typename T>
__device__ __forceinline__ T ld_coherent(const T* p) {
  return __hip_atomic_load(gmem(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_coherent(T* p, T v) {
  __hip_atomic_store(gmem(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent_f32(float* p, float v) {
  st_coherent(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
__device__ __forceinline__ void st_coherent_f64(double* p, double v) {
  st_coherent(reinterpret_cast<uint64_t*>(p), __builtin_bit_cast(uint64_t, v));
}
// Wait until every memory operation this wave issued has completed.
__device__ __forceinline__ void drain_memory() { __builtin_amdgcn_s_waitcnt(0); }

// r + (a > b) for 64-bit unsigned a and b: the borrow out of b - a, carried
// into r (three VALU operations through VCC; the compiler's 64-bit compare
// writes a lane mask that a select then has to read back).
__device__ __forceinline__ int add_gt_u64(int r, uint64_t a, uint64_t b) {
  uint32_t t;
  asm("v_sub_co_u32_e32 %1, vcc, %2, %3\n\t"
      "v_subb_co_u32_e32 %1, vcc, %4, %5, vcc\n\t"
      "v_addc_co_u32_e32 %0, vcc, 0, %0, vcc"
      : "+v"(r), "=&v"(t)
      : "v"((uint32_t)b), "v"((uint32_t)a), "v"((uint32_t)(b >> 32)), "v"((uint32_t)(a >> 32))
      : "vcc");
  return r;
}

// A read-only value at a uniform address, through the scalar data cache (a
// load from the constant address space): such loads count apart from the
// vector loads, which complete in order, so they do not wait behind a slice
// in flight.  The address passes through an SGPR pair as an integer, or the
// compiler would trace it back to a global pointer and load it as such.
// `p` must be the same in every lane.
template <typename T>
__device__ __forceinline__ T load_uniform(const T* p) {
  uint64_t a = (uint64_t)p;
  asm volatile("" : "+s"(a));
  return *(const __attribute__((address_space(4))) T*)a;
}

// Work-group barrier for LDS traffic only: each wave waits for its own LDS
// (and scalar) operations, not for its global loads, so loads in flight keep
// streaming across it.  It orders nothing in global memory.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt untouched
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Arrival on a per-row counter; true in every thread of the last arriver.
// `flag` is an LDS int.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t expected, int* flag) {
  drain_memory();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(gmem(counter), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = prev == expected - 1u;
  }
  __syncthreads();
  return *flag != 0;
}

}  // namespace dev
}  // namespace lsamp
